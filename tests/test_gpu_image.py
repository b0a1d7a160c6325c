"""The direct-to-device load path on the GPU: the encoder on the GPU writes
the same cache bytes as on the CPU; a device image loads through
cbq_file_upload into tensors whose GEMVs match the oracle on the cache's
reference-format data; a decoder loaded from an image generates the same
tokens as the decoder built in memory (fixed width and Huffman split)."""
import ctypes

import numpy as np
import pytest
import torch

import cache_io
import cbq_compress
import cbq_image
import cbq_native as nat
import synthetic
from conftest import rel_l2

pytestmark = pytest.mark.gpu

SHAPES = {"model.layers.0.self_attn.q_proj.weight": (256, 4096),
          "model.layers.0.mlp.down_proj.weight": (64, 2048),
          "model.layers.0.mlp.up_proj.weight": (96, 1000),
          "model.norm.weight": (4096,)}


@pytest.fixture(scope="module")
def ckpt(tmp_path_factory):
    from safetensors.torch import save_file
    d = tmp_path_factory.mktemp("model")
    ts = {n: synthetic.make_bf16(s, n, std=0.02 if len(s) == 2 else 0.5, device="cpu")
          for n, s in SHAPES.items()}
    save_file(ts, str(d / "model.safetensors"))
    return d, ts


@pytest.mark.parametrize("enc", [False, True])
def test_gpu_encoder_equals_cpu(cuda, ckpt, tmp_path, enc):
    d, _ = ckpt
    for dev in ("cpu", "cuda"):
        cbq_compress.compress_checkpoint(d, tmp_path / dev, entropy_code=enc, device=dev,
                                         write_image=False, log=lambda *a: None)
    a = cache_io.load_cache(tmp_path / "cpu")
    b = cache_io.load_cache(tmp_path / "cuda")
    assert set(a) == set(b) == set(SHAPES)
    for n in a:
        assert set(a[n]) == set(b[n]), n
        for k, v in a[n].items():
            if isinstance(v, np.ndarray):
                assert np.array_equal(v, b[n][k]), (n, k)
            else:
                assert v == b[n][k], (n, k)


@pytest.mark.parametrize("enc", [False, True])
def test_loaded_image_against_oracle(cuda, ckpt, tmp_path, oracle, enc):
    d, ts = ckpt
    s = cbq_compress.compress_checkpoint(d, tmp_path, entropy_code=enc, device="cuda",
                                         log=lambda *a: None)
    if enc:
        assert s["split"] == 2                               # K % 1024 == 0: q and down
    cache = cache_io.load_cache(tmp_path)
    tensors, h, stats = cbq_image.load_image(tmp_path / "device.cbq", cuda, threads=3,
                                             chunk_mb=1)
    assert stats["bytes"] == h["payload_bytes"]
    lib = nat.load()
    st = nat.stream_ptr(cuda)
    norm = tensors["model.norm.weight"]
    assert torch.equal(norm.cpu().view(torch.int16), ts["model.norm.weight"].view(torch.int16))
    for n, t in tensors.items():
        if n == "model.norm.weight":
            continue
        M, K = t.shape
        x = np.random.default_rng(M + K).standard_normal((1, K)).astype(np.float32)
        xd = torch.from_numpy(x).to(cuda)
        y = torch.empty(1, M, device=cuda)
        data = cache[n]
        cb = np.asarray(data["codebook"], np.float32)
        if isinstance(t, synthetic.FixedTensor):
            nat.check(lib.ck_linear_f32(xd.data_ptr(), t.packed.data_ptr(),
                                        t.codebook.data_ptr(), y.data_ptr(), 1, M, K,
                                        t.codebook.numel(), t.bits, st), "ck_linear_f32")
            ref = oracle.fixed_gemv(x, data["indices"], cb, M, K, int(data["bits"]),
                                    chunk_rows=None)
        elif isinstance(t, synthetic.SplitTensor):
            nat.check(lib.cbq_split_linear_f32(
                xd.data_ptr(), None, None, 0, 1e-6, 1,
                (ctypes.POINTER(nat.SplitMatrix) * 1)(ctypes.pointer(t.desc)),
                (ctypes.c_void_p * 1)(y.data_ptr()), (ctypes.c_int * 1)(M), K, st),
                "cbq_split_linear_f32")
            ref = oracle.huff_gemv(x, data, cb, M, K)
        else:                          # a stream (K % 1024 != 0): its decoded symbols
            from gpu_huffman_functions import SymbolDecoder
            dec = SymbolDecoder(t.words, t.chunk_off, t.sub_len, t.lengths, cuda).indices(M * K)
            want = oracle.huff_decode_indices(data, M, K).reshape(-1)
            assert np.array_equal(dec.cpu().numpy(), want), n
            continue
        torch.cuda.synchronize()
        assert rel_l2(y.cpu().numpy(), ref) <= 1e-5, (n, type(t).__name__)


def test_decoder_from_image_tokens(cuda, tmp_path):
    import decoder
    dec = synthetic.SyntheticDecoder("qwen3-8b", layers=2, log=lambda *a: None)
    c = dec.cfg
    cfg = decoder.DecoderConfig(layers=c["layers"], hidden=c["hidden"], inter=c["inter"],
                                n_q=c["n_q"], n_kv=c["n_kv"], head_dim=c["head_dim"],
                                vocab=c["vocab"])
    names = dec.all_linears() + [dec.embed]
    prompt = list(range(500, 520))
    for enc in ("fixed", "huffman"):
        tensors = dec.build_huffman(names) if enc == "huffman" else dec.build_fixed(names)
        want = decoder.from_synthetic(cfg, tensors, max_len=64).generate(prompt, 8)
        if enc == "huffman":       # linears in the split format, the embedding's stream
            tensors = {n: t if n == "model.embed_tokens" else (synthetic.to_split(t) or t)
                       for n, t in tensors.items()}
        path = tmp_path / f"{enc}.cbq"
        cbq_image.write_image(path, tensors)
        del tensors
        torch.cuda.empty_cache()
        loaded, h, stats = cbq_image.load_image(path, cuda)
        kinds = {e["kind"] for e in h["tensors"].values()}
        assert kinds == ({"fixed"} if enc == "fixed" else {"split", "stream"}), kinds
        m = decoder.from_synthetic(cfg, loaded, max_len=64)
        assert m.generate(prompt, 8) == want, enc
        assert m.generate_graph(prompt, 8) == want, enc
        del m, loaded
        torch.cuda.empty_cache()


class _Tiny(torch.nn.Module):
    """HF-style parameter names: embed_tokens, layers.0.{self_attn,mlp}, norm,
    lm_head tied to the embedding (no tensor of its own)."""

    def __init__(self, vocab=300, hidden=1024):
        super().__init__()
        nn = torch.nn
        self.model = nn.Module()
        self.model.embed_tokens = nn.Embedding(vocab, hidden)
        layer = nn.Module()
        layer.self_attn = nn.Module()
        layer.self_attn.q_proj = nn.Linear(hidden, 512, bias=False)
        layer.self_attn.k_proj = nn.Linear(hidden, 96, bias=True)
        layer.mlp = nn.Module()
        layer.mlp.down_proj = nn.Linear(2048, hidden, bias=False)
        self.model.layers = nn.ModuleList([layer])
        self.model.norm = nn.Module()
        self.model.norm.weight = nn.Parameter(torch.ones(hidden))
        self.lm_head = nn.Linear(hidden, vocab, bias=False)

    def forward(self, ids):
        h = self.model.embed_tokens(ids).float() * self.model.norm.weight.float()
        att = self.model.layers[0].self_attn
        q = att.q_proj(h)
        k = att.k_proj(h)
        d = self.model.layers[0].mlp.down_proj(torch.cat([q, q, q, q], -1))
        return q, k, d, self.lm_head(h)


@pytest.mark.parametrize("enc", [False, True])
def test_replace_modules_from_image(cuda, tmp_path, enc):
    """A model's Linear / Embedding modules swapped for compressed modules
    bound to a loaded device image give the dense bf16 model's outputs
    (fp32 arithmetic both sides, rel-L2 <= 1e-5); the tied lm_head uses the
    embedding's tensor; dense tensors (the norm) are loaded too."""
    from safetensors.torch import save_file
    torch.manual_seed(0)
    dense = _Tiny()
    sd = {k: (v.detach() * (0.02 if "norm" not in k else 1.0) + (0.5 if "norm" in k else 0.0))
          .bfloat16().contiguous() for k, v in dense.state_dict().items() if "lm_head" not in k}
    d = tmp_path / "ckpt"
    d.mkdir()
    save_file(sd, str(d / "model.safetensors"))
    cbq_compress.compress_checkpoint(d, tmp_path / "out", entropy_code=enc, device="cuda",
                                     write_npz=False, log=lambda *a: None)
    dense.load_state_dict({k: v.float() for k, v in sd.items()}, strict=False)
    dense.lm_head.weight = dense.model.embed_tokens.weight
    dense = dense.to(cuda)
    comp = _Tiny()
    n, stats = cache_io.replace_modules_from_image(comp, tmp_path / "out" / "device.cbq", cuda)
    assert n == 5 and stats["bytes"] > 0                  # embed, q, k, down, tied lm_head
    comp.model.layers[0].self_attn.k_proj.bias.data = \
        dense.model.layers[0].self_attn.k_proj.bias.data.clone()
    comp = comp.to(cuda)
    assert comp.model.norm.weight.dtype == torch.bfloat16
    ids = torch.tensor([[3, 17, 299, 0, 150]], device=cuda)
    with torch.no_grad():
        want = dense(ids)
        got = comp(ids)
    for a, b in zip(got, want):
        assert rel_l2(a.float().cpu().numpy(), b.float().cpu().numpy()) <= 1e-5


def test_load_rejects_inconsistent_arrays(cuda, ckpt, tmp_path):
    """Array values the kernels trust (split row offsets, stream chunk
    offsets) are checked after the upload: a tampered image raises before
    any descriptor reaches a kernel; so does a truncated file."""
    import struct
    d, _ = ckpt
    cbq_compress.compress_checkpoint(d, tmp_path, entropy_code=True, device="cuda",
                                     write_npz=False, log=lambda *a: None)
    path = tmp_path / "device.cbq"
    h = cbq_image.read_header(path)
    raw = bytearray(path.read_bytes())
    e = h["tensors"]["model.layers.0.self_attn.q_proj.weight"]
    assert e["kind"] == "split"
    off = h["data_offset"] + e["sections"]["row_off"][0]
    good = bytes(raw)
    raw[off + 4 * 3:off + 4 * 4] = struct.pack("<i", 1 << 20)      # a chunk of 2^20 rows
    bad = tmp_path / "bad.cbq"
    bad.write_bytes(bytes(raw))
    with pytest.raises(ValueError):
        cbq_image.load_image(bad, cuda)
    e = h["tensors"]["model.layers.0.mlp.up_proj.weight"]           # K = 1000: a stream
    assert e["kind"] == "stream"
    raw = bytearray(good)
    off = h["data_offset"] + e["sections"]["chunk_off"][0]
    raw[off + 8:off + 16] = struct.pack("<q", 1 << 40)              # a chunk past the stream
    bad.write_bytes(bytes(raw))
    with pytest.raises(ValueError):
        cbq_image.load_image(bad, cuda)
    bad.write_bytes(good[:-4096])
    with pytest.raises(ValueError):
        cbq_image.load_image(bad, cuda)
    tensors, _, _ = cbq_image.load_image(path, cuda)                 # the untouched image loads
    assert len(tensors) == len(h["tensors"])
