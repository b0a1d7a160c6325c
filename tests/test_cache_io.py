"""On-disk compression cache (CPU only): the .npz schema of the reference's
writer, global codebook files, flat .idx export and the module walk."""
import numpy as np
import pytest
import torch
import torch.nn as nn

import cache_io
import codebook_builder as cbb
import huffman_codebook as hc


def _fixed(rng, M, K, ttype="mlp_ffn", local=True):
    w = cbb.bf16_round(rng.standard_normal((M, K)) * 0.02)
    d = cbb.compress_fixed(w)
    d.pop("_raw_indices")
    d["codebook_type"] = ttype
    if not local:
        d.pop("codebook")
    return w, d


def _huffman(rng, M, K):
    w = cbb.bf16_round(rng.standard_normal((M, K)) * 0.02)
    cb, idx = cbb.frequency_sorted_codebook(w)
    d = {"mode": "direct_codebook", "shape": (M, K), "bits": cbb.bits_for(len(cb)),
         "codebook": cb.astype(np.float32), "codebook_type": "attention",
         "encoding": "huffman"}
    d.update(hc.huffman_encode_indices(idx, shape=(M, K)))
    return w, d


def _same(a, b):
    assert set(a) == set(b), (sorted(a), sorted(b))
    for k in a:
        if isinstance(a[k], np.ndarray) or isinstance(b[k], np.ndarray):
            x, y = np.asarray(a[k]), np.asarray(b[k])
            assert x.dtype == y.dtype and np.array_equal(x.reshape(-1), y.reshape(-1)), k
        else:
            assert a[k] == b[k] and type(a[k]) == type(b[k]), (k, a[k], b[k])


def test_roundtrip_every_mode(tmp_path):
    rng = np.random.default_rng(0)
    _, fx = _fixed(rng, 8, 64)
    _, hf = _huffman(rng, 16, 128)
    cases = {
        "model.layers.0.mlp.up_proj.weight": fx,
        "model.layers.0.self_attn.q_proj.weight": hf,
        "model.norm.weight": {"mode": "exact", "shape": (64,),
                              "data": rng.integers(0, 1 << 16, 64).astype(np.uint16)},
        "lq.weight": {"mode": "linear_quant", "shape": (4, 4),
                      "indices": rng.integers(0, 256, 16).astype(np.uint8),
                      "scale": 0.25, "v_min": -1.5, "bits": 8},
        "cb.weight": {"mode": "codebook", "shape": (2, 3), "type": "attention",
                      "indices": np.arange(6, dtype=np.uint16)},
        "q8.weight": {"mode": "q8_packed_7bit", "shape": (3,), "packed": np.arange(5, dtype=np.uint8),
                      "original_len": 3, "scale": 0.5, "offset": 1.0,
                      "unique_q8": np.arange(4, dtype=np.int8),
                      "codebook_values": np.linspace(0, 1, 4).astype(np.float32)},
    }
    cache_io.save_cache(tmp_path, cases)
    got = cache_io.load_cache(tmp_path, threads=4)
    assert set(got) == set(cases)
    for name, d in cases.items():
        want = {k: v for k, v in d.items()}
        want["name"] = name
        want["shape"] = np.asarray(d["shape"], np.int64)
        if d["mode"] == "direct_codebook":
            want["bits"] = int(d["bits"])
        _same(got[name], want)
    # single-file API and the stored file name
    p = tmp_path / "tensors" / "model_layers_0_mlp_up_proj_weight.npz"
    name, d = cache_io.load_cached_tensor(p)
    assert name == "model.layers.0.mlp.up_proj.weight" and d["bits"] == fx["bits"]


def test_reads_reference_writer_layout(tmp_path):
    """Files laid out as src/compressor.py:199-243 writes them: str name and
    mode, tuple shape, length-1 arrays for metadata, no local codebook, and a
    Huffman file without this package's chunk index."""
    rng = np.random.default_rng(1)
    packed = rng.integers(0, 256, 13).astype(np.uint8)
    p1 = tmp_path / "a.npz"
    np.savez_compressed(p1, name="model.layers.1.self_attn.k_proj.weight",
                        mode="direct_codebook", shape=(4, 2),
                        codebook_type=np.array(["attention"]), bits=np.array([13]),
                        indices=packed)
    name, d = cache_io.load_cached_tensor(p1)
    assert name == "model.layers.1.self_attn.k_proj.weight"
    assert d["codebook_type"] == "attention" and d["bits"] == 13 and "codebook" not in d
    assert tuple(d["shape"]) == (4, 2) and np.array_equal(d["indices"], packed)

    _, hf = _huffman(rng, 8, 64)
    ref_keys = {k: hf[k] for k in ("huff_lengths", "huff_stream", "huff_n") + cache_io.HUFF_TABLE_KEYS}
    p2 = tmp_path / "b.npz"
    np.savez_compressed(p2, name="h.weight", mode="direct_codebook", shape=(8, 64),
                        codebook_type=np.array(["mlp_ffn"]), bits=np.array([hf["bits"]]),
                        codebook=hf["codebook"], encoding=np.array(["huffman"]), **ref_keys)
    _, d2 = cache_io.load_cached_tensor(p2)
    assert d2["encoding"] == "huffman" and "huff_chunk_offsets" not in d2
    for k, v in ref_keys.items():
        assert np.array_equal(d2[k], v), k
    # the reader never unpickles: an object array is refused
    p3 = tmp_path / "c.npz"
    np.savez(p3, name=np.array([{"x": 1}], dtype=object), mode="exact", shape=(1,),
             data=np.zeros(1, np.float32))
    with pytest.raises(ValueError):
        cache_io.load_cached_tensor(p3)


def test_global_codebooks(tmp_path):
    assert cache_io.codebook_type_of("mlp_ffn_codebook.npy") == "mlp_ffn"
    assert cache_io.codebook_type_of("attention_codebook_e8m7.npy") == "attention"
    assert cache_io.codebook_type_of("embedding.npy") == "embedding"
    cb = cbb.bf16_round(np.random.default_rng(2).standard_normal(300) * 0.02).astype(np.float32)
    cache_io.save_global_codebook(tmp_path, "attention", cb)
    np.save(tmp_path / "codebooks" / "mlp_ffn_codebook_e8m7.npy", cb[:10])
    g = cache_io.load_global_codebooks(tmp_path)
    assert set(g) == {"attention", "mlp_ffn"}
    assert g["attention"].dtype == torch.bfloat16
    assert np.array_equal(g["attention"].float().numpy(), cb)     # bf16 values: exact
    assert cache_io.load_global_codebooks(tmp_path / "missing") == {}


def test_export_flat_idx(tmp_path):
    rng = np.random.default_rng(3)
    _, a = _fixed(rng, 4, 32)
    _, b = _fixed(rng, 6, 16)
    _, h = _huffman(rng, 4, 64)
    model = tmp_path / "model"
    cache_io.save_cache(model / "codebook", {"x.a.weight": a, "x.b.weight": b, "x.h.weight": h})
    assert cache_io.export_flat_idx(model) == 2
    for name, d in (("x.a.weight", a), ("x.b.weight", b)):
        p = cache_io.idx_file_for(name, model, use_mmap=True)
        assert p.name == "x_a_weight.idx" or p.name == "x_b_weight.idx"
        assert np.array_equal(np.fromfile(p, np.uint8), d["indices"])
    assert cache_io.idx_file_for("x.a.weight", model, use_mmap=False) is None
    assert cache_io.export_flat_idx(model) == 0                   # existing files are kept
    with pytest.raises(FileNotFoundError):
        cache_io.export_flat_idx(tmp_path / "nothing")


class _Tiny(nn.Module):
    def __init__(self):
        super().__init__()
        self.model = nn.Module()
        self.model.embed_tokens = nn.Embedding(32, 16)
        self.model.proj = nn.Linear(16, 24)
        self.model.norm = nn.LayerNorm(16)
        self.lm_head = nn.Linear(16, 32, bias=False)


def test_module_walk_on_cpu(tmp_path):
    rng = np.random.default_rng(4)
    m = _Tiny()
    # only exact tensors: nothing is swapped
    cache = {"model.proj.weight": {"mode": "exact", "shape": (24, 16),
                                   "data": np.zeros((24, 16), np.float32)}}
    assert cache_io.replace_modules(m, cache, {}) == 0
    # a direct_codebook tensor needs the GPU: use_gpu=False raises, as the
    # compressed path has no CPU fallback here
    _, d = _fixed(rng, 24, 16)
    with pytest.raises(RuntimeError, match="GPU-only"):
        cache_io.replace_modules(m, {"model.proj.weight": d}, {}, use_gpu=False)
    assert isinstance(m.model.proj, nn.Linear)
