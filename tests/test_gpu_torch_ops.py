"""torch.ops.cbq (libcbq_torch.so over the C ABI) on the GPU vs the oracle:
eagerly, and captured in a torch.cuda.graph that is replayed several times
with new inputs copied in between (each replay checked against the oracle
for that replay's x).

Bar: rel-L2 <= 1e-5 for fp32 outputs, 2e-3 for bf16 outputs (bf16 rounding
of the output, bf16 MFMA at T >= 64); embedding rows bit-exact."""
import numpy as np
import pytest
import torch

import codebook_builder as cbb
import huffman_codebook as hc
from conftest import rel_l2

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops(cuda):
    import cbq_ops
    return cbq_ops.load()


def _fixed(M, K, seed):
    w = cbb.bf16_round(np.random.default_rng(seed).standard_normal((M, K)) * 0.02)
    return w, cbb.compress_fixed(w)


def _dev(a, dev, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    return t if dtype is None else t.to(dtype)


def _fixed_dev(d, dev):
    import bitpack
    return (_dev(bitpack.device_padded(np.asarray(d["indices"]).reshape(-1)), dev),
            _dev(np.asarray(d["codebook"], np.float32), dev))


@pytest.mark.parametrize("T", [1, 4, 16, 64])
def test_linear_f32(cuda, ops, oracle, T):
    M, K = 1024, 2048
    w, d = _fixed(M, K, 3)
    pk, cb = _fixed_dev(d, cuda)
    x = np.random.default_rng(T).standard_normal((T, K)).astype(np.float32)
    y = ops.linear(_dev(x, cuda), pk, cb, M, d["bits"])
    assert y.shape == (T, M) and y.dtype == torch.float32
    ref = oracle.fixed_gemv(x, d["indices"], d["codebook"], M, K, d["bits"])
    e = rel_l2(y.cpu().numpy(), ref)
    print(f"linear f32 T={T}: rel-L2 {e:.2e}", flush=True)
    assert e <= 1e-5


@pytest.mark.parametrize("T", [1, 64])
def test_linear_bf16(cuda, ops, oracle, T):
    M, K = 768, 1024
    w, d = _fixed(M, K, 4)
    pk, cb = _fixed_dev(d, cuda)
    x = cbb.bf16_round(np.random.default_rng(T + 10).standard_normal((T, K)))
    y = ops.linear(_dev(x, cuda, torch.bfloat16), pk, cb, M, d["bits"])
    assert y.dtype == torch.bfloat16
    ref = oracle.fixed_gemv(x, d["indices"], d["codebook"], M, K, d["bits"])
    e = rel_l2(y.float().cpu().numpy(), ref)
    print(f"linear bf16 T={T}: rel-L2 {e:.2e}", flush=True)
    assert e <= 2e-3


def test_embedding(cuda, ops, oracle):
    V, H = 500, 256
    w, d = _fixed(V, H, 5)
    pk, cb = _fixed_dev(d, cuda)
    ids = np.array([0, 499, 17, 17, 250], np.int32)
    y = ops.embedding(_dev(ids, cuda), pk, cb, V, d["bits"], H)
    assert np.array_equal(y.cpu().numpy(), w[ids])


def _huff_module(M, K, seed, layout):
    from gpu_huffman_functions import HuffmanCodebookLinear
    w = cbb.bf16_round(np.random.default_rng(seed).standard_normal((M, K)) * 0.02)
    cb, idx = cbb.frequency_sorted_codebook(w)
    enc = hc.huffman_encode_indices(idx, shape=(M, K))
    lin = HuffmanCodebookLinear(f"h{seed}", enc["huff_stream"], enc["huff_lengths"],
                                int(enc["huff_n"][0]), cb, (M, K), cbb.bits_for(len(cb)),
                                huff_row_bit_starts=enc["huff_row_bit_starts"], layout=layout)
    return w, cb, enc, lin


@pytest.mark.parametrize("layout", ["split", "stream"])
def test_huff_linear(cuda, ops, oracle, layout):
    M, K = 512, 2048
    w, cb, enc, lin = _huff_module(M, K, 6, layout)
    x = np.random.default_rng(7).standard_normal((1, K)).astype(np.float32)
    if layout == "split":
        y = ops.split_linear(_dev(x, cuda), *lin.split[0], M)
    else:
        y = ops.huff_linear(_dev(x, cuda), *lin.dev.op_args(), M)
    ref = oracle.huff_gemv(x, enc, cb, M, K)
    e = rel_l2(y.cpu().numpy(), ref)
    print(f"{layout} linear: rel-L2 {e:.2e}", flush=True)
    assert e <= 1e-5


@pytest.mark.parametrize("K", [2048, 4096, 6144])
def test_split_linear_tokens(cuda, ops, oracle, K):
    """split_linear with 2..20 tokens runs the fused few-token kernel (one
    pass per phase at K = 2048 / 4096, two at 6144, x's parts staged from 5
    tokens on); the module's batched forward is the same op."""
    M = 256
    w, cb, enc, lin = _huff_module(M, K, 20 + K // 1024, "split")
    rng = np.random.default_rng(K)
    for T in (2, 4, 5, 16, 20):
        x = rng.standard_normal((T, K)).astype(np.float32)
        y = ops.split_linear(_dev(x, cuda), *lin.split[0], M)
        e = rel_l2(y.cpu().numpy(), oracle.huff_gemv(x, enc, cb, M, K))
        assert e <= 1e-5, (K, T, e)
        assert torch.equal(lin(_dev(x, cuda)), y)


def test_split_linear_refuses_untaken_k(cuda, ops):
    """K = 9216: the few-token kernel's row-group tile does not fit, and the
    op says so instead of computing anything."""
    M, K = 64, 9216
    _, cb, enc, lin = _huff_module(M, K, 31, "split")
    with pytest.raises(RuntimeError, match="does not take K = 9216"):
        ops.split_linear(torch.zeros(3, K, device=cuda), *lin.split[0], M)


def test_huff_embedding(cuda, ops):
    from gpu_huffman_functions import HuffmanCodebookEmbedding
    V, H = 300, 128
    w = cbb.bf16_round(np.random.default_rng(8).standard_normal((V, H)) * 0.02)
    cb, idx = cbb.frequency_sorted_codebook(w)
    enc = hc.huffman_encode_indices(idx, shape=(V, H))
    emb = HuffmanCodebookEmbedding("he", enc["huff_stream"], enc["huff_lengths"],
                                   int(enc["huff_n"][0]), cb, (V, H), cbb.bits_for(len(cb)),
                                   huff_row_bit_starts=enc["huff_row_bit_starts"])
    ids = np.array([299, 0, 5], np.int32)
    y = ops.huff_embedding(_dev(ids, cuda), *emb.dev.op_args(), V, H)
    assert np.array_equal(y.cpu().numpy(), w[ids])


def test_graph_capture_replays(cuda, ops, oracle):
    """fixed T=1 and T=64 (workspace from the graph's pool), split Huffman at
    T = 1 and 8 (the few-token kernel, its workspace from the graph's pool),
    stream Huffman, embedding: one graph, 3 replays with fresh inputs, each against
    the oracle; eager launches run between the replays."""
    M, K = 1024, 2048
    _, d = _fixed(M, K, 9)
    pk, cb = _fixed_dev(d, cuda)
    _, hcb, henc, hs = _huff_module(512, K, 10, "split")
    _, tcb, tenc, ht = _huff_module(256, K, 11, "stream")
    xs1 = torch.zeros(1, K, device=cuda)
    xs64 = torch.zeros(64, K, device=cuda)
    xs8 = torch.zeros(8, K, device=cuda)
    ids = torch.zeros(4, dtype=torch.int32, device=cuda)
    emb_w, emb_d = _fixed(200, 128, 12)
    epk, ecb = _fixed_dev(emb_d, cuda)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):                  # warm-up outside the graph
        ops.linear(xs1, pk, cb, M, d["bits"])
        ops.linear(xs64, pk, cb, M, d["bits"])
        ops.split_linear(xs1, *hs.split[0], 512)
        ops.split_linear(xs8, *hs.split[0], 512)
        ops.huff_linear(xs1, *ht.dev.op_args(), 256)
        ops.embedding(ids, epk, ecb, 200, emb_d["bits"], 128)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        y1 = ops.linear(xs1, pk, cb, M, d["bits"])
        y64 = ops.linear(xs64, pk, cb, M, d["bits"])
        ysp = ops.split_linear(xs1, *hs.split[0], 512)
        ysp8 = ops.split_linear(xs8, *hs.split[0], 512)
        yst = ops.huff_linear(xs1, *ht.dev.op_args(), 256)
        ye = ops.embedding(ids, epk, ecb, 200, emb_d["bits"], 128)
    for r in range(3):
        rng = np.random.default_rng(100 + r)
        x1 = rng.standard_normal((1, K)).astype(np.float32)
        x64 = rng.standard_normal((64, K)).astype(np.float32)
        x8 = rng.standard_normal((8, K)).astype(np.float32)
        idv = rng.integers(0, 200, 4).astype(np.int32)
        xs1.copy_(torch.from_numpy(x1))
        xs64.copy_(torch.from_numpy(x64))
        xs8.copy_(torch.from_numpy(x8))
        ids.copy_(torch.from_numpy(idv))
        g.replay()
        eager = ops.linear(xs1, pk, cb, M, d["bits"])          # eager work between replays
        torch.cuda.synchronize()
        e = {"T1": rel_l2(y1.cpu().numpy(), oracle.fixed_gemv(x1, d["indices"], d["codebook"],
                                                               M, K, d["bits"])),
             "T64": rel_l2(y64.cpu().numpy(), oracle.fixed_gemv(x64, d["indices"],
                                                                 d["codebook"], M, K, d["bits"])),
             "split": rel_l2(ysp.cpu().numpy(), oracle.huff_gemv(x1, henc, hcb, 512, K)),
             "split T8": rel_l2(ysp8.cpu().numpy(), oracle.huff_gemv(x8, henc, hcb, 512, K)),
             "stream": rel_l2(yst.cpu().numpy(), oracle.huff_gemv(x1, tenc, tcb, 256, K))}
        print(f"replay {r}: " + ", ".join(f"{k} {v:.2e}" for k, v in e.items()), flush=True)
        assert max(e.values()) <= 1e-5, (r, e)
        assert torch.equal(eager, y1)
        assert np.array_equal(ye.cpu().numpy(), emb_w[idv])


def test_modules_route_through_ops(cuda, monkeypatch):
    """The modules' forward is the torch op: with the op namespace swapped
    for a recorder, a forward records one linear call."""
    import cbq_ops
    import gpu_accelerated_functions as gaf
    w, d = _fixed(256, 512, 13)
    lin = gaf.GPUAcceleratedLinear("r", d["indices"], torch.from_numpy(d["codebook"]),
                                   (256, 512), d["bits"])
    calls = []
    real = cbq_ops.load()

    class Rec:
        def __getattr__(self, name):
            def f(*a):
                calls.append(name)
                return getattr(real, name)(*a)
            return f
    monkeypatch.setattr(cbq_ops, "load", lambda: Rec())
    lin(torch.zeros(2, 512, device=cuda))
    assert calls == ["linear"]
