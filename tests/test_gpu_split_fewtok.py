"""Few tokens straight from the split Huffman format
(cbq_split_linear_fewtok_f32, csrc/cbq_split.hip): every weight decoded once
per 16 tokens into LDS and multiplied on the bf16 matrix cores, against the
oracle's fixed-width GEMV over the same indices (the split weights are the
codebook values; src/compressed_matmul.c:208-239 / :416-450 restated).

Only the fp32 summation order differs from the oracle (x is split exactly
into three bf16 parts): rel-L2 <= 1e-5.  Shapes: K % 4096 == 0 with one and
three chunks per row, K = 2048 and 1024 (two and four rows per chunk), a
last tile with fewer rows than waves, more tiles than CUs (the persistent
loop), T from 1 to 32 (two launches), rows past T untouched; K = 6144 is
refused by the kernel and served by the transient stream instead.
"""
import ctypes

import numpy as np
import pytest
import torch

import cbq_native as nat
import codebook_builder as cbb
from conftest import rel_l2
from gpu_huffman_functions import build_split, split_prefill

pytestmark = pytest.mark.gpu
TOL = 1e-5


def _case(cuda, M, K, seed):
    rng = np.random.default_rng(seed)
    w = cbb.bf16_round(rng.standard_normal((M, K)) * 0.02)
    cb, idx = cbb.frequency_sorted_codebook(w)
    sp = build_split(torch.from_numpy(idx.astype(np.int32)).to(cuda), cb, cuda)
    assert sp is not None
    return rng, cb, idx, sp


def _ref(oracle, x, cb, idx, M, K):
    bits = cbb.bits_for(len(cb))
    packed = oracle.pack_lsb(idx.reshape(-1).astype(np.int64), bits)
    return oracle.fixed_gemv(x, packed, cb, M, K, bits, chunk_rows=None)


def _call(sps, xd, outs, Ms, K, cuda, ws=True):
    """ws: stage x's bf16 parts in a workspace (the path the modules take);
    False: every lane splits its x in the GEMM."""
    n = len(sps)
    mats = (ctypes.POINTER(nat.SplitMatrix) * n)(*[ctypes.pointer(sp[1]) for sp in sps])
    optr = (ctypes.c_void_p * n)(*[o.data_ptr() for o in outs])
    mptr = (ctypes.c_int * n)(*Ms)
    lib = nat.load()
    wsb = int(lib.cbq_split_fewtok_ws_bytes(K)) if ws else 0
    _call.keep = torch.empty(max(wsb, 16), dtype=torch.uint8, device=cuda)
    return lib.cbq_split_linear_fewtok_f32(xd.data_ptr(), xd.shape[0], n, mats, optr, mptr, K,
                                           _call.keep.data_ptr() if ws else None, wsb,
                                           nat.stream_ptr(cuda))


def _fewtok(cuda, sp, x, M, K, extra_rows=0):
    T = x.shape[0]
    xd = torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(cuda)
    out = torch.full((T + extra_rows, M), float("nan"), device=cuda)
    rc = _call([sp], xd, [out], [M], K, cuda)
    torch.cuda.synchronize()
    return rc, out.cpu().numpy()


@pytest.mark.parametrize("M,K", [(300, 4096), (70, 12288), (640, 2048), (96, 1024),
                                 (5000, 4096), (256, 6144), (2048, 6144), (96, 3072),
                                 (120, 5120), (64, 7168)])
def test_against_oracle(cuda, oracle, M, K):
    rng, cb, idx, sp = _case(cuda, M, K, M + K)
    for T in (1, 2, 5, 16, 17, 32):
        x = rng.standard_normal((T, K)).astype(np.float32)
        rc, y = _fewtok(cuda, sp, x, M, K, extra_rows=1)
        assert rc == 0, (M, K, T)
        assert np.isnan(y[T:]).all(), "rows past T written"
        assert rel_l2(y[:T], _ref(oracle, x, cb, idx, M, K)) <= TOL, (M, K, T)


def test_refused_shape_uses_transient_stream(cuda, oracle):
    """K = 9216 (a chunk group's 4 rows need 9 chunks: more than the 16-wave
    tile's passes take): the kernel refuses it, and split_prefill takes the
    transient fixed-width stream with the same result."""
    from gpu_huffman_functions import split_fewtok_eligible
    M, K = 64, 9216
    assert not split_fewtok_eligible(K) and split_fewtok_eligible(6144)
    rng, cb, idx, sp = _case(cuda, M, K, 9)
    x = rng.standard_normal((4, K)).astype(np.float32)
    rc, _ = _fewtok(cuda, sp, x, M, K)
    assert rc == nat.CK_ERR_ARG
    from gpu_huffman_functions import split_inverse
    cbt = torch.from_numpy(cb).to(cuda)
    inv = split_inverse(cb, cuda)
    y = split_prefill(sp, inv, torch.from_numpy(x).to(cuda), M, K, cbt)
    assert rel_l2(y.cpu().numpy(), _ref(oracle, x, cb, idx, M, K)) <= TOL


def test_module_batched_tokens(cuda, oracle):
    """HuffmanCodebookLinear with 4 tokens runs the fused kernel (split
    format, K = 4096) and matches the oracle and its own one-token rows."""
    import huffman_codebook as hc
    from test_gpu_huffman import _lin
    M, K = 512, 4096
    rng = np.random.default_rng(21)
    w = cbb.bf16_round(rng.standard_normal((M, K)) * 0.02)
    cb, idx = cbb.frequency_sorted_codebook(w)
    enc = hc.huffman_encode_indices(idx, shape=(M, K))
    lin = _lin(enc, cb, M, K)
    assert lin.split is not None
    x = torch.from_numpy(rng.standard_normal((4, K)).astype(np.float32)).to(cuda)
    y = lin(x)
    ref = oracle.huff_gemv(x.cpu().numpy(), enc, cb, M, K, chunk_rows=None)
    assert rel_l2(y.cpu().numpy(), ref) <= TOL
    for t in range(4):
        assert rel_l2(lin(x[t:t + 1]).cpu().numpy(), ref[t:t + 1]) <= TOL


def test_graph_replays_match_eager(cuda):
    M, K = 1024, 4096
    rng, cb, idx, sp = _case(cuda, M, K, 5)
    x = torch.from_numpy(rng.standard_normal((8, K)).astype(np.float32)).to(cuda)
    out = torch.empty(8, M, device=cuda)

    def run():
        nat.check(_call([sp], x, [out], [M], K, cuda), "cbq_split_linear_fewtok_f32")
    run()
    torch.cuda.synchronize()
    eager = out.clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        run()
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        run()
    for _ in range(3):
        out.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)


@pytest.mark.parametrize("Ms,K", [((2048, 1024, 1024), 2048), ((6144, 6144), 2048),
                                  ((4096, 1024, 1024, 512), 4096)])
def test_grouped_matrices(cuda, oracle, Ms, K):
    """Up to four matrices sharing x in one launch (the decoder's q/k/v and
    gate/up), blocks shared out by tiles: each equals its own launch bit for
    bit and the oracle within fp32 tolerance."""
    rng = np.random.default_rng(sum(Ms) + K)
    cases = [_case(cuda, M, K, 100 + i) for i, M in enumerate(Ms)]
    x = rng.standard_normal((6, K)).astype(np.float32)
    xd = torch.from_numpy(x).to(cuda)
    outs = [torch.full((6, M), float("nan"), device=cuda) for M in Ms]
    assert _call([c[3] for c in cases], xd, outs, list(Ms), K, cuda) == 0
    torch.cuda.synchronize()
    for (r, cb, idx, sp), M, o in zip(cases, Ms, outs):
        single = torch.full((6, M), float("nan"), device=cuda)
        assert _call([sp], xd, [single], [M], K, cuda) == 0
        torch.cuda.synchronize()
        assert torch.equal(o, single)
        assert rel_l2(o.cpu().numpy(), _ref(oracle, x, cb, idx, M, K)) <= TOL


def test_two_pass_shapes_need_the_workspace(cuda):
    M, K = 256, 6144
    rng, cb, idx, sp = _case(cuda, M, K, 31)
    xd = torch.from_numpy(rng.standard_normal((4, K)).astype(np.float32)).to(cuda)
    out = torch.empty(4, M, device=cuda)
    assert _call([sp], xd, [out], [M], K, cuda, ws=False) == nat.CK_ERR_ARG


@pytest.mark.parametrize("M,K", [(300, 4096), (640, 2048)])
def test_workspace_and_in_kernel_split_agree(cuda, M, K):
    """x's parts staged in the workspace or split by every lane in the GEMM:
    the same bf16 operands, so the outputs are equal bit for bit."""
    rng, cb, idx, sp = _case(cuda, M, K, 77)
    for T in (3, 16, 20):
        xd = torch.from_numpy(rng.standard_normal((T, K)).astype(np.float32)).to(cuda)
        a = torch.full((T, M), float("nan"), device=cuda)
        b = torch.full((T, M), float("nan"), device=cuda)
        assert _call([sp], xd, [a], [M], K, cuda, ws=True) == 0
        assert _call([sp], xd, [b], [M], K, cuda, ws=False) == 0
        torch.cuda.synchronize()
        assert torch.equal(a, b), T
