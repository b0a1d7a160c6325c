"""Few-token fixed-width GEMM (2..16 tokens) on the bf16 matrix cores
(fixed_fewtok_kernel, csrc/cbq_tiny.hip) through ck_linear_f32 /
ck_linear_bf16, against the oracle (src/compressed_matmul.c:416-450 restated).

The kernel splits fp32 x exactly into three bf16 parts, and a codebook that
is not bf16 into three parts as well, so its products are exact and only the
fp32 summation order differs from the oracle's: rel-L2 <= 1e-5.  Cases:
every width it takes, bf16 and non-bf16 codebooks, indices past C, each of
the four row-tiles-per-block plans (chosen from the CU count), ragged M,
K with fewer 128-column steps than waves, a wide dynamic range of x, and
the shapes it refuses (K % 128 != 0, x off 16-byte alignment), which run on
the other kernels with the same result.
"""
import numpy as np
import pytest
import torch

import codebook_builder as cbb
from conftest import rel_l2

pytestmark = pytest.mark.gpu
TOL = 1e-5


def _nat():
    import cbq_native
    return cbq_native, cbq_native.load()


def _dev_packed(pk, dev):
    import bitpack
    return torch.from_numpy(bitpack.device_padded(pk)).to(dev)


def _case(rng, M, K, bits, C, bf16_cb):
    raw = rng.integers(0, 1 << bits, size=M * K)          # indices >= C: clamped to C - 1
    cb = (rng.standard_normal(C) * 0.02).astype(np.float32)
    if bf16_cb:
        cb = cbb.bf16_round(cb).astype(np.float32)
    return raw, cb


def _linear(dev, x, pk, cb, M, K, C, bits, x_offset=0):
    nat, lib = _nat()
    assert np.asarray(pk).size >= (M * K * bits + 7) // 8
    T = x.shape[0]
    xbuf = torch.zeros(T * K + 8, device=dev)
    xd = xbuf[x_offset:x_offset + T * K]
    xd.copy_(torch.from_numpy(np.ascontiguousarray(x, np.float32)).reshape(-1))
    pd = _dev_packed(pk, dev)
    cd = torch.from_numpy(np.ascontiguousarray(cb, np.float32)).to(dev)
    out = torch.full((T, M), float("nan"), device=dev)
    nat.check(lib.ck_linear_f32(xd.data_ptr(), pd.data_ptr(), cd.data_ptr(), out.data_ptr(), T,
                                M, K, C, bits, nat.stream_ptr(dev)), "ck_linear_f32")
    torch.cuda.synchronize()
    return out.cpu().numpy()


@pytest.mark.parametrize("bits", [8, 10, 11, 12, 13, 14, 16])
@pytest.mark.parametrize("bf16_cb", [True, False])
def test_widths_and_codebooks(cuda, oracle, bits, bf16_cb):
    rng = np.random.default_rng(bits * 7 + bf16_cb)
    M, K = 200, 1024
    C = min(1 << bits, 3000)
    raw, cb = _case(rng, M, K, bits, C, bf16_cb)
    pk = oracle.pack_lsb(raw, bits)
    for T in (2, 3, 16):
        x = rng.standard_normal((T, K)).astype(np.float32)
        y = _linear(cuda, x, pk, cb, M, K, C, bits)
        ref = oracle.fixed_gemv(x, pk, cb, M, K, bits, C=C, chunk_rows=None)
        assert rel_l2(y, ref) <= TOL, (bits, bf16_cb, T)


def _plan_rows(ncu):
    # tiles of 16 rows, R tiles per block of least rounds x (R + 1):
    # 6 ncu - 2 tiles -> 6, 2.5 ncu + 1 -> 3, 1.5 ncu + 1 -> 2, ncu - 4 -> 1 (ragged M)
    return {6: 96 * ncu - 40, 3: 40 * ncu + 8, 2: 24 * ncu + 8, 1: ncu * 16 - 72}


@pytest.mark.parametrize("plan", [6, 3, 2, 1])
def test_row_tile_plans(cuda, oracle, plan):
    ncu = torch.cuda.get_device_properties(cuda).multi_processor_count
    M = _plan_rows(ncu)[plan]
    K, bits, C = 512, 13, 5000
    rng = np.random.default_rng(plan)
    raw, cb = _case(rng, M, K, bits, C, True)
    pk = oracle.pack_lsb(raw, bits)
    x = rng.standard_normal((5, K)).astype(np.float32)
    y = _linear(cuda, x, pk, cb, M, K, C, bits)
    ref = oracle.fixed_gemv(x, pk, cb, M, K, bits, C=C, chunk_rows=None)
    assert rel_l2(y, ref) <= TOL, (plan, M)


@pytest.mark.parametrize("K", [128, 384, 896, 12288])
def test_few_steps_and_long_rows(cuda, oracle, K):
    """K / 128 below, at and above the 8 waves of a block (waves with no
    step contribute zeros), and a 12288-column row."""
    rng = np.random.default_rng(K)
    M, bits, C = 333, 12, 4096
    raw, cb = _case(rng, M, K, bits, C, True)
    pk = oracle.pack_lsb(raw, bits)
    for T in (2, 16):
        x = rng.standard_normal((T, K)).astype(np.float32)
        y = _linear(cuda, x, pk, cb, M, K, C, bits)
        ref = oracle.fixed_gemv(x, pk, cb, M, K, bits, C=C, chunk_rows=None)
        assert rel_l2(y, ref) <= TOL, (K, T)


def test_x_dynamic_range(cuda, oracle):
    """x spanning 1e-12 .. 1e12 per token: each bf16 part of the split keeps
    its own exponent, so the products stay exact."""
    rng = np.random.default_rng(11)
    M, K, bits, C = 160, 1024, 13, 8192
    raw, cb = _case(rng, M, K, bits, C, True)
    pk = oracle.pack_lsb(raw, bits)
    T = 6
    x = (rng.standard_normal((T, K)) * 10.0 ** rng.integers(-12, 13, size=(T, 1))).astype(np.float32)
    y = _linear(cuda, x, pk, cb, M, K, C, bits)
    ref = oracle.fixed_gemv(x, pk, cb, M, K, bits, C=C, chunk_rows=None)
    for t in range(T):
        assert rel_l2(y[t], ref[t]) <= TOL, t


def test_refused_shapes_fall_back(cuda, oracle):
    """K % 128 != 0 and x 4 bytes off 16-byte alignment take the other
    few-token kernels; results agree with the oracle either way."""
    rng = np.random.default_rng(5)
    bits, C = 13, 6000
    for M, K, off in ((300, 1056, 0), (300, 1024, 1)):
        raw, cb = _case(rng, M, K, bits, C, True)
        pk = oracle.pack_lsb(raw, bits)
        for T in (3, 9):
            x = rng.standard_normal((T, K)).astype(np.float32)
            y = _linear(cuda, x, pk, cb, M, K, C, bits, x_offset=off)
            ref = oracle.fixed_gemv(x, pk, cb, M, K, bits, C=C, chunk_rows=None)
            assert rel_l2(y, ref) <= TOL, (M, K, off, T)


@pytest.mark.parametrize("plan", [6, 2])
def test_bf16_row_tile_plans(cuda, oracle, plan):
    """bf16 x and out (ck_linear_bf16) through the 6- and 2-tile plans."""
    nat, lib = _nat()
    ncu = torch.cuda.get_device_properties(cuda).multi_processor_count
    M, K, bits, C = _plan_rows(ncu)[plan], 512, 13, 5000
    rng = np.random.default_rng(40 + plan)
    raw, cb = _case(rng, M, K, bits, C, True)
    pk = oracle.pack_lsb(raw, bits)
    pd = _dev_packed(pk, cuda)
    cd = torch.from_numpy(cb).to(cuda)
    xb = torch.from_numpy(rng.standard_normal((7, K)).astype(np.float32)).bfloat16()
    xd = xb.to(cuda)
    out = torch.empty(7, M, dtype=torch.bfloat16, device=cuda)
    nat.check(lib.ck_linear_bf16(xd.data_ptr(), pd.data_ptr(), cd.data_ptr(), out.data_ptr(), 7,
                                 M, K, C, bits, nat.stream_ptr(cuda)), "ck_linear_bf16")
    ref = oracle.fixed_gemv(xb.float().numpy(), pk, cb, M, K, bits, C=C, chunk_rows=None)
    y = out.float().cpu().numpy()
    assert rel_l2(y, ref) <= 4e-3, plan
    assert (y == torch.from_numpy(ref).bfloat16().float().numpy()).mean() >= 0.99


def test_bf16_io_two_tokens(cuda, oracle):
    """bf16 x is one exact part: ck_linear_bf16 with 2 and 16 tokens."""
    nat, lib = _nat()
    M, K = 640, 2048
    w = cbb.bf16_round(np.random.default_rng(8).standard_normal((M, K)) * 0.02)
    d = cbb.compress_fixed(w)
    bits = d["bits"]
    # named device tensors: a temporary's memory would be recycled before the launch
    pd = _dev_packed(d["indices"], cuda)
    cd = torch.from_numpy(d["codebook"]).to(cuda)
    for T in (2, 16):
        xb = torch.randn(T, K).bfloat16()
        ref = oracle.fixed_gemv(xb.float().numpy(), d["indices"], d["codebook"], M, K, bits,
                                chunk_rows=None)
        xd = xb.to(cuda)
        out = torch.empty(T, M, dtype=torch.bfloat16, device=cuda)
        nat.check(lib.ck_linear_bf16(xd.data_ptr(), pd.data_ptr(), cd.data_ptr(), out.data_ptr(),
                                     T, M, K, len(d["codebook"]), bits, nat.stream_ptr(cuda)),
                  "ck_linear_bf16")
        y = out.float().cpu().numpy()
        assert rel_l2(y, ref) <= 4e-3
        assert (y == torch.from_numpy(ref).bfloat16().float().numpy()).mean() >= 0.99


def test_graph_replays_match_eager(cuda):
    """Captured in a HIP graph and replayed (no allocation, no memset inside),
    every replay equals the eager result bit for bit."""
    nat, lib = _nat()
    rng = np.random.default_rng(3)
    M, K, bits, C = 4096, 2048, 13, 8192
    raw = torch.from_numpy(rng.integers(0, C, size=M * K, dtype=np.int32)).to(cuda)
    pk = cbb.pack_torch(raw, bits)
    cd = torch.from_numpy(cbb.bf16_round(rng.standard_normal(C) * 0.02).astype(np.float32)).to(cuda)
    x = torch.randn(16, K, device=cuda)
    out = torch.empty(16, M, device=cuda)

    def run():
        nat.check(lib.ck_linear_f32(x.data_ptr(), pk.data_ptr(), cd.data_ptr(), out.data_ptr(), 16,
                                    M, K, C, bits, nat.stream_ptr(cuda)), "ck_linear_f32")
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
