"""bf16 MFMA prefill path of ck_linear_bf16 (T >= 64) vs the oracle.

Bar for the bf16-MFMA prefill: rel-L2 <= 2e-3 against the fp32 reference GEMV
on the same bf16 inputs; outputs are bf16, so >= 95% of them must also equal
the oracle's fp32 result rounded to bf16 within one bf16 ulp.
"""
import numpy as np
import pytest
import torch

import codebook_builder as cbb
from conftest import rel_l2

pytestmark = pytest.mark.gpu
TOL = 2e-3


def _prefill(cuda, xb, pk, cb, M, K, bits, split=False):
    """ck_linear_bf16 (x read row-major), or with split cbq_linear_bf16_ws
    with its workspace (x copied to fragment order, K split when the grid is
    small)."""
    import bitpack
    import cbq_native as nat
    lib = nat.load()
    T = xb.shape[0]
    pd = torch.from_numpy(bitpack.device_padded(pk)).to(cuda)
    cd = torch.from_numpy(np.ascontiguousarray(cb, np.float32)).to(cuda)
    xd = xb.to(cuda).contiguous()
    out = torch.full((T, M), float("nan"), dtype=torch.bfloat16, device=cuda)
    if split:
        nws = int(lib.cbq_linear_bf16_workspace(T, M, K))
        assert nws > 0, "shape expected to take the MFMA path"
        ws = torch.full((nws // 4,), float("nan"), dtype=torch.float32, device=cuda)
        rc = lib.cbq_linear_bf16_ws(xd.data_ptr(), pd.data_ptr(), cd.data_ptr(), out.data_ptr(),
                                    T, M, K, len(cb), bits, ws.data_ptr(), nws,
                                    nat.stream_ptr(cuda))
        nat.check(rc, "cbq_linear_bf16_ws")
    else:
        rc = lib.ck_linear_bf16(xd.data_ptr(), pd.data_ptr(), cd.data_ptr(), out.data_ptr(), T,
                                M, K, len(cb), bits, nat.stream_ptr(cuda))
        nat.check(rc, "ck_linear_bf16")
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


def _check(y, ref):
    assert np.isfinite(y).all()
    assert rel_l2(y, ref) <= TOL, rel_l2(y, ref)
    ref_b = torch.from_numpy(ref).bfloat16().float().numpy()
    ulp = np.abs(ref_b) * 2.0 ** -7 + 1e-30
    assert (np.abs(y - ref_b) <= ulp).mean() >= 0.95


@pytest.mark.parametrize("T,M,K", [(64, 128, 256), (100, 300, 4096), (256, 384, 2048),
                                   (300, 200, 1024), (512, 136, 12288)])
def test_lossless_bf16(cuda, oracle, T, M, K):
    """Config 4 style: bf16 N(0, 0.02) weights, lossless frequency-sorted
    codebook (13 bits), bf16 activations N(0, 1)."""
    w = cbb.bf16_round(np.random.default_rng(T + M).standard_normal((M, K)) * 0.02)
    d = cbb.compress_fixed(w)
    bits = d["bits"]
    xb = torch.randn(T, K, generator=torch.Generator().manual_seed(T)).bfloat16()
    y = _prefill(cuda, xb, d["indices"], d["codebook"], M, K, bits)
    ref = oracle.fixed_gemv(xb.float().numpy(), d["indices"], d["codebook"], M, K, bits,
                            chunk_rows=None)
    _check(y, ref)


@pytest.mark.parametrize("bits,C", [(8, 200), (12, 4000), (13, 5000), (14, 9000)])
def test_widths_and_clamp(cuda, oracle, bits, C):
    """Raw indices above C-1 clamp; codebook values are bf16-exact here."""
    T, M, K = 128, 160, 512
    rng = np.random.default_rng(bits)
    raw = rng.integers(0, 1 << bits, size=M * K)
    cb = cbb.bf16_round(rng.standard_normal(C) * 0.05).astype(np.float32)
    pk = oracle.pack_lsb(raw, bits)
    xb = torch.from_numpy(rng.standard_normal((T, K)).astype(np.float32)).bfloat16()
    y = _prefill(cuda, xb, pk, cb, M, K, bits)
    ref = oracle.fixed_gemv(xb.float().numpy(), pk, cb, M, K, bits, C=C, chunk_rows=None)
    _check(y, ref)


def test_fp32_codebook_rounds_to_bf16(cuda, oracle):
    """A codebook that is not bf16-exact feeds the MFMA rounded to bf16; the
    result stays within the prefill tolerance."""
    T, M, K, bits, C = 192, 256, 2048, 12, 3000
    rng = np.random.default_rng(7)
    raw = rng.integers(0, C, size=M * K)
    cb = (rng.standard_normal(C) * 0.05).astype(np.float32)
    pk = oracle.pack_lsb(raw, bits)
    xb = torch.from_numpy(rng.standard_normal((T, K)).astype(np.float32)).bfloat16()
    y = _prefill(cuda, xb, pk, cb, M, K, bits)
    ref = oracle.fixed_gemv(xb.float().numpy(), pk, cb, M, K, bits, C=C, chunk_rows=None)
    assert rel_l2(y, ref) <= TOL


def test_matches_token_tile_path(cuda):
    """T = 64 runs the MFMA path, T = 16 the VALU token tiles: rows common to
    both agree within bf16 output rounding."""
    M, K = 512, 4096
    w = cbb.bf16_round(np.random.default_rng(1).standard_normal((M, K)) * 0.02)
    d = cbb.compress_fixed(w)
    xb = torch.randn(64, K, generator=torch.Generator().manual_seed(3)).bfloat16()
    y64 = _prefill(cuda, xb, d["indices"], d["codebook"], M, K, d["bits"])
    y16 = _prefill(cuda, xb[:16].clone(), d["indices"], d["codebook"], M, K, d["bits"])
    assert rel_l2(y64[:16], y16) <= TOL


@pytest.mark.parametrize("T,M,K", [(100, 300, 4096), (512, 136, 12288), (512, 1024, 4096),
                                   (300, 2048, 4096)])
def test_split_k_matches_oracle(cuda, oracle, T, M, K):
    """Small output grids split K across blocks (fp32 partials in the
    caller's workspace, summed in split order): the same tolerance against
    the oracle, and the same output as the unsplit kernel within it."""
    w = cbb.bf16_round(np.random.default_rng(T * 3 + M).standard_normal((M, K)) * 0.02)
    d = cbb.compress_fixed(w)
    xb = torch.randn(T, K, generator=torch.Generator().manual_seed(M)).bfloat16()
    ys = _prefill(cuda, xb, d["indices"], d["codebook"], M, K, d["bits"], split=True)
    ref = oracle.fixed_gemv(xb.float().numpy(), d["indices"], d["codebook"], M, K, d["bits"],
                            chunk_rows=None)
    _check(ys, ref)
    y1 = _prefill(cuda, xb, d["indices"], d["codebook"], M, K, d["bits"])
    assert rel_l2(ys, y1) <= TOL


def _tiles(T, M):
    return -(-T // 512) * -(-M // 128)


@pytest.mark.parametrize("T,M,K", [(1030, 8200, 512), (2048, 12288, 128), (1100, 12288, 512)])
def test_workspace_path_ragged(cuda, oracle, T, M, K):
    """Large grids through cbq_linear_bf16_ws (x in fragment order): T and M
    off every tile multiple, the padded last token block and feature tile
    included.  195 tiles run whole; 384 tiles at K = 128 too (too few K
    groups to split); 288 tiles (32 past a full round of the CUs) split the
    last 32 tiles' K in two, with partials in the workspace after x."""
    import cbq_native as nat
    xf = ((T + 15) // 16 * 16 * K * 2 + 255) // 256 * 256
    nws = nat.load().cbq_linear_bf16_workspace(T, M, K)
    cus = torch.cuda.get_device_properties(cuda).multi_processor_count
    left = _tiles(T, M) % cus
    if K // 32 >= 16 and _tiles(T, M) > cus and 0 < 2 * left <= cus:
        assert nws == xf + left * min(cus // left, 16, K // 256) * 512 * 128 * 4
    else:
        assert nws == xf
    w = cbb.bf16_round(np.random.default_rng(T + K).standard_normal((M, K)) * 0.02)
    d = cbb.compress_fixed(w)
    xb = torch.randn(T, K, generator=torch.Generator().manual_seed(K)).bfloat16()
    y = _prefill(cuda, xb, d["indices"], d["codebook"], M, K, d["bits"], split=True)
    ref = oracle.fixed_gemv(xb.float().numpy(), d["indices"], d["codebook"], M, K, d["bits"],
                            chunk_rows=None)
    _check(y, ref)
    y1 = _prefill(cuda, xb, d["indices"], d["codebook"], M, K, d["bits"])
    assert rel_l2(y, y1) <= TOL


def test_split_workspace_reused_and_replayed(cuda, oracle):
    """One workspace (x in fragment order, split partials) reused by eager
    calls and by graph replays with new x in between: every result against
    the oracle (a stale x copy or partial would not match)."""
    import bitpack
    import cbq_native as nat
    lib = nat.load()
    T, M, K = 512, 1024, 4096                     # 8 tiles, K in 16
    w = cbb.bf16_round(np.random.default_rng(77).standard_normal((M, K)) * 0.02)
    d = cbb.compress_fixed(w)
    pd = torch.from_numpy(bitpack.device_padded(d["indices"])).to(cuda)
    cd = torch.from_numpy(np.ascontiguousarray(d["codebook"], np.float32)).to(cuda)
    nws = int(lib.cbq_linear_bf16_workspace(T, M, K))
    ws = torch.full((nws // 4,), float("nan"), dtype=torch.float32, device=cuda)
    xd = torch.empty(T, K, dtype=torch.bfloat16, device=cuda)
    out = torch.empty(T, M, dtype=torch.bfloat16, device=cuda)

    def call():
        nat.check(lib.cbq_linear_bf16_ws(xd.data_ptr(), pd.data_ptr(), cd.data_ptr(),
                                         out.data_ptr(), T, M, K, len(d["codebook"]),
                                         d["bits"], ws.data_ptr(), nws,
                                         nat.stream_ptr(cuda)), "cbq_linear_bf16_ws")

    def check():
        xb = xd.float().cpu().numpy()
        ref = oracle.fixed_gemv(xb, d["indices"], d["codebook"], M, K, d["bits"],
                                chunk_rows=None)
        _check(out.float().cpu().numpy(), ref)

    for seed in (1, 2):                           # eager, same workspace
        xd.copy_(torch.randn(T, K, generator=torch.Generator().manual_seed(seed)).bfloat16())
        out.fill_(float("nan"))
        call()
        torch.cuda.synchronize()
        check()
    s = torch.cuda.Stream(cuda)
    s.wait_stream(torch.cuda.current_stream(cuda))
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            call()
    torch.cuda.current_stream(cuda).wait_stream(s)
    for seed in (3, 4, 5):                        # replays, new x each time
        xd.copy_(torch.randn(T, K, generator=torch.Generator().manual_seed(seed)).bfloat16())
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        check()


def test_split_k_inexact_codebook_and_clamp(cuda, oracle):
    T, M, K, bits, C = 128, 200, 8192, 12, 3000
    rng = np.random.default_rng(9)
    raw = rng.integers(0, 1 << bits, size=M * K)
    cb = (rng.standard_normal(C) * 0.05).astype(np.float32)
    pk = oracle.pack_lsb(raw, bits)
    xb = torch.from_numpy(rng.standard_normal((T, K)).astype(np.float32)).bfloat16()
    y = _prefill(cuda, xb, pk, cb, M, K, bits, split=True)
    ref = oracle.fixed_gemv(xb.float().numpy(), pk, cb, M, K, bits, C=C, chunk_rows=None)
    assert rel_l2(y, ref) <= TOL
