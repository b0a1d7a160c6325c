"""Fixed-width GEMV / embedding on the GPU through the C ABI vs the oracle.

Bar: rel-L2 <= 1e-5 for fp32 outputs (fp32 accumulation, different order
from the oracle's sequential k loop); embedding gathers are bit-exact; bf16
I/O within bf16 output rounding (rel-L2 <= 4e-3, >= 99% of outputs equal to
the oracle's fp32 result rounded to bf16).
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


def _run_linear(dev, x, pk, cb, M, K, C, bits):
    nat, lib = _nat()
    # the C ABI trusts its sizes: never hand it a stream shorter than M*K*bits
    assert np.asarray(pk).size >= (M * K * bits + 7) // 8, "packed stream too short"
    xd = torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(dev)
    pd = _dev_packed(pk, dev)
    cd = torch.from_numpy(np.ascontiguousarray(cb, np.float32)).to(dev)
    out = torch.full((x.shape[0], M), float("nan"), device=dev)
    rc = lib.ck_linear_f32(xd.data_ptr(), pd.data_ptr(), cd.data_ptr(), out.data_ptr(),
                           x.shape[0], M, K, C, bits, nat.stream_ptr(dev))
    nat.check(rc, "ck_linear_f32")
    torch.cuda.synchronize()
    return out.cpu().numpy()


def test_golden_cases(cuda, golden):
    for name, c in golden["fixed"].items():
        M, K, bits, C = int(c["M"]), int(c["K"]), int(c["bits"]), int(c["C"])
        y = _run_linear(cuda, c["x"], c["packed"], c["cb"], M, K, C, bits)
        ref = c["y_T16"] if name == "bf16slice" else c["y"]
        print(name, M, K, bits, rel_l2(y, ref), flush=True)
        assert rel_l2(y, ref) <= TOL, name


@pytest.mark.parametrize("T", [1, 2, 4, 7, 16, 20])
def test_config1_shape(cuda, oracle, T):
    """Config 1: W[M=6144, K=2048] bf16 N(0, 0.02), 13-bit frequency-sorted."""
    M, K = 6144, 2048
    w = cbb.bf16_round(np.random.default_rng(0).standard_normal((M, K)) * 0.02)
    d = cbb.compress_fixed(w)
    assert d["bits"] == 13
    x = np.random.default_rng(1).standard_normal((T, K)).astype(np.float32)
    y = _run_linear(cuda, x, d["indices"], d["codebook"], M, K, len(d["codebook"]), 13)
    ref = oracle.fixed_gemv(x, d["indices"], d["codebook"], M, K, 13, chunk_rows=None)
    assert rel_l2(y, ref) <= TOL


@pytest.mark.parametrize("M,K,bits,C", [(100, 96, 7, 100), (77, 33, 13, 5000),
                                        (64, 128, 16, 40000), (33, 64, 10, 1024),
                                        (130, 4096, 14, 9686), (50, 12288, 13, 5091),
                                        (64, 1024, 12, 4000), (40, 160, 8, 200)])
def test_widths_shapes_and_generic_path(cuda, oracle, M, K, bits, C):
    rng = np.random.default_rng(M + K + bits)
    raw = rng.integers(0, 1 << bits, size=M * K)       # includes indices >= C: clamp
    cb = (rng.standard_normal(C) * 0.02).astype(np.float32)
    pk = oracle.pack_lsb(raw, bits)
    for T in (1, 3):
        x = rng.standard_normal((T, K)).astype(np.float32)
        y = _run_linear(cuda, x, pk, cb, M, K, C, bits)
        ref = oracle.fixed_gemv(x, pk, cb, M, K, bits, C=C, chunk_rows=None)
        assert rel_l2(y, ref) <= TOL, (M, K, bits, C, T)


@pytest.mark.parametrize("M,K,T", [(300, 12288, 4), (200, 16384, 3), (96, 32768, 2),
                                   (130, 10240, 4)])
def test_column_ranges_large_x(cuda, oracle, M, K, T):
    """2..4 tokens whose x does not fit in LDS beside the codebook: the
    streaming GEMV runs over balanced column ranges, the first launch writing
    out, the rest adding (5..16 tokens take the matrix cores instead)."""
    rng = np.random.default_rng(M * 7 + K + T)
    w = cbb.bf16_round(rng.standard_normal((M, K)) * 0.02)
    d = cbb.compress_fixed(w)
    x = rng.standard_normal((T, K)).astype(np.float32)
    y = _run_linear(cuda, x, d["indices"], d["codebook"], M, K, len(d["codebook"]), d["bits"])
    ref = oracle.fixed_gemv(x, d["indices"], d["codebook"], M, K, d["bits"], chunk_rows=None)
    assert rel_l2(y, ref) <= TOL, (M, K, T)


@pytest.mark.parametrize("bits", [8, 10, 11, 12, 13, 14, 16])
@pytest.mark.parametrize("T", [5, 16])
def test_matrix_core_token_tiles(cuda, oracle, bits, T):
    """5..16 fp32 tokens with K % 128 != 0 run on the fp32 matrix cores
    (fixed_tiny_mfma_kernel, cbq_tiny.hip): every width it takes, indices past
    C clamped, rows not a multiple of 32.  (K % 128 == 0 takes the bf16
    matrix-core kernel, tests/test_gpu_fewtok.py.)"""
    rng = np.random.default_rng(bits * 31 + T)
    M, K = 200, 1056
    C = min(1 << bits, 3000)
    raw = rng.integers(0, 1 << bits, size=M * K)
    cb = (rng.standard_normal(C) * 0.02).astype(np.float32)
    pk = oracle.pack_lsb(raw, bits)
    x = rng.standard_normal((T, K)).astype(np.float32)
    y = _run_linear(cuda, x, pk, cb, M, K, C, bits)
    ref = oracle.fixed_gemv(x, pk, cb, M, K, bits, C=C, chunk_rows=None)
    assert rel_l2(y, ref) <= TOL, (bits, T)


@pytest.mark.parametrize("T", [1, 8, 64])
def test_codebook_staging_unaligned(cuda, oracle, T):
    """The streaming (T = 1), bf16 few-token (T = 8) and fp32-prefill (T = 64)
    kernels stage the codebook in 16-byte pieces when it is 16-byte aligned;
    a codebook 4 bytes off alignment, with C not a multiple of 4 and indices
    past C, takes the element-wise copy and must give the same result."""
    nat, lib = _nat()
    rng = np.random.default_rng(41 + T)
    M, K, bits, C = 200, 1024, 12, 3001
    raw = rng.integers(0, 1 << bits, size=M * K)
    cb = (rng.standard_normal(C) * 0.02).astype(np.float32)
    pk = oracle.pack_lsb(raw, bits)
    x = rng.standard_normal((T, K)).astype(np.float32)
    ref = oracle.fixed_gemv(x, pk, cb, M, K, bits, C=C, chunk_rows=None)
    buf = torch.zeros(C + 8, device=cuda)
    cd = buf[1:1 + C]                                 # 4 bytes past a 16-byte boundary
    cd.copy_(torch.from_numpy(cb))
    assert cd.data_ptr() % 16 == 4
    xd = torch.from_numpy(x).to(cuda)
    pd = _dev_packed(pk, cuda)
    out = torch.full((T, M), float("nan"), device=cuda)
    nat.check(lib.ck_linear_f32(xd.data_ptr(), pd.data_ptr(), cd.data_ptr(), out.data_ptr(), T,
                                M, K, C, bits, nat.stream_ptr(cuda)), "ck_linear_f32")
    torch.cuda.synchronize()
    assert rel_l2(out.cpu().numpy(), ref) <= TOL
    y = _run_linear(cuda, x, pk, cb, M, K, C, bits)   # aligned codebook, same kernel
    assert rel_l2(out.cpu().numpy(), y) <= TOL
    if T == 1:
        # the one-token GEMVs that stage x through a transform, and the
        # gate/up pair launch: bit-equal with an aligned copy of the codebook
        ca = torch.from_numpy(cb).to(cuda)
        assert ca.data_ptr() % 16 == 0
        st = nat.stream_ptr(cuda)
        for cbd in (cd, ca):
            o1 = torch.full((1, M), float("nan"), device=cuda)
            o2 = torch.full((1, M // 2), float("nan"), device=cuda)
            nat.check(lib.cbq_linear_xform_f32(xd.data_ptr(), None, None, nat.XF_RMS, 1e-6,
                                               pd.data_ptr(), cbd.data_ptr(), o1.data_ptr(), M,
                                               K, C, bits, st), "cbq_linear_xform_f32")
            nat.check(lib.cbq_linear_xform_glu_f32(xd.data_ptr(), None, None, 0, 1e-6,
                                                   pd.data_ptr(), cbd.data_ptr(), o2.data_ptr(),
                                                   M // 2, K, C, bits, st),
                      "cbq_linear_xform_glu_f32")
            torch.cuda.synchronize()
            if cbd is cd:
                u1, u2 = o1.clone(), o2.clone()
        assert torch.equal(u1, o1) and torch.equal(u2, o2)
        assert not torch.isnan(o1).any() and not torch.isnan(o2).any()


@pytest.mark.parametrize("K,Ts", [(2048, (1, 5)), (4096, (16, 3, 9))])
def test_bf16_io(cuda, oracle, K, Ts):
    """ck_linear_bf16: streaming kernel (T <= 4) and matrix cores (5..16
    tokens, x of 16 tokens at K = 4096 larger than LDS)."""
    nat, lib = _nat()
    M = 512
    w = cbb.bf16_round(np.random.default_rng(2).standard_normal((M, K)) * 0.02)
    d = cbb.compress_fixed(w)
    bits = d["bits"]                      # 12-bit indices at K = 2048, 13 at 4096
    assert d["indices"].size >= (M * K * bits + 7) // 8
    for T in Ts:
        xb = torch.randn(T, K).bfloat16()
        x32 = xb.float().numpy()
        ref = oracle.fixed_gemv(x32, d["indices"], d["codebook"], M, K, bits, chunk_rows=None)
        xd = xb.to(cuda)
        pd = _dev_packed(d["indices"], cuda)
        cd = torch.from_numpy(d["codebook"]).to(cuda)
        out = torch.empty(T, M, dtype=torch.bfloat16, device=cuda)
        rc = lib.ck_linear_bf16(xd.data_ptr(), pd.data_ptr(), cd.data_ptr(), out.data_ptr(), T, M,
                                K, len(d["codebook"]), bits, nat.stream_ptr(cuda))
        nat.check(rc, "ck_linear_bf16")
        y = out.float().cpu().numpy()
        assert rel_l2(y, ref) <= 4e-3
        ref_b = torch.from_numpy(ref).bfloat16().float().numpy()
        assert (y == ref_b).mean() >= 0.99


def test_int64_offsets_large(cuda, oracle):
    """M*K*bits > 2^31 bits (tests/test_c_kernel.py:109-138 of the reference)."""
    M, K, bits = 41472, 4096, 13            # 170M indices, 2.2G bits
    rng = np.random.default_rng(7)
    raw = rng.integers(0, 1 << bits, size=M * K, dtype=np.uint16)
    cb = (rng.standard_normal(1 << bits) * 0.02).astype(np.float32)
    pk = cbb.pack_torch(torch.from_numpy(raw).to(cuda), bits).cpu().numpy()
    x = rng.standard_normal((1, K)).astype(np.float32)
    y = _run_linear(cuda, x, pk, cb, M, K, 1 << bits, bits)
    rows = np.array([0, 1, M // 2, M - 2, M - 1])
    ref = (x.astype(np.float64) @ cb[raw.reshape(M, K)[rows]].astype(np.float64).T)
    assert rel_l2(y[:, rows], ref) <= TOL


def test_determinism_and_back_to_back(cuda):
    from gpu_accelerated_functions import GPUAcceleratedLinear
    M, K = 2048, 4096
    w = cbb.bf16_round(np.random.default_rng(4).standard_normal((M, K)) * 0.02)
    d = cbb.compress_fixed(w)
    lin = GPUAcceleratedLinear("det", d["indices"], torch.from_numpy(d["codebook"]), (M, K),
                               d["bits"])
    x = torch.randn(3, K, device=cuda)
    outs = [lin(x) for _ in range(5)]
    torch.cuda.synchronize()
    for o in outs[1:]:
        assert torch.equal(o, outs[0])


@pytest.mark.parametrize("H,bits,C", [(4096, 13, 5000), (2048, 14, 9000), (96, 7, 100),
                                      (100, 12, 3000)])
def test_embedding_exact(cuda, oracle, H, bits, C):
    nat, lib = _nat()
    vocab = 300
    rng = np.random.default_rng(H + bits)
    raw = rng.integers(0, 1 << bits, size=vocab * H)
    cb = (rng.standard_normal(C) * 0.02).astype(np.float32)
    pk = oracle.pack_lsb(raw, bits)
    ids = np.array([0, vocab - 1, 17, 17, 250, 3], np.int32)
    ref = oracle.fixed_embedding(ids, pk, cb, H, bits, C=C)
    pd = _dev_packed(pk, cuda)
    cd = torch.from_numpy(cb).to(cuda)
    idd = torch.from_numpy(ids).to(cuda)
    for fn in ("ck_embedding_f32", "cbq_embedding_f32"):
        out = torch.full((len(ids), H), float("nan"), device=cuda)
        if fn == "ck_embedding_f32":
            rc = lib.ck_embedding_f32(idd.data_ptr(), pd.data_ptr(), cd.data_ptr(), out.data_ptr(),
                                      len(ids), H, C, bits, nat.stream_ptr(cuda))
        else:
            rc = lib.cbq_embedding_f32(idd.data_ptr(), pd.data_ptr(), cd.data_ptr(),
                                       out.data_ptr(), len(ids), vocab, H, C, bits,
                                       nat.stream_ptr(cuda))
        nat.check(rc, fn)
        assert np.array_equal(out.cpu().numpy(), ref), fn


def test_embedding_clamps_ids(cuda, oracle):
    from gpu_accelerated_functions import GPUAcceleratedEmbedding
    vocab, H, bits = 10, 64, 8
    raw = np.random.default_rng(0).integers(0, 256, size=vocab * H)
    cb = np.arange(256, dtype=np.float32)
    emb = GPUAcceleratedEmbedding("e", oracle.pack_lsb(raw, bits), torch.from_numpy(cb),
                                  (vocab, H), bits)
    out = emb(torch.tensor([[-5, 3, 99]], device=cuda)).cpu().numpy()
    assert out.shape == (1, 3, H)
    assert np.array_equal(out[0, 0], cb[raw[:H]])
    assert np.array_equal(out[0, 2], cb[raw[(vocab - 1) * H:]])


@pytest.mark.parametrize("T", [1, 3, 20])
def test_affine_implicit_codebook_bit_exact(cuda, oracle, T):
    """cbq_linear_affine_f32 over re-indexed weights equals ck_linear_f32 over
    the frequency-sorted codebook bit for bit at T = 1 (same values, same
    streaming kernel and order of accumulation), zeros of either sign
    included; with 2..16-token tiles (T = 3, 20) the table path runs on the
    matrix cores (another order of accumulation), so there the two agree to
    rounding; both match the oracle."""
    import bitpack
    import cbq_native as nat
    rng = np.random.default_rng(40 + T)
    M, K = 200, 1024
    w = cbb.bf16_round(rng.standard_normal((M, K)) * 0.02)
    w[3, 7], w[150, 1000] = 0.0, -0.0
    cb, idx = cbb.frequency_sorted_codebook(w)
    bits = 13                  # the 9B-shape width; a small sample's codebook is narrower
    assert len(cb) <= 1 << bits
    aff = cbb.affine_form(cb, bits)
    assert aff is not None
    lo, wid, remap = aff
    packed = bitpack.device_padded(bitpack.pack_any_bits(idx.reshape(-1), bits))
    packed_aff = bitpack.device_padded(bitpack.pack_any_bits(remap[idx.reshape(-1)], bits))
    lib = nat.load()
    x = torch.from_numpy(rng.standard_normal((T, K)).astype(np.float32)).to(cuda)
    cbt = torch.from_numpy(cb).to(cuda)
    pk = torch.from_numpy(packed).to(cuda)
    pka = torch.from_numpy(packed_aff).to(cuda)
    y = torch.empty(T, M, device=cuda)
    ya = torch.empty(T, M, device=cuda)
    st = nat.stream_ptr(cuda)
    nat.check(lib.ck_linear_f32(x.data_ptr(), pk.data_ptr(), cbt.data_ptr(), y.data_ptr(), T, M, K,
                                len(cb), bits, st), "table")
    nat.check(lib.cbq_linear_affine_f32(x.data_ptr(), pka.data_ptr(), lo, wid, ya.data_ptr(), T, M,
                                        K, bits, st), "affine")
    if T == 1:
        assert torch.equal(y, ya)
    else:
        assert rel_l2(y.cpu().numpy(), ya.cpu().numpy()) <= 2e-6
    ref = oracle.fixed_gemv(x.cpu().numpy(), packed, cb, M, K, bits)
    assert rel_l2(ya.cpu().numpy(), ref) <= 1e-5
    assert rel_l2(y.cpu().numpy(), ref) <= 1e-5

