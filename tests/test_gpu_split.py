"""Split format on the GPU: cbq_split_pack writes exactly the CPU
packer's layout, and cbq_split_linear_f32 (single, grouped, with the folded
glue) equals the column-layout Huffman GEMV bit for bit on the same weights."""
import ctypes

import numpy as np
import pytest
import torch

import cbq_native as nat
import decoder
import synthetic
from gpu_huffman_functions import build_columns, build_split, decode_symbols
import huffman_codebook as hc
from test_split_format import bf16_codebook, cpu_pack

pytestmark = pytest.mark.gpu


def test_pack_matches_cpu_packer(cuda):
    rng = np.random.default_rng(3)
    cb = bf16_codebook(rng, 700)
    p = 1.0 / np.arange(1, cb.size + 1) ** 1.1
    idx = rng.choice(cb.size, size=3 * 4096, p=p / p.sum()).astype(np.int32)
    keep, desc = build_split(torch.from_numpy(idx).to(cuda), cb, cuda)
    cwords, row_off, raw, lut = keep
    sym_code, sym_raw, lut_h = hc.split_tables(cb, np.bincount(idx))
    cw, ro, rw = cpu_pack(idx.astype(np.int64), sym_code, sym_raw)
    assert np.array_equal(row_off.cpu().numpy(), ro)
    got = cwords.cpu().numpy().view(np.uint32).reshape(-1, 64)
    assert np.array_equal(got[:cw.shape[0]], cw) and got.shape[0] == cw.shape[0] + 3
    assert not got[cw.shape[0]:].any()                     # readable zero rows past the end
    assert np.array_equal(raw.cpu().numpy(), rw)
    assert np.array_equal(lut.cpu().numpy().view(np.uint32), lut_h)


@pytest.fixture(scope="module")
def huff(cuda):
    dec = synthetic.SyntheticDecoder("qwen3-8b", layers=1, log=lambda *a: None)
    p = "model.layers.0."
    names = [n for n in dec.all_linears() if n[0].startswith(p)]
    return dec, dec.build_huffman(names)


def _desc(t):
    tb = t.tables
    return nat.HuffStream(words=t.words.data_ptr(), n_words=t.words.numel(),
                          chunk_off=t.chunk_off.data_ptr(), sub_len=t.sub_len.data_ptr(),
                          lut1=tb["lut1"].data_ptr(), lut2=tb["lut2"].data_ptr(),
                          n_lut2=tb["lut2"].numel(), canon=tb["canon"].data_ptr(),
                          canon_pay=tb["pay"].data_ptr(), value_cb=None,
                          C=tb["codebook"].numel(), stage_words=tb["stage_words"])


def _both(t, cuda):
    M, K = t.shape
    d = _desc(t)
    cb = t.tables["codebook"].cpu().numpy()
    col = build_columns(d, M * K, cuda, t.lengths, cb)
    idx = decode_symbols(t.words, t.chunk_off, t.sub_len, t.lengths, M * K, cuda)
    sp = build_split(idx, cb, cuda)
    assert sp is not None
    return d, col, sp


def _split(lib, x, sps, Ms, K, mode=0, x1=None, h_out=None, eps=1e-6):
    n = len(sps)
    out = torch.empty(1, sum(Ms), device=x.device)
    offs = [out.data_ptr() + 4 * sum(Ms[:i]) for i in range(n)]
    nat.check(lib.cbq_split_linear_f32(
        x.data_ptr(), None if x1 is None else x1.data_ptr(),
        None if h_out is None else h_out.data_ptr(), mode, eps, n,
        (ctypes.POINTER(nat.SplitMatrix) * n)(*[ctypes.pointer(s[1]) for s in sps]),
        (ctypes.c_void_p * n)(*offs), (ctypes.c_int * n)(*Ms), K, nat.stream_ptr(x.device)),
        "cbq_split_linear_f32")
    return out


@pytest.mark.parametrize("name", ["mlp.gate_proj", "self_attn.k_proj", "mlp.down_proj"])
def test_split_equals_column_gemv(cuda, huff, name):
    dec, tensors = huff
    t = tensors["model.layers.0." + name]
    M, K = t.shape
    d, col, sp = _both(t, cuda)
    lib = nat.load()
    gen = torch.Generator(device=cuda).manual_seed(1)
    for rep in range(2):
        x = torch.randn(1, K, device=cuda, generator=gen)
        want = torch.empty(1, M, device=cuda)
        nat.check(lib.cbq_huff_linear_col_f32(x.data_ptr(), ctypes.byref(d), ctypes.byref(col[1]),
                                              want.data_ptr(), M, K, nat.stream_ptr(cuda)), "col")
        got = _split(lib, x, [sp], [M], K)
        assert torch.equal(got, want), (name, rep, float((got - want).abs().max()))
    # and against the dense weights (decoded values) in fp64
    idx = decode_symbols(t.words, t.chunk_off, t.sub_len, t.lengths, M * K, cuda).to(torch.int64)
    cbt = t.tables["codebook"].to(cuda)
    W = cbt[idx.clamp_max(cbt.numel() - 1)].reshape(M, K).double()
    ref = (W @ x.double().reshape(K, 1)).reshape(1, M)
    rel = float((got.double() - ref).norm() / ref.norm())
    assert rel < 1e-5, rel


def test_grouped_split_and_folded_glue(cuda, huff):
    dec, tensors = huff
    p = "model.layers.0."
    ts = [tensors[p + n] for n in ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj")]
    K = ts[0].shape[1]
    Ms = [t.shape[0] for t in ts]
    built = [_both(t, cuda) for t in ts]
    lib = nat.load()
    gen = torch.Generator(device=cuda).manual_seed(2)
    h = torch.randn(1, K, device=cuda, generator=gen) * 2
    dl = torch.randn(1, K, device=cuda, generator=gen)
    n = 3
    hs = (ctypes.POINTER(nat.HuffStream) * n)(*[ctypes.pointer(b[0]) for b in built])
    cols = (ctypes.POINTER(nat.HuffColumns) * n)(*[ctypes.pointer(b[1][1]) for b in built])
    for mode in (0, nat.XF_RMS, nat.XF_ADD_RMS):
        want = torch.empty(1, sum(Ms), device=cuda)
        offs = [want.data_ptr() + 4 * sum(Ms[:i]) for i in range(n)]
        h1 = torch.full_like(h, float("nan"))
        nat.check(lib.cbq_huff_linear_col_xform_f32(
            h.data_ptr(), dl.data_ptr() if mode == nat.XF_ADD_RMS else None,
            h1.data_ptr() if mode == nat.XF_ADD_RMS else None, mode, 1e-6, n, hs, cols,
            (ctypes.c_void_p * n)(*offs), (ctypes.c_int * n)(*Ms), K, nat.stream_ptr(cuda)), "col")
        h2 = torch.full_like(h, float("nan"))
        got = _split(lib, h, [b[2] for b in built], Ms, K, mode,
                     dl if mode == nat.XF_ADD_RMS else None,
                     h2 if mode == nat.XF_ADD_RMS else None)
        assert torch.equal(got, want), mode
        if mode == nat.XF_ADD_RMS:
            assert torch.equal(h1, h2)
    # SiLU product into down_proj
    t = tensors[p + "mlp.down_proj"]
    M, Kd = t.shape
    d, col, sp = _both(t, cuda)
    a = torch.randn(1, Kd, device=cuda, generator=gen)
    b = torch.randn(1, Kd, device=cuda, generator=gen)
    want = torch.empty(1, M, device=cuda)
    nat.check(lib.cbq_huff_linear_col_xform_f32(
        a.data_ptr(), b.data_ptr(), None, nat.XF_SILU, 1e-6, 1,
        (ctypes.POINTER(nat.HuffStream) * 1)(ctypes.pointer(d)),
        (ctypes.POINTER(nat.HuffColumns) * 1)(ctypes.pointer(col[1])),
        (ctypes.c_void_p * 1)(want.data_ptr()), (ctypes.c_int * 1)(M), Kd, nat.stream_ptr(cuda)),
        "col silu")
    got = _split(lib, a, [sp], [M], Kd, nat.XF_SILU, b)
    assert torch.equal(got, want)


@pytest.mark.parametrize("M,K", [(300, 4096), (70, 12288)])
def test_module_split_equals_columns(cuda, oracle, M, K):
    """HuffmanCodebookLinear builds the split format from the reference-format
    stream; its one-token output equals the column path's bit for bit and
    the reference C kernel's within fp32 tolerance."""
    import codebook_builder as cbb
    from conftest import rel_l2
    from test_gpu_huffman import _lin
    rng = np.random.default_rng(M + K)
    w = cbb.bf16_round(rng.standard_normal((M, K)) * 0.02)
    cb, idx = cbb.frequency_sorted_codebook(w)
    enc = hc.huffman_encode_indices(idx, shape=(M, K))
    a = _lin(enc, cb, M, K)
    b = _lin(enc, cb, M, K, layout="columns")
    assert a.split is not None and b.split is None and b.cols is not None
    x = torch.from_numpy(rng.standard_normal((1, K)).astype(np.float32)).to(cuda)
    ya, yb = a(x), b(x)
    assert torch.equal(ya, yb)
    ref = oracle.huff_gemv(x.cpu().numpy(), enc, cb, M, K, chunk_rows=None)
    assert rel_l2(ya.cpu().numpy(), ref) <= 1e-5
    y3 = a(torch.cat([x, x, x]))                   # T > 1: transient fixed-width stream
    assert rel_l2(y3[1:2].cpu().numpy(), ref) <= 1e-5


def _split_of(cuda, w):
    """(codebook, indices, split format) of bf16 weights w [M, K]."""
    import codebook_builder as cbb
    cb, idx = cbb.frequency_sorted_codebook(w)
    sp = build_split(torch.from_numpy(idx.astype(np.int32)).to(cuda), cb, cuda)
    assert sp is not None
    return cb, idx, sp


@pytest.mark.parametrize("Ms,K", [((2048, 1024, 1024), 2048), ((6144,), 2048),
                                  ((2048,), 6144), ((96, 40), 1024), ((64, 128), 3072),
                                  ((512,), 5120), ((8194, 6), 6144), ((36, 4), 7168),
                                  ((66, 2), 8192), ((2050, 2), 12288), ((40, 4), 9216),
                                  ((22, 2), 10240)])
def test_row_groups_against_oracle(cuda, oracle, Ms, K):
    """K % 4096 != 0: the split GEMV walks groups of 4096 / gcd(K, 4096) rows
    (2 for K = 2048, 6144; 4 for K = 1024, 3072, 5120).  Each matrix against
    the reference C kernel on the same indices (rel-L2 <= 1e-5), the grouped
    launch equal to one launch per matrix bit for bit.  With several chunks
    per group or row (K = 3072, 5120, 6144, 7168, 9216, 10240; 8192 and 12288
    as whole rows) one matrix goes to the kernel that puts a group's chunks on
    separate waves and a grouped launch to the row walk, so that equality
    holds between the two kernels; (8194, 6) x 6144 and (2050, 2) x 12288
    give that kernel several tiles per block."""
    import codebook_builder as cbb
    from conftest import rel_l2
    lib = nat.load()
    rng = np.random.default_rng(K + sum(Ms))
    x = rng.standard_normal((1, K)).astype(np.float32)
    xd = torch.from_numpy(x).to(cuda)
    built, singles = [], []
    for i, M in enumerate(Ms):
        w = cbb.bf16_round(rng.standard_normal((M, K)) * 0.02)
        cb, idx, sp = _split_of(cuda, w)
        y = _split(lib, xd, [sp], [M], K)
        packed = oracle.pack_lsb(idx.reshape(-1).astype(np.int64), cbb.bits_for(len(cb)))
        ref = oracle.fixed_gemv(x, packed, cb, M, K, cbb.bits_for(len(cb)), chunk_rows=None)
        assert rel_l2(y.cpu().numpy(), ref) <= 1e-5, (M, K)
        built.append(sp)
        singles.append(y)
    if len(Ms) > 1:
        got = _split(lib, xd, built, list(Ms), K)
        assert torch.equal(got, torch.cat(singles, dim=1))


@pytest.mark.parametrize("K", [2048, 6144, 1024])
def test_row_groups_folded_glue(cuda, K):
    """The folded RMSNorm / SiLU staging with row groups equals the glue
    kernel followed by the plain split GEMV bit for bit."""
    import codebook_builder as cbb
    lib = nat.load()
    rng = np.random.default_rng(K)
    M = 4096 // K * 96 if K < 4096 else 64
    w = cbb.bf16_round(rng.standard_normal((M, K)) * 0.02)
    _, _, sp = _split_of(cuda, w)
    cfg = decoder.DecoderConfig(layers=1, hidden=K, inter=K, n_q=1, n_kv=1, head_dim=64,
                                vocab=16)
    g = decoder._Glue(cfg)
    gen = torch.Generator(device=cuda).manual_seed(K)
    h = torch.randn(1, K, device=cuda, generator=gen) * 2
    dl = torch.randn(1, K, device=cuda, generator=gen)
    want = _split(lib, g.add_rms(h.clone(), None), [sp], [M], K)
    assert torch.equal(_split(lib, h, [sp], [M], K, nat.XF_RMS), want)
    hc_ = h.clone()
    want = _split(lib, g.add_rms(hc_, dl), [sp], [M], K)
    h2 = torch.full_like(h, float("nan"))
    assert torch.equal(_split(lib, h, [sp], [M], K, nat.XF_ADD_RMS, dl, h2), want)
    assert torch.equal(h2, hc_)
    want = _split(lib, g.silu_mul(h, dl), [sp], [M], K)
    assert torch.equal(_split(lib, h, [sp], [M], K, nat.XF_SILU, dl), want)


def test_split_decode_indices_exact(cuda, oracle):
    """decode_indices() of a split-only module (stream freed) returns the
    stored indices bit for bit, against the reference C decoder; T = 2..63
    and T >= 64 run through the transient fixed-width stream."""
    import codebook_builder as cbb
    from conftest import rel_l2
    from test_gpu_huffman import _lin
    rng = np.random.default_rng(21)
    M, K = 200, 6144
    w = cbb.bf16_round(rng.standard_normal((M, K)) * 0.02)
    cb, idx = cbb.frequency_sorted_codebook(w)
    enc = hc.huffman_encode_indices(idx, shape=(M, K))
    lin = _lin(enc, cb, M, K)
    assert lin.split is not None and lin.dev is None
    kind = "ref" if oracle.ref_available() else "oracle"
    want = oracle.huff_decode_indices(enc, M, K, kind=kind)
    assert np.array_equal(lin.decode_indices().cpu().numpy(), want)
    for T in (1, 3, 17, 70):
        x = rng.standard_normal((T, K)).astype(np.float32)
        y = lin(torch.from_numpy(x).to(cuda)).cpu().numpy()
        assert rel_l2(y, oracle.huff_gemv(x, enc, cb, M, K, chunk_rows=None)) <= 1e-5, T


@pytest.mark.parametrize("M,K", [(12288, 4096),      # 8B gate/up shape (reduced to 1 layer's)
                                 (1003, 4096),       # ragged pair count
                                 (40, 8192)])        # fewer pairs than waves, two chunks a row
def test_stacked_glu_equals_split_then_silu(cuda, oracle, M, K):
    """cbq_split_linear_glu_f32 over a [gate; up] pair re-coded under one
    shared table (stack_split) equals the two matrices' own split GEMVs
    followed by cbq_silu_mul_f32, bit for bit, for plain x and both folded
    norms; the part descriptors into the stacked arrays give each matrix's
    own outputs bit for bit; plain x agrees with the oracle's C GEMVs."""
    from gpu_huffman_functions import stack_split, split_indices, split_inverse
    lib = nat.load()
    st = nat.stream_ptr(cuda)
    import bitpack
    import codebook_builder as cbb
    # one codebook for both matrices, as the MLP category's
    ws = [synthetic.make_bf16((M, K), f"glu.{nm}.{M}x{K}", device=cuda) for nm in ("gate", "up")]
    cbt, lut = cbb.codebook_from_counts_torch(cbb.counts_torch(ws[0]) + cbb.counts_torch(ws[1]))
    cb = cbt.cpu().numpy()
    bits = cbb.bits_for(cb.size)
    sps, idxs = [], []
    for wb in ws:
        idx = lut[cbb.patterns_torch(wb).reshape(-1).to(torch.int64)].to(torch.int32)
        sp = build_split(idx, cb, cuda)
        assert sp is not None
        sps.append(sp)
        idxs.append(idx.cpu().numpy())
    del ws
    keep, sdesc, parts = stack_split(sps, cb, [M, M], K, cuda)
    inv = split_inverse(cb, cuda)
    for i in range(2):                            # parts decode to each matrix's indices
        got = split_indices((keep, parts[i]), inv, M * K, cuda).cpu().numpy()
        assert np.array_equal(got, idxs[i])
    gen = torch.Generator(device=cuda).manual_seed(M + K)

    def silu_mul(g, u):
        out = torch.empty(1, M, device=cuda)
        nat.check(lib.cbq_silu_mul_f32(g.data_ptr(), u.data_ptr(), out.data_ptr(), M, st),
                  "cbq_silu_mul_f32")
        return out

    def glu(x, d, h_out, mode):
        out = torch.full((1, M), float("nan"), device=cuda)
        nat.check(lib.cbq_split_linear_glu_f32(
            x.data_ptr(), None if d is None else d.data_ptr(),
            None if h_out is None else h_out.data_ptr(), mode, 1e-6, ctypes.byref(sdesc),
            out.data_ptr(), M, K, st), "cbq_split_linear_glu_f32")
        return out

    for mode in (0, nat.XF_RMS, nat.XF_ADD_RMS):
        h = torch.randn(1, K, device=cuda, generator=gen) * 2
        d = torch.randn(1, K, device=cuda, generator=gen) if mode == nat.XF_ADD_RMS else None
        h1 = torch.full_like(h, float("nan"))
        yg = _split(lib, h, [sps[0]], [M], K, mode, d, h1 if d is not None else None)
        yu = _split(lib, h, [sps[1]], [M], K, mode, d, None)
        # the part descriptors (shared table) give the same outputs
        both = _split(lib, h, [(keep, parts[0]), (keep, parts[1])], [M, M], K, mode, d, None)
        assert torch.equal(both[:, :M], yg) and torch.equal(both[:, M:], yu), mode
        want = silu_mul(yg, yu)
        h2 = torch.full_like(h, float("nan"))
        got = glu(h, d, h2 if d is not None else None, mode)
        assert torch.equal(got, want), mode
        if d is not None:
            assert torch.equal(h1, h2)
        if mode == 0:
            xs = h.cpu().numpy()
            gref = oracle.fixed_gemv(xs, bitpack.pack_any_bits(idxs[0], bits), cb, M, K, bits)
            uref = oracle.fixed_gemv(xs, bitpack.pack_any_bits(idxs[1], bits), cb, M, K, bits)
            g64, u64 = gref.astype(np.float64), uref.astype(np.float64)
            ref = g64 / (1.0 + np.exp(-g64)) * u64
            rel = float(np.linalg.norm(got.cpu().numpy() - ref) / np.linalg.norm(ref))
            assert rel <= 1e-5, rel
