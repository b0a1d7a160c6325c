"""fp32 MFMA path of ck_linear_f32 (T >= 64) and its split-K form
cbq_linear_f32_ws vs the oracle (compressed_matmul_f32_chunk restated).

Products are exact in fp32 (v_mfma_f32_32x32x2_f32) and only the summation
order differs, so the bar is the fp32 GEMV's: rel-L2 <= 1e-5."""
import numpy as np
import pytest
import torch

import codebook_builder as cbb
from conftest import rel_l2

pytestmark = pytest.mark.gpu
TOL = 1e-5


def _run(cuda, x, pk, cb, M, K, bits, split=False):
    import bitpack
    import cbq_native as nat
    lib = nat.load()
    T = x.shape[0]
    pd = torch.from_numpy(bitpack.device_padded(pk)).to(cuda)
    cd = torch.from_numpy(np.ascontiguousarray(cb, np.float32)).to(cuda)
    xd = torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(cuda)
    out = torch.full((T, M), float("nan"), dtype=torch.float32, device=cuda)
    if split:
        nws = int(lib.cbq_linear_f32_workspace(T, M, K))
        if nws == 0:
            pytest.skip("no K split for this shape")
        ws = torch.full((nws // 4,), float("nan"), dtype=torch.float32, device=cuda)
        nat.check(lib.cbq_linear_f32_ws(xd.data_ptr(), pd.data_ptr(), cd.data_ptr(),
                                        out.data_ptr(), T, M, K, len(cb), bits, ws.data_ptr(),
                                        nws, nat.stream_ptr(cuda)), "cbq_linear_f32_ws")
    else:
        nat.check(lib.ck_linear_f32(xd.data_ptr(), pd.data_ptr(), cd.data_ptr(), out.data_ptr(),
                                    T, M, K, len(cb), bits, nat.stream_ptr(cuda)), "ck_linear_f32")
    torch.cuda.synchronize()
    return out.cpu().numpy()


@pytest.mark.parametrize("T,M,K", [(64, 128, 256), (100, 300, 4096), (300, 200, 1024),
                                   (513, 136, 2048)])
@pytest.mark.parametrize("split", [False, True])
def test_lossless_bf16_weights(cuda, oracle, T, M, K, split):
    w = cbb.bf16_round(np.random.default_rng(T + M).standard_normal((M, K)) * 0.02)
    d = cbb.compress_fixed(w)
    x = np.random.default_rng(K).standard_normal((T, K)).astype(np.float32)
    y = _run(cuda, x, d["indices"], d["codebook"], M, K, d["bits"], split)
    ref = oracle.fixed_gemv(x, d["indices"], d["codebook"], M, K, d["bits"], chunk_rows=None)
    assert np.isfinite(y).all()
    assert rel_l2(y, ref) <= TOL, rel_l2(y, ref)


@pytest.mark.parametrize("bits,C", [(8, 200), (10, 1000), (12, 4000), (13, 5000)])
def test_widths_clamp_and_fp32_codebook(cuda, oracle, bits, C):
    """Raw indices above C-1 clamp; codebook values are arbitrary fp32."""
    T, M, K = 128, 160, 1024
    rng = np.random.default_rng(bits)
    raw = rng.integers(0, 1 << bits, size=M * K)
    cb = (rng.standard_normal(C) * 0.05).astype(np.float32)
    pk = oracle.pack_lsb(raw, bits)
    x = rng.standard_normal((T, K)).astype(np.float32)
    y = _run(cuda, x, pk, cb, M, K, bits)
    ref = oracle.fixed_gemv(x, pk, cb, M, K, bits, C=C, chunk_rows=None)
    assert rel_l2(y, ref) <= TOL, rel_l2(y, ref)


def test_matches_token_tile_path(cuda):
    """T = 64 runs the MFMA path, T = 16 the GEMV token tiles: rows common to
    both agree within fp32 rounding."""
    M, K = 512, 4096
    w = cbb.bf16_round(np.random.default_rng(1).standard_normal((M, K)) * 0.02)
    d = cbb.compress_fixed(w)
    x = np.random.default_rng(3).standard_normal((64, K)).astype(np.float32)
    y64 = _run(cuda, x, d["indices"], d["codebook"], M, K, d["bits"])
    y16 = _run(cuda, x[:16].copy(), d["indices"], d["codebook"], M, K, d["bits"])
    assert rel_l2(y64[:16], y16) <= TOL


@pytest.mark.parametrize("M,K", [(300, 4096), (70, 12288)])
def test_huffman_module_batched_tokens(cuda, oracle, M, K):
    """HuffmanCodebookLinear with T >= 64 decodes its format to transient
    fixed-width indices (the split format through cbq_split_to_packed, the
    stream through cbq_huff_decode_indices + cbq_pack_indices) and runs the
    fp32 matrix-core GEMM; both layouts against the reference C kernel."""
    import huffman_codebook as hc
    from test_gpu_huffman import _lin
    rng = np.random.default_rng(M)
    w = cbb.bf16_round(rng.standard_normal((M, K)) * 0.02)
    cb, idx = cbb.frequency_sorted_codebook(w)
    enc = hc.huffman_encode_indices(idx, shape=(M, K))
    x = rng.standard_normal((96, K)).astype(np.float32)
    ref = oracle.huff_gemv(x, enc, cb, M, K, chunk_rows=None)
    for layout in ("auto", "stream"):
        lin = _lin(enc, cb, M, K, layout=layout)
        assert (lin.split is not None) == (layout == "auto")
        y = lin(torch.from_numpy(x).to(cuda)).cpu().numpy()
        assert rel_l2(y, ref) <= TOL, (layout, rel_l2(y, ref))


@pytest.mark.parametrize("M,K", [(96, 8192), (33, 4096)])
def test_split_to_packed(cuda, oracle, M, K):
    """cbq_split_to_packed turns the split format back into the reference's
    LSB-first index stream bit for bit, and the module's batched-token path
    on it equals the stream-decode path exactly."""
    import ctypes
    import cbq_native as nat
    import huffman_codebook as hc
    from gpu_huffman_functions import prefill_bits, split_inverse
    from test_gpu_huffman import _lin
    rng = np.random.default_rng(M + K)
    w = cbb.bf16_round(rng.standard_normal((M, K)) * 0.02)
    cb, idx = cbb.frequency_sorted_codebook(w)
    enc = hc.huffman_encode_indices(idx, shape=(M, K))
    lin = _lin(enc, cb, M, K)
    assert lin.split is not None
    bits = prefill_bits(len(cb))
    inv = split_inverse(cb, cuda)
    out = torch.zeros(M * K * bits // 8 + 16, dtype=torch.uint8, device=cuda)
    nat.check(nat.load().cbq_split_to_packed(ctypes.byref(lin.split[1]), inv.data_ptr(), bits,
                                             out.data_ptr(), nat.stream_ptr(cuda)), "s2p")
    want = oracle.pack_lsb(idx.reshape(-1), bits)
    assert np.array_equal(out.cpu().numpy()[:want.size], want)
    x = torch.from_numpy(rng.standard_normal((80, K)).astype(np.float32)).to(cuda)
    lin_stream = _lin(enc, cb, M, K, layout="stream")
    assert torch.equal(lin(x), lin_stream(x))


def test_pack_indices_layout(cuda, oracle):
    """cbq_pack_indices writes the reference's LSB-first stream bit for bit,
    clamping to 2^bits - 1."""
    import cbq_native as nat
    lib = nat.load()
    rng = np.random.default_rng(4)
    for bits in (8, 10, 11, 12, 13):
        idx = rng.integers(-3, (1 << bits) + 50, size=32 * 37).astype(np.int32)
        want = oracle.pack_lsb(np.clip(idx, 0, (1 << bits) - 1), bits)
        d = torch.from_numpy(idx).to(cuda)
        out = torch.zeros(idx.size * bits // 8 + 8, dtype=torch.uint8, device=cuda)
        nat.check(lib.cbq_pack_indices(d.data_ptr(), idx.size, bits, out.data_ptr(),
                                       nat.stream_ptr(cuda)), "cbq_pack_indices")
        got = out.cpu().numpy()[:want.size]
        assert np.array_equal(got, want), bits
