"""The reference's functional API (src/compressed_matmul_cpu.py) on the GPU:
compressed_matmul, huffman_matmul, huffman_embedding, huffman_decode_weights
against the oracle's restatements on the same inputs (rel-L2 <= 1e-5 for
products; gathers and decoded weights exact), with C below the codebook size
(clamped indices) and leading batch dimensions."""
import numpy as np
import pytest
import torch

import codebook_builder as cbb
import compressed_matmul_gpu as cmg
from conftest import rel_l2

pytestmark = pytest.mark.gpu


def _huff_data(enc):
    return {"huff_stream": enc["huff_stream"],
            "lut_sym": np.asarray(enc["huff_lut_sym"]).astype(np.uint16),
            "lut_len": np.asarray(enc["huff_lut_len"]).astype(np.uint8),
            "sl_first_code": np.asarray(enc["huff_sl_first_code"], np.int64),
            "sl_base_offset": np.asarray(enc["huff_sl_base_offset"], np.int32),
            "sl_sym": np.asarray(enc["huff_sl_sym"]).astype(np.uint16),
            "row_bit_starts": np.asarray(enc["huff_row_bit_starts"], np.int64),
            "sl_max_len": int(np.asarray(enc["huff_lengths"]).max())}


@pytest.mark.parametrize("T,C_cut", [(1, None), (3, None), (2, 900)])
def test_compressed_matmul(cuda, oracle, T, C_cut):
    rng = np.random.default_rng(T)
    M, K = 300, 2048
    w = cbb.bf16_round(rng.standard_normal((M, K)) * 0.02)
    d = cbb.compress_fixed(w)
    x = rng.standard_normal((T, K)).astype(np.float32)
    y = cmg.compressed_matmul(x, d["indices"], d["codebook"], M, K, d["bits"], C=C_cut)
    ref = oracle.fixed_gemv(x, d["indices"], d["codebook"], M, K, d["bits"], C=C_cut,
                            chunk_rows=None)
    assert y.shape == (T, M) and y.dtype == np.float32
    assert rel_l2(y, ref) <= 1e-5
    y3 = cmg.compressed_matmul(torch.from_numpy(x.reshape(1, T, K)), d["indices"],
                               torch.from_numpy(d["codebook"]), M, K, d["bits"], C=C_cut)
    assert y3.shape == (1, T, M) and np.array_equal(y3[0], y)


@pytest.mark.parametrize("C_cut", [None, 1000])
def test_huffman_functions(cuda, oracle, C_cut):
    rng = np.random.default_rng(11)
    M, K = 96, 4096
    w = cbb.bf16_round(rng.standard_normal((M, K)) * 0.02)
    cb, idx = cbb.frequency_sorted_codebook(w)
    enc = oracle.huffman_encode(idx.reshape(-1), shape=(M, K))
    hd = _huff_data(enc)
    for T in (1, 4):
        x = rng.standard_normal((T, K)).astype(np.float32)
        y = cmg.huffman_matmul(x, hd, cb, M, K, C=C_cut)
        ref = oracle.huff_gemv(x, enc, cb, M, K, C=C_cut)
        assert rel_l2(y, ref) <= 1e-5, T
    ids = np.array([0, 5, M - 1, 17, 5])
    e = cmg.huffman_embedding(ids, hd, cb, K, C=C_cut)
    assert np.array_equal(e, oracle.huff_embedding(ids, enc, cb, K, C=C_cut))
    wd = cmg.huffman_decode_weights(hd, cb, M, K, C=C_cut)
    assert np.array_equal(wd, oracle.huff_decode_weights(enc, cb, M, K, C=C_cut))
    if C_cut is None:
        assert np.array_equal(wd, w)


@pytest.mark.parametrize("M,K", [(16, 32), (7, 100), (40, 1536)])
def test_huffman_functions_any_k(cuda, oracle, M, K):
    """Shapes whose rows are not whole 64-symbol sub-blocks (the reference
    decodes a 16 x 32 tensor in tests/test_compressed_roundtrip.py:747-756):
    the flat stream is decoded to transient indices, then gathered (decode,
    embedding) or multiplied by ck_linear_f32's kernels."""
    rng = np.random.default_rng(M * K)
    w = cbb.bf16_round(rng.standard_normal((M, K)) * 0.02)
    cb, idx = cbb.frequency_sorted_codebook(w)
    enc = oracle.huffman_encode(idx.reshape(-1), shape=(M, K))
    hd = _huff_data(enc)
    wd = cmg.huffman_decode_weights(hd, cb, M, K)
    assert np.array_equal(wd, w)
    assert np.array_equal(wd, oracle.huff_decode_weights(enc, cb, M, K))
    for T in (1, 5):
        x = rng.standard_normal((T, K)).astype(np.float32)
        y = cmg.huffman_matmul(x, hd, cb, M, K)
        assert rel_l2(y, oracle.huff_gemv(x, enc, cb, M, K)) <= 1e-5, T
    ids = np.array([M - 1, 0, 3 % M])
    assert np.array_equal(cmg.huffman_embedding(ids, hd, cb, K), w[ids])


def test_functional_reuses_device_format(cuda):
    """Repeated calls on the same Huffman data reuse one device format."""
    rng = np.random.default_rng(2)
    M, K = 64, 4096
    w = cbb.bf16_round(rng.standard_normal((M, K)) * 0.02)
    cb, idx = cbb.frequency_sorted_codebook(w)
    import huffman_codebook as hc
    hd = _huff_data(hc.huffman_encode_indices(idx, shape=(M, K)))
    a = cmg._huff_linear(hd, cb, M, K)
    assert cmg._huff_linear(dict(hd), cb.copy(), M, K) is a
    cb2 = cb.copy()
    cb2[0] = 0.5
    assert cmg._huff_linear(hd, cb2, M, K) is not a
