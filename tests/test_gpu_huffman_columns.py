"""Column layout of the Huffman stream (struct cbq_huff_columns) and the
single-token GEMV over it.

The layout is a pure bit copy: every sub-block's bits must appear, LSB-first
from bit 0, in its column, followed by zeros; rows per chunk = the longest
sub-block in words.  The column GEMV must equal the packed-stream GEMV
exactly (same per-lane accumulation order) and the oracle within rel-L2 1e-5,
including chunks too tall for its LDS slot and codes beyond 24 bits.
"""
import numpy as np
import pytest
import torch

import codebook_builder as cbb
import huffman_codebook as hc
from conftest import rel_l2
from test_gpu_huffman import _lin

pytestmark = pytest.mark.gpu
TOL = 1e-5


def _bits(words_u32: np.ndarray) -> np.ndarray:
    return np.unpackbits(words_u32.view(np.uint8), bitorder="little")


def test_columns_hold_sub_block_bits(cuda):
    rng = np.random.default_rng(3)
    M, K = 40, 4096
    w = cbb.bf16_round(rng.standard_normal((M, K)) * 0.02)
    cb, idx = cbb.frequency_sorted_codebook(w)
    enc = hc.huffman_encode_indices(idx, shape=(M, K))
    lin = _lin(enc, cb, M, K, layout="columns")
    assert lin.cols is not None
    stream_bits = _bits(lin.dev.words.cpu().numpy().view(np.uint32))
    cw = lin._cwords.cpu().numpy().view(np.uint32)
    ro = lin._row_off.cpu().numpy().astype(np.int64)
    off = np.asarray(enc["huff_chunk_offsets"], np.int64)
    sub = np.asarray(enc["huff_sub_lens"], np.int64)
    n_chunks = M * K // 4096
    assert ro[0] == 0 and ro.size == n_chunks + 1 and cw.size == (ro[-1] + 4) * 64
    assert not cw[ro[-1] * 64:].any()                                  # zero pad rows
    for c in range(n_chunks):
        lens = sub[c * 64:(c + 1) * 64]
        H = ro[c + 1] - ro[c]
        assert H == max(1, int(((lens + 31) // 32).max()))
        block = cw[ro[c] * 64:(ro[c] + H) * 64].reshape(H, 64)
        starts = off[c] + np.concatenate([[0], np.cumsum(lens)[:-1]])
        for l in range(64):
            col = _bits(np.ascontiguousarray(block[:, l]))
            assert np.array_equal(col[:lens[l]], stream_bits[starts[l]:starts[l] + lens[l]]), (c, l)
            assert not col[lens[l]:].any(), (c, l)


@pytest.mark.parametrize("M,K", [(300, 4096), (70, 12288), (1024, 4096)])
def test_column_gemv_equals_packed(cuda, oracle, M, K):
    rng = np.random.default_rng(M * 7 + K)
    w = cbb.bf16_round(rng.standard_normal((M, K)) * 0.02)
    cb, idx = cbb.frequency_sorted_codebook(w)
    enc = hc.huffman_encode_indices(idx, shape=(M, K))
    lin = _lin(enc, cb, M, K, layout="columns")
    assert lin.cols is not None
    assert lin.cols.ulut1, "unified tables expected for a 24-bit code"
    x = torch.from_numpy(rng.standard_normal((1, K)).astype(np.float32)).to(cuda)
    y_col = lin(x)                                         # unified tables
    u = (lin.cols.ulut1, lin.cols.ulut2, lin.cols.n_ulut2)
    lin.cols.ulut1 = lin.cols.ulut2 = None                 # leaf/pointer tables of the stream
    lin.cols.n_ulut2 = 0
    y_sel = lin(x)
    lin.cols.ulut1, lin.cols.ulut2, lin.cols.n_ulut2 = u
    cols, lin.cols = lin.cols, None
    y_packed = lin(x)                                      # packed-stream tile kernel
    lin.cols = cols
    assert torch.equal(y_col, y_sel) and torch.equal(y_col, y_packed)
    ref = oracle.huff_gemv(x.cpu().numpy(), enc, cb, M, K, chunk_rows=None)
    assert rel_l2(y_col.cpu().numpy(), ref) <= TOL


def test_column_gemv_tall_chunks(cuda, oracle):
    """Uniform 12-bit codes: 768 bits per sub-block = 24 rows per chunk, more
    than the LDS slot holds, so every chunk reads its columns from memory."""
    rng = np.random.default_rng(5)
    M, K = 64, 8192
    idx = rng.integers(0, 4096, size=M * K)
    cb = cbb.bf16_round(rng.standard_normal(4096) * 0.02).astype(np.float32)
    enc = hc.huffman_encode_indices(idx, shape=(M, K))
    assert int(np.asarray(enc["huff_lengths"]).max()) == 12
    lin = _lin(enc, cb, M, K, layout="columns")
    assert lin.cols is not None
    H = np.diff(lin._row_off.cpu().numpy())
    assert (H >= 24).all()
    x = rng.standard_normal((1, K)).astype(np.float32)
    ref = oracle.huff_gemv(x, enc, cb, M, K)
    y = lin(torch.from_numpy(x).to(cuda)).cpu().numpy()    # unified tables
    assert rel_l2(y, ref) <= TOL
    lin.cols.ulut1 = lin.cols.ulut2 = None
    lin.cols.n_ulut2 = 0
    y2 = lin(torch.from_numpy(x).to(cuda)).cpu().numpy()   # stream tables
    assert rel_l2(y2, ref) <= TOL


def test_column_gemv_long_codes(cuda, oracle):
    """Codes up to 30 bits: the lut2 holds unresolved entries, every block
    takes the general path (canonical stage)."""
    rng = np.random.default_rng(11)
    lengths = np.array(list(range(1, 31)) + [30], np.uint8)
    M, K = 24, 4096
    p = 0.5 ** np.minimum(lengths, 12).astype(np.float64)
    idx = rng.choice(31, size=M * K, p=p / p.sum())
    enc = oracle.huffman_encode(idx, shape=(M, K), lengths=lengths)
    cb = cbb.bf16_round(rng.standard_normal(31) * 0.02).astype(np.float32)
    lin = _lin(enc, cb, M, K, layout="columns")
    assert lin.cols is not None and not lin.cols.ulut1     # no unified tables past 24 bits
    x = rng.standard_normal((1, K)).astype(np.float32)
    y = lin(torch.from_numpy(x).to(cuda)).cpu().numpy()
    assert rel_l2(y, oracle.huff_gemv(x, enc, cb, M, K)) <= TOL
