"""Unified decode tables (cbq_huff_build_ulut), host only: decoding a stream
with them - window -> ulut1 -> ulut2[base + next nb bits], the column GEMV's
step written in numpy - must give every symbol's codebook value and code
length, for skewed and flat codes up to 24 bits; codes beyond 24 bits are
refused."""
import numpy as np
import pytest

import codebook_builder as cbb
import huffman_codebook as hc


def _decode_with_ulut(enc, u1, u2, n):
    words = hc.device_words_from_stream(enc["huff_stream"]).astype(np.uint64)
    vals = np.empty(n, np.uint32)
    lens = np.empty(n, np.int64)
    pos = 0
    for i in range(n):
        d, s = pos >> 5, pos & 31
        win = int(((words[d + 1] << np.uint64(32)) | words[d]) >> np.uint64(s)) & 0xFFFFFFFF
        e1 = int(u1[win & 4095])
        nb = e1 & 15
        ext = (win >> 12) & ((1 << nb) - 1)
        e = int(u2[(e1 >> 18) + ext])
        vals[i] = e >> 16
        lens[i] = e & 63
        pos += e & 63
    return vals, lens


@pytest.mark.parametrize("case", ["gauss", "flat", "deep"])
def test_unified_tables_decode(case):
    rng = np.random.default_rng({"gauss": 1, "flat": 2, "deep": 3}[case])
    if case == "gauss":
        w = cbb.bf16_round(rng.standard_normal(20000) * 0.02)
        cb, idx = cbb.frequency_sorted_codebook(w)
        lengths = None
    elif case == "flat":
        idx = rng.integers(0, 4096, 6000)
        cb = cbb.bf16_round(rng.standard_normal(4096) * 0.02).astype(np.float32)
        lengths = None
    else:                                   # lengths 1..24: a maximal-depth code
        lengths = np.array(list(range(1, 25)) + [24], np.uint8)
        p = 0.5 ** np.minimum(lengths, 14).astype(np.float64)
        idx = rng.choice(25, size=6000, p=p / p.sum())
        cb = cbb.bf16_round(rng.standard_normal(25) * 0.02).astype(np.float32)
    enc = hc.huffman_encode_indices(idx, lengths=lengths)
    L = np.asarray(enc["huff_lengths"], np.uint8)
    u = hc.unified_luts(L, cb)
    assert u is not None
    u1, u2 = u
    n_short = int(((L > 0) & (L <= 12)).sum())
    assert u2.size >= 1 + n_short
    vals, lens = _decode_with_ulut(enc, u1, u2, idx.size)
    want = (np.asarray(cb, np.float32)[np.minimum(idx, cb.size - 1)].view(np.uint32) >> 16)
    assert np.array_equal(vals, want.astype(np.uint32))
    assert np.array_equal(lens, L[idx].astype(np.int64))


def test_unified_tables_refuse_long_codes():
    lengths = np.array(list(range(1, 31)) + [30], np.uint8)
    cb = np.zeros(31, np.float32)
    assert hc.unified_luts(lengths, cb) is None
