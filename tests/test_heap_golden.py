"""The oracle's heap code lengths and stream encoder, and the package's
encoder given the same lengths, reproduce the reference's own Python
encoder (src/huffman_codebook.py:42-86, 126-226) on the fixtures written by
tests/golden/gen_heap_golden.py: tie-broken lengths on large alphabets, the
32-bit cap, single-symbol and empty alphabets, stream bytes, row starts and
the GPU tables."""
import os
import sys

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
sys.path.insert(0, os.path.join(ROOT, "oracle"))
import cbq_oracle as O  # noqa: E402
import huffman_codebook as H  # noqa: E402

G = np.load(os.path.join(HERE, "golden", "heap_golden.npz"))
N_FREQ = int(G["n_freq"][0])
N_ENC = int(G["n_enc"][0])
KEYS = ("huff_lengths", "huff_stream", "huff_n", "huff_row_bit_starts", "huff_lut_sym",
        "huff_lut_len", "huff_sl_first_code", "huff_sl_base_offset", "huff_sl_sym")


@pytest.mark.parametrize("i", range(N_FREQ))
def test_heap_lengths_match_reference(i):
    assert np.array_equal(O.heap_code_lengths(G[f"freq_{i}"]), G[f"lengths_{i}"]), i


def test_fixture_covers_ties_and_cap():
    big = G["lengths_0"]
    assert big.size > 1000 and np.unique(G["freq_0"]).size < big.size / 2   # long tied tail
    assert int(max(G[f"lengths_{i}"].max(initial=0) for i in range(N_FREQ))) == 32


@pytest.mark.parametrize("i", range(N_ENC))
def test_oracle_encoder_matches_reference(i):
    idx, shape = G[f"enc_{i}_idx"], tuple(int(s) for s in G[f"enc_{i}_shape"])
    enc = O.huffman_encode(idx, shape=shape)
    for k in KEYS:
        assert np.array_equal(np.asarray(enc[k]), G[f"enc_{i}_{k}"]), (i, k)


@pytest.mark.parametrize("i", range(N_ENC))
def test_package_encoder_matches_reference_given_lengths(i):
    idx, shape = G[f"enc_{i}_idx"], tuple(int(s) for s in G[f"enc_{i}_shape"])
    enc = H.huffman_encode_indices(idx, shape=shape, lengths=G[f"enc_{i}_huff_lengths"])
    for k in KEYS:
        assert np.array_equal(np.asarray(enc[k]), G[f"enc_{i}_{k}"]), (i, k)
