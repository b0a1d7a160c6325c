"""Code lengths read back from the reference's Huffman decode tables
(compressed_matmul_gpu.lengths_from_tables), CPU only: the tables of the
oracle's restated encoder (heap lengths, codes past 12 bits included), in the
GPU dtypes and in the CPU coercion of src/compressed_modules.py:240-249."""
import numpy as np
import pytest

import compressed_matmul_gpu as cmg


def _huff_data(enc, cpu_coerced):
    lut_sym = np.asarray(enc["huff_lut_sym"])
    lut_len = np.asarray(enc["huff_lut_len"])
    if cpu_coerced:
        lut_sym, lut_len = lut_sym.astype(np.uint16), lut_len.astype(np.uint8)
    return {"huff_stream": enc["huff_stream"], "lut_sym": lut_sym, "lut_len": lut_len,
            "sl_first_code": np.asarray(enc["huff_sl_first_code"], np.int64),
            "sl_base_offset": np.asarray(enc["huff_sl_base_offset"], np.int32),
            "sl_sym": np.asarray(enc["huff_sl_sym"]).astype(np.uint16),
            "row_bit_starts": enc["huff_row_bit_starts"], "sl_max_len": 1}


@pytest.mark.parametrize("cpu_coerced", [False, True])
@pytest.mark.parametrize("case", ["geometric", "flat", "two", "bf16"])
def test_lengths_from_tables(oracle, case, cpu_coerced):
    rng = np.random.default_rng(7)
    if case == "geometric":                      # codes well past 12 bits
        p = 0.5 ** np.arange(30)
        idx = rng.choice(30, size=20000, p=p / p.sum())
        idx[:30] = np.arange(30)                 # every symbol present
    elif case == "flat":
        idx = rng.integers(0, 700, size=20000)
    elif case == "two":
        idx = rng.integers(0, 2, size=640)
    else:
        import codebook_builder as cbb
        w = cbb.bf16_round(rng.standard_normal(64 * 512) * 0.02)
        _, idx = cbb.frequency_sorted_codebook(w)
    K = 64
    M = len(idx) // K
    idx = idx[:M * K]
    enc = oracle.huffman_encode(idx, shape=(M, K))
    want = np.asarray(enc["huff_lengths"], np.uint8)
    if case == "geometric":
        assert want.max() > 12
    got = cmg.lengths_from_tables(_huff_data(enc, cpu_coerced), len(want))
    assert np.array_equal(got, want)
