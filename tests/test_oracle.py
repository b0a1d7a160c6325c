"""Pins the CPU oracle (oracle/) before anything is checked against it.

* C restatement == compiled reference C, bitwise, on the golden fixtures
  (tests/golden/gen_golden.py) and on fresh seeded inputs when oracle/_ref
  is built;
* fixed-width GEMV == float64 dense recomputation (tests/test_c_kernel.py:
  42-59 of the reference), chunk-size invariance, determinism, int64 bit
  offsets (tests/test_c_kernel.py:109-138);
* packing: closed form via brute-force bit loops, nibble order KAT
  (tests/test_bitpack.py:50-55);
* Huffman: the hand-derived stream KAT of diagnostics/test_huffman_gpu.py:
  30-35, canonical codes prefix-free + Kraft, heap lengths optimal
  (brute force) and their tie-breaks (hand-derived), LUT / slow tables by
  exhaustive decode of every 12-bit prefix, decoder == bit-serial decoder.
"""
import itertools

import numpy as np
import pytest

from conftest import rel_l2


def _fixed_inputs(case):
    return case["x"], case["packed"], case["cb"], int(case["M"]), int(case["K"]), int(case["bits"])


# ---------------------------------------------------------------------------
# golden fixtures (outputs of the compiled reference C)
# ---------------------------------------------------------------------------

def test_fixed_golden_bitwise(oracle, golden):
    for name, c in golden["fixed"].items():
        x, pk, cb, M, K, bits = _fixed_inputs(c)
        T = x.shape[0]
        y = oracle.fixed_gemv(x, pk, cb, M, K, bits, C=int(c["C"]))
        ys = oracle.fixed_gemv(x, pk, cb, M, K, bits, C=int(c["C"]), chunk_rows=None)
        ref = c["y"] if name != "bf16slice" else c["y_T16"]
        assert np.array_equal(y.view(np.uint32), ref.view(np.uint32)), name
        assert np.array_equal(ys.view(np.uint32), c["y_single"].view(np.uint32)), name
        if name == "bf16slice":
            for t in (1, 4):
                yt = oracle.fixed_gemv(x[:t], pk, cb, M, K, bits)
                assert np.array_equal(yt, c[f"y_T{t}"]), (name, t)
        assert T == int(c["T"])


def test_fixed_golden_unpack_and_embedding(oracle, golden):
    for name, c in golden["fixed"].items():
        n = int(c["M"]) * int(c["K"])
        idx = oracle.unpack_indices_c(c["packed"], int(c["bits"]), n)
        assert np.array_equal(idx, c["raw"].astype(np.int32)), name
        emb = oracle.fixed_embedding(c["ids"], c["packed"], c["cb"], int(c["K"]), int(c["bits"]),
                                     C=int(c["C"]))
        assert np.array_equal(emb, c["emb"]), name


def test_huffman_golden_bitwise(oracle, golden):
    for name, c in golden["huffman"].items():
        M, K = int(c["M"]), int(c["K"])
        enc = {k: c[k] for k in c if k.startswith("huff_")}
        dec = oracle.huff_decode_indices(enc, M, K)
        assert np.array_equal(dec, c["dec"]), name
        assert np.array_equal(dec.reshape(-1), c["idx"].astype(np.int32)), name
        y = oracle.huff_gemv(c["x"], enc, c["cb"], M, K, C=int(c["C"]))
        assert np.array_equal(y.view(np.uint32), c["y"].view(np.uint32)), name
        e = oracle.huff_embedding(c["ids"], enc, c["cb"], K, C=int(c["C"]))
        assert np.array_equal(e, c["emb"]), name


def test_huffman_golden_encoder_reproduces_streams(oracle, golden):
    """Re-encoding each fixture's indices gives its stored stream and tables."""
    for name, c in golden["huffman"].items():
        enc = oracle.huffman_encode(c["idx"], shape=(int(c["M"]), int(c["K"])))
        for k in ("huff_lengths", "huff_stream", "huff_row_bit_starts", "huff_lut_sym",
                  "huff_lut_len", "huff_sl_first_code", "huff_sl_base_offset", "huff_sl_sym"):
            assert np.array_equal(enc[k], c[k]), (name, k)


# ---------------------------------------------------------------------------
# fresh inputs against the compiled reference (this container only)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("M,K,T,bits", [(300, 96, 1, 13), (257, 64, 5, 12), (64, 160, 2, 7),
                                        (40, 64, 16, 14), (128, 128, 3, 8)])
def test_fixed_vs_compiled_reference(oracle, M, K, T, bits):
    if not oracle.ref_available():
        pytest.skip("oracle/_ref not built (reference tree absent)")
    rng = np.random.default_rng(M * 31 + K)
    raw = rng.integers(0, 1 << bits, size=M * K)
    C = max(2, (1 << bits) - 17)
    cb = (rng.standard_normal(C) * 0.02).astype(np.float32)
    x = rng.standard_normal((T, K)).astype(np.float32)
    pk = oracle.pack_lsb(raw, bits)
    a = oracle.fixed_gemv(x, pk, cb, M, K, bits)
    b = oracle.fixed_gemv(x, pk, cb, M, K, bits, kind="ref")
    assert np.array_equal(a, b)


def test_huffman_vs_compiled_reference(oracle):
    if not oracle.ref_available():
        pytest.skip("oracle/_ref not built (reference tree absent)")
    rng = np.random.default_rng(5)
    f = np.ones(2500)
    f[:150] = rng.uniform(500, 20000, 150)
    M, K = 96, 128
    idx = rng.choice(2500, size=M * K, p=f / f.sum())
    enc = oracle.huffman_encode(idx, shape=(M, K))
    assert enc["huff_lengths"].max() > 12
    cb = (rng.standard_normal(2500) * 0.02).astype(np.float32)
    x = rng.standard_normal((3, K)).astype(np.float32)
    assert np.array_equal(oracle.huff_gemv(x, enc, cb, M, K),
                          oracle.huff_gemv(x, enc, cb, M, K, kind="ref"))
    assert np.array_equal(oracle.huff_decode_indices(enc, M, K),
                          oracle.huff_decode_indices(enc, M, K, kind="ref"))


# ---------------------------------------------------------------------------
# closed forms / invariants
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("M,K,T,bits", [(64, 32, 1, 8), (64, 32, 4, 8), (256, 128, 1, 13),
                                        (256, 128, 3, 13), (128, 64, 8, 13)])
def test_fixed_matches_dense(oracle, M, K, T, bits):
    rng = np.random.default_rng(0)
    raw = rng.integers(0, 1 << bits, size=M * K)
    cb = (rng.standard_normal(1 << bits) * 0.02).astype(np.float32)
    x = (rng.standard_normal((T, K)) * 0.1).astype(np.float32)
    y = oracle.fixed_gemv(x, oracle.pack_lsb(raw, bits), cb, M, K, bits)
    dense = x.astype(np.float64) @ cb[raw].reshape(M, K).astype(np.float64).T
    np.testing.assert_allclose(y, dense, atol=1e-5, rtol=1e-4)
    assert rel_l2(y, dense) < 1e-6


def test_fixed_chunk_invariance_and_determinism(oracle):
    rng = np.random.default_rng(3)
    M, K, bits = 300, 64, 13
    raw = rng.integers(0, 1 << bits, size=M * K)
    cb = rng.standard_normal(1 << bits).astype(np.float32)
    x = rng.standard_normal((2, K)).astype(np.float32)
    pk = oracle.pack_lsb(raw, bits)
    outs = [oracle.fixed_gemv(x, pk, cb, M, K, bits, chunk_rows=cr) for cr in (None, 32, 64, 256)]
    for o in outs[1:]:
        assert np.array_equal(o, outs[0])
    assert np.array_equal(oracle.fixed_gemv_serial(x, pk, cb, M, K, bits), outs[0])


def test_fixed_clamps_indices(oracle):
    """Indices >= C read codebook[C-1] (src/compressed_matmul.c:443)."""
    M, K, bits, C = 4, 32, 8, 10
    raw = np.full(M * K, 255)
    cb = np.arange(C, dtype=np.float32)
    x = np.ones((1, K), np.float32)
    y = oracle.fixed_gemv(x, oracle.pack_lsb(raw, bits), cb, M, K, bits, C=C)
    assert np.all(y == K * (C - 1))


def test_fixed_int64_bit_offsets(oracle):
    """Element * bits beyond 2^31 (tests/test_c_kernel.py:109-138)."""
    M, K, bits = 165200, 1, 13
    rng = np.random.default_rng(7)
    raw = rng.integers(0, 1 << bits, size=M * K)
    cb = (rng.standard_normal(1 << bits) * 0.02).astype(np.float32)
    x = rng.standard_normal((1, K)).astype(np.float32)
    y = oracle.fixed_gemv(x, oracle.pack_lsb(raw, bits), cb, M, K, bits, chunk_rows=None)
    np.testing.assert_allclose(y, x @ cb[raw].reshape(M, K).T, atol=1e-5)


def test_pack_closed_form(oracle):
    rng = np.random.default_rng(1)
    for bits in range(1, 17):
        for n in (1, 5, 8, 13, 64, 257):
            vals = rng.integers(0, 1 << bits, size=n)
            pk = oracle.pack_lsb(vals, bits)
            assert pk.size == (n * bits + 7) // 8
            # brute force: bit j of the stream is bit j%8 of byte j//8
            for i, v in enumerate(vals):
                for b in range(bits):
                    j = i * bits + b
                    assert (pk[j // 8] >> (j % 8)) & 1 == (v >> b) & 1
            assert np.array_equal(oracle.unpack_lsb(pk, bits, n), vals)
            assert np.array_equal(oracle.unpack_indices_c(pk, bits, n), vals)


def test_pack_nibble_order_kat(oracle):
    # tests/test_bitpack.py:50-55: 4-bit packing is low nibble first
    assert oracle.pack_lsb([0x2, 0x1, 0x4, 0x3], 4).tolist() == [0x12, 0x34]
    assert oracle.pack_lsb([0xABC], 12).tolist() == [0xBC, 0x0A]


# ---------------------------------------------------------------------------
# Huffman
# ---------------------------------------------------------------------------

def test_huffman_stream_kat(oracle):
    """diagnostics/test_huffman_gpu.py:30-35: freq [4,4,3,5] -> all lengths 2,
    codes 00/01/10/11; rows [3,1,0,3,2,1,0,3] and [0,1,2,3,0,1,2,3] give
    11 01 00 11 | 10 01 00 11 | 00 01 10 11 | 00 01 10 11."""
    idx = [3, 1, 0, 3, 2, 1, 0, 3, 0, 1, 2, 3, 0, 1, 2, 3]
    enc = oracle.huffman_encode(np.array(idx), shape=(2, 8))
    assert enc["huff_lengths"].tolist() == [2, 2, 2, 2]
    assert enc["huff_stream"].tolist() == [0xD3, 0x93, 0x1B, 0x1B, 0, 0, 0, 0]
    assert enc["huff_row_bit_starts"].tolist() == [0, 16]
    assert enc["huff_lut_sym"][0b110100000000] == 3


def test_heap_lengths_tie_breaks(oracle):
    # hand-derived with (freq, id) heap order, merged ids counting up from n
    assert oracle.heap_code_lengths([4, 4, 3, 5]).tolist() == [2, 2, 2, 2]
    # (1,0)+(1,1)->4:2 ; (2,2)+(2,4)->5:4 ; (4,3)+(4,5)->root
    assert oracle.heap_code_lengths([1, 1, 2, 4]).tolist() == [3, 3, 2, 1]
    assert oracle.heap_code_lengths([0, 7, 0]).tolist() == [0, 1, 0]
    assert oracle.heap_code_lengths([0, 0]).tolist() == [0, 0]


def _brute_force_cost(freq):
    """Minimum sum f*L over length vectors with Kraft sum <= 1."""
    act = [f for f in freq if f > 0]
    n = len(act)
    best = None
    for Ls in itertools.product(range(1, n), repeat=n):
        if sum(2.0 ** -L for L in Ls) <= 1.0 + 1e-12:
            c = sum(f * L for f, L in zip(act, Ls))
            best = c if best is None else min(best, c)
    return best


def test_heap_lengths_optimal(oracle):
    rng = np.random.default_rng(11)
    for _ in range(25):
        n = int(rng.integers(2, 7))
        freq = rng.integers(1, 30, size=n)
        L = oracle.heap_code_lengths(freq)
        assert (freq * L).sum() == _brute_force_cost(freq.tolist())
        assert abs(sum(2.0 ** -int(l) for l in L) - 1.0) < 1e-12


def test_canonical_codes_prefix_free(oracle):
    rng = np.random.default_rng(4)
    freq = rng.integers(1, 1000, size=300) ** 2
    L = oracle.heap_code_lengths(freq)
    codes = oracle.canonical_codes(L)
    strs = sorted(format(c, f"0{l}b") for c, l in codes.values())
    for a, b in zip(strs, strs[1:]):
        assert not b.startswith(a)
    # RFC 1951: same length -> consecutive codes in symbol order
    by_len = {}
    for s, (c, l) in sorted(codes.items()):
        by_len.setdefault(l, []).append(c)
    for cs in by_len.values():
        assert cs == list(range(cs[0], cs[0] + len(cs)))


def test_lut_and_slow_tables_exhaustive(oracle):
    """Every 24-bit pattern prefix: table decode == inverse-map decode."""
    rng = np.random.default_rng(8)
    f = np.ones(600)
    f[:40] = rng.uniform(100, 5000, 40)
    idx = rng.choice(600, size=20000, p=f / f.sum())
    enc = oracle.huffman_encode(idx, shape=(20000 // 8, 8)) if 20000 % 8 == 0 else None
    L = enc["huff_lengths"]
    codes = oracle.canonical_codes(L)
    inv = {(c, l): s for s, (c, l) in codes.items()}
    lut_sym, lut_len = enc["huff_lut_sym"], enc["huff_lut_len"]
    for key in range(4096):
        hit = [(inv[(key >> (12 - l), l)], l) for l in range(1, 13) if (key >> (12 - l), l) in inv]
        if hit:
            assert (lut_sym[key], lut_len[key]) == hit[0]
        else:
            assert lut_sym[key] == -1 and lut_len[key] == 0
    first, base, sl = (enc["huff_sl_first_code"], enc["huff_sl_base_offset"], enc["huff_sl_sym"])
    for (c, l), s in inv.items():
        if l > 12:
            assert sl[base[l] + c - first[l]] == s


def test_decoder_matches_bitserial(oracle):
    rng = np.random.default_rng(9)
    for dist in ("zipf", "deep", "two"):
        if dist == "zipf":
            p = 1.0 / np.arange(1, 400) ** 1.5
            idx = rng.choice(399, size=32 * 64, p=p / p.sum())
        elif dist == "deep":
            f = np.ones(1500)
            f[:50] = rng.uniform(1000, 9000, 50)
            idx = rng.choice(1500, size=32 * 64, p=f / f.sum())
        else:
            idx = rng.integers(0, 2, size=32 * 64)
        enc = oracle.huffman_encode(idx, shape=(32, 64))
        dec = oracle.huff_decode_indices(enc, 32, 64).reshape(-1)
        assert np.array_equal(dec, idx)
        bs = oracle.huffman_decode_bitserial(enc["huff_stream"], enc["huff_lengths"], idx.size)
        assert np.array_equal(bs, idx)


def test_huffman_corrupt_guard(oracle):
    """A prefix that matches no code decodes to symbol 0 and advances one bit
    (src/compressed_matmul.c:183-185): single-symbol code '0', stream of 1s."""
    enc = oracle.huffman_encode(np.zeros(64, np.int64), shape=(1, 64))
    assert enc["huff_lengths"].tolist() == [1]
    enc = dict(enc)
    enc["huff_stream"] = np.array([0xFF] * 8 + [0] * 4, np.uint8)
    dec = oracle.huff_decode_indices(enc, 1, 64).reshape(-1)
    assert np.all(dec == 0)
    cb = np.array([2.5], np.float32)
    w = oracle.huff_decode_weights(enc, cb, 1, 64)
    assert np.all(w == 2.5)
