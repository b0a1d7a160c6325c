"""Writes tests/golden/*.npz: inputs and reference outputs for parity tests.

Outputs come from the reference's own C kernel compiled from
/root/reference/src/compressed_matmul.c (oracle/_ref, built by
`make -C oracle ref`), called through oracle/cbq_oracle.py with the
reference wrapper's conventions.  Inputs are seeded (numpy PCG64) and encoded
with the oracle's format restatements; the reference C decoding them back to
the generating indices is what pins those encoders.

Run from the repo root:  python tests/golden/gen_golden.py
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
import cbq_oracle as O  # noqa: E402

OUT = os.path.dirname(os.path.abspath(__file__))


def bf16_weights(rng, shape, scale=0.02):
    """N(0, scale) rounded to bf16 (round-to-nearest-even), as float32."""
    w = (rng.standard_normal(shape).astype(np.float32) * np.float32(scale))
    u = w.view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return (u.astype(np.uint32) << 16).view(np.float32)


def freq_sorted_codebook(w):
    """Unique values by descending count, ties by ascending bf16 pattern."""
    pat = (w.reshape(-1).view(np.uint32) >> 16).astype(np.int64)
    cnt = np.bincount(pat, minlength=65536)
    present = np.nonzero(cnt)[0]
    order = np.lexsort((present, -cnt[present]))
    sym_pat = present[order]
    lut = np.zeros(65536, np.int64)
    lut[sym_pat] = np.arange(len(sym_pat))
    cb = (sym_pat.astype(np.uint32) << 16).view(np.float32)
    return cb.astype(np.float32), lut[pat].astype(np.uint16)


def fixed_cases(rng):
    cases = {}
    # Shapes of tests/test_c_kernel.py:42-49 plus other widths, clamps and
    # a config-1-like bf16 slice with a frequency-sorted codebook.
    spec = [(64, 32, 1, 8, None), (64, 32, 4, 8, None), (256, 128, 1, 13, None),
            (256, 128, 3, 13, None), (512, 64, 1, 13, None), (128, 64, 8, 13, None),
            (96, 64, 2, 4, None), (80, 96, 1, 7, None), (64, 128, 5, 12, None),
            (48, 64, 2, 16, 6000), (70, 96, 3, 13, 3000), (33, 160, 1, 11, 1500)]
    for i, (M, K, T, bits, C) in enumerate(spec):
        Cfull = 1 << bits
        raw = rng.integers(0, Cfull, size=M * K, dtype=np.uint32)
        Cv = Cfull if C is None else C          # C < 2^b: indices >= C clamp
        cb = (rng.standard_normal(Cv) * 0.02).astype(np.float32)
        x = (rng.standard_normal((T, K)) * 0.1).astype(np.float32)
        packed = O.pack_lsb(raw, bits)
        y = O.fixed_gemv(x, packed, cb, M, K, bits, kind="ref")
        y_single = O.fixed_gemv(x, packed, cb, M, K, bits, kind="ref", chunk_rows=None)
        ids = rng.integers(0, M, size=5).astype(np.int32)
        emb = cb[np.minimum(raw.reshape(M, K)[ids], Cv - 1)]
        cases[f"fixed{i}"] = dict(M=M, K=K, T=T, bits=bits, C=Cv, raw=raw.astype(np.uint16),
                                  packed=packed, cb=cb, x=x, y=y, y_single=y_single,
                                  ids=ids, emb=emb)
    # bf16 lossless slice, 13-bit, frequency-sorted codebook (config 1 style)
    M, K = 16, 2048
    w = bf16_weights(np.random.default_rng(0), (M, K))
    cb, idx = freq_sorted_codebook(w)
    bits = int(np.ceil(np.log2(max(len(cb), 2))))
    packed = O.pack_lsb(idx, bits)
    x = np.random.default_rng(1).standard_normal((16, K)).astype(np.float32)
    d = dict(M=M, K=K, T=16, bits=bits, C=len(cb), raw=idx, packed=packed, cb=cb, x=x,
             ids=np.array([0, M - 1, 7], np.int32), emb=cb[idx.reshape(M, K)[[0, M - 1, 7]]])
    for T in (1, 4, 16):
        d[f"y_T{T}"] = O.fixed_gemv(x[:T], packed, cb, M, K, bits, kind="ref")
    d["y"] = d["y_single"] = d["y_T16"]
    cases["bf16slice"] = d
    return cases


def huff_cases(rng):
    cases = {}

    def add(name, idx, M, K, T, cb=None):
        idx = np.asarray(idx, np.uint16)
        enc = O.huffman_encode(idx, shape=(M, K))
        C = int(idx.max()) + 1
        if cb is None:
            cb = (rng.standard_normal(C) * 0.02).astype(np.float32)
        x = (rng.standard_normal((T, K)) * 0.1).astype(np.float32)
        dec = O.huff_decode_indices(enc, M, K, kind="ref")
        y = O.huff_gemv(x, enc, cb, M, K, kind="ref")
        ids = rng.integers(0, M, size=min(M, 4)).astype(np.int32)
        emb = O.huff_embedding(ids, enc, cb, K, kind="ref")
        cases[name] = dict(M=M, K=K, T=T, C=len(cb), idx=idx, cb=cb, x=x, dec=dec, y=y,
                           ids=ids, emb=emb,
                           **{k: np.asarray(v) for k, v in enc.items()})

    add("kat", [3, 1, 0, 3, 2, 1, 0, 3, 0, 1, 2, 3, 0, 1, 2, 3], 2, 8, 1)
    # Zipf-1.5 skew (tests/test_compressed_roundtrip.py:261-279)
    p = 1.0 / np.arange(1, 1025) ** 1.5
    add("zipf", rng.choice(1024, size=64 * 64, p=p / p.sum()), 64, 64, 2)
    add("single", np.zeros(256, np.uint16), 4, 64, 1)
    add("two", rng.integers(0, 2, size=512), 8, 64, 3)
    # deep codes > 12 bits: slow path (tests/test_compressed_roundtrip.py:374-410)
    f = np.ones(3000)
    f[:200] = rng.uniform(500, 10000, 200)
    add("deep", rng.choice(3000, size=128 * 256, p=f / f.sum()), 128, 256, 1)
    # codebook shorter than the alphabet: decoded symbols >= C clamp to C-1
    idx = rng.integers(0, 300, size=32 * 64)
    add("clamp", idx, 32, 64, 2, cb=(rng.standard_normal(200) * 0.02).astype(np.float32))
    # bf16 N(0, 0.02) weights, frequency-sorted lossless codebook
    w = bf16_weights(np.random.default_rng(0), (64, 512))
    cb, idx = freq_sorted_codebook(w)
    add("bf16", idx, 64, 512, 1, cb=cb)
    return cases


def main():
    if not O.ref_available():
        O.build(ref=True)
    rng = np.random.default_rng(20251201)
    for name, cases in (("fixed_golden.npz", fixed_cases(rng)),
                        ("huffman_golden.npz", huff_cases(rng))):
        flat = {}
        for case, d in cases.items():
            for k, v in d.items():
                flat[f"{case}/{k}"] = np.asarray(v)
        np.savez_compressed(os.path.join(OUT, name), **flat)
        print(name, len(cases), "cases",
              os.path.getsize(os.path.join(OUT, name)) // 1024, "KiB")


if __name__ == "__main__":
    main()
