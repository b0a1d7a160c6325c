"""Writes tests/golden/heap_golden.npz: Huffman code lengths and encoded
streams produced by the reference's own Python encoder.

The reference's heap tie-breaking (`_build_code_lengths`,
src/huffman_codebook.py:42-86) and its stream layout
(`huffman_encode_indices`, src/huffman_codebook.py:126-226) are not fixed by
any closed form or by the reference C (which only decodes), so this script
imports that one module, straight from its file (it needs only heapq and
numpy), and records its outputs on seeded inputs.  The fixture holds data
only: inputs and the outputs the reference returned.

Run from the repo root (in a tree that has /root/reference):
    python tests/golden/gen_heap_golden.py
"""
import importlib.util
import os

import numpy as np

OUT = os.path.dirname(os.path.abspath(__file__))
REF = "/root/reference/src/huffman_codebook.py"


def load_reference():
    spec = importlib.util.spec_from_file_location("ref_huffman_codebook", REF)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def bf16_freq_sorted(rng, n, scale=0.02):
    """Indices of n N(0, scale) bf16 weights under a codebook sorted by
    descending count (ties by ascending bit pattern), as the reference's
    lossless codebook builder orders it."""
    w = rng.standard_normal(n).astype(np.float32) * np.float32(scale)
    u = w.view(np.uint32).astype(np.uint64)
    pat = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.int64)
    cnt = np.bincount(pat, minlength=65536)
    present = np.nonzero(cnt)[0]
    order = np.lexsort((present, -cnt[present]))
    lut = np.zeros(65536, np.int64)
    lut[present[order]] = np.arange(len(present))
    return lut[pat].astype(np.uint16)


def main():
    ref = load_reference()
    rng = np.random.default_rng(11)
    out = {}
    # -- code lengths ---------------------------------------------------------
    freqs = []
    idx_big = bf16_freq_sorted(rng, 1 << 17)
    freqs.append(np.bincount(idx_big).astype(np.int64))          # ~3000 symbols, long tied tail
    w = rng.standard_normal(1 << 15).astype(np.float32) * np.float32(0.05)
    pat = (w.view(np.uint32) >> 16).astype(np.int64)
    f = np.bincount(pat, minlength=65536)
    freqs.append(f[np.nonzero(f)[0]].astype(np.int64))           # unsorted: ties in bit order
    for k in range(40):                                          # small alphabets, many ties / zeros
        n = int(rng.integers(2, 48))
        freqs.append(rng.integers(0, 1 + k % 6, n).astype(np.int64))
    fib = [1, 1]
    while len(fib) < 40:
        fib.append(fib[-1] + fib[-2])
    freqs.append(np.array(fib[::-1], np.int64))                  # depth 39: the 32 cap binds
    freqs.append(np.array([0, 0, 7, 0], np.int64))                # one active symbol
    freqs.append(np.zeros(5, np.int64))                           # none active
    freqs.append(np.array([3, 3], np.int64))
    freqs.append(np.full(37, 4, np.int64))                        # all tied
    for i, f in enumerate(freqs):
        out[f"freq_{i}"] = f
        out[f"lengths_{i}"] = np.asarray(ref._build_code_lengths(f), np.uint8)
    out["n_freq"] = np.array([len(freqs)], np.int64)
    # -- encoded streams -------------------------------------------------------
    cases = [
        (bf16_freq_sorted(rng, 48 * 256).reshape(48, 256), (48, 256)),
        (rng.integers(0, 9, 300).astype(np.uint16).reshape(1, 300), (1, 300)),
        (np.zeros((4, 16), np.uint16), (4, 16)),                 # single symbol
        (rng.integers(0, 3000, 40).astype(np.uint16).reshape(5, 8), (5, 8)),   # sparse alphabet
    ]
    for i, (idx, shape) in enumerate(cases):
        enc = ref.huffman_encode_indices(idx, shape=shape)
        out[f"enc_{i}_idx"] = idx
        out[f"enc_{i}_shape"] = np.array(shape, np.int64)
        for k, v in enc.items():
            out[f"enc_{i}_{k}"] = np.asarray(v)
    out["n_enc"] = np.array([len(cases)], np.int64)
    path = os.path.join(OUT, "heap_golden.npz")
    np.savez_compressed(path, **out)
    print("wrote", path, os.path.getsize(path), "bytes,", len(freqs), "length cases,",
          len(cases), "streams")


if __name__ == "__main__":
    main()
