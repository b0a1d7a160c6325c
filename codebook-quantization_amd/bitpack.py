"""Fixed-width index streams (format producer).

Layout of the reference (src/bitpack.py:32-157): index i of a b-bit stream
occupies stream bits [i*b, (i+1)*b), stream bit j being bit j%8 of byte j//8;
the stored array is exactly ceil(N*b/8) bytes (8-bit = one byte per index,
4-bit = low nibble first, 16-bit = little-endian uint16 are all this same
layout).  Implemented here with 64-bit word scatter, not the reference's LCM
grouping.
"""
from __future__ import annotations

import numpy as np


def calculate_packed_size(num_indices: int, bits: int) -> int:
    return (int(num_indices) * int(bits) + 7) // 8


def pack_any_bits(indices, bits: int) -> np.ndarray:
    """Pack indices (< 2**bits, 1 <= bits <= 16) LSB-first into bytes."""
    idx = np.asarray(indices).reshape(-1).astype(np.uint64)
    if not 1 <= bits <= 16:
        raise ValueError(f"bits must be in [1, 16], got {bits}")
    n = idx.size
    nbytes = calculate_packed_size(n, bits)
    if n == 0:
        return np.zeros(0, np.uint8)
    idx &= np.uint64((1 << bits) - 1)
    pos = np.arange(n, dtype=np.uint64) * np.uint64(bits)
    word = (pos >> np.uint64(6)).astype(np.int64)
    sh = pos & np.uint64(63)
    nwords = (n * bits + 63) // 64 + 1
    out = np.zeros(nwords, np.uint64)
    # low part: bits that land in word `word`
    np.bitwise_or.at(out, word, idx << sh)
    # high part: bits that spill into word+1 (sh + bits > 64)
    spill = sh + np.uint64(bits) > np.uint64(64)
    if spill.any():
        np.bitwise_or.at(out, word[spill] + 1, idx[spill] >> (np.uint64(64) - sh[spill]))
    return out.view(np.uint8)[:nbytes].copy()


def unpack_any_bits(packed, bits: int, original_len: int) -> np.ndarray:
    """Inverse of pack_any_bits -> uint16[original_len]."""
    n = int(original_len)
    pk = np.asarray(packed, np.uint8).reshape(-1)
    need = (n * bits + 63) // 64 * 8 + 8
    buf = np.zeros(need, np.uint8)
    m = min(pk.size, need)
    buf[:m] = pk[:m]
    words = buf.view(np.uint64)
    pos = np.arange(n, dtype=np.uint64) * np.uint64(bits)
    w = (pos >> np.uint64(6)).astype(np.int64)
    sh = pos & np.uint64(63)
    lo = words[w] >> sh
    hi_sh = (np.uint64(64) - sh) & np.uint64(63)
    hi = np.where(sh > 0, words[w + 1] << hi_sh, np.uint64(0))
    return ((lo | hi) & np.uint64((1 << bits) - 1)).astype(np.uint16)


def device_padded(packed: np.ndarray, pad: int = 16) -> np.ndarray:
    """Packed bytes + zero padding up to a multiple of 16 plus `pad` bytes:
    the device kernels read whole 32-bit words (wide loads) and need >= 4
    readable bytes past the last index (src/gpu_accelerated_functions.py:860-864)."""
    pk = np.asarray(packed, np.uint8).reshape(-1)
    total = ((pk.size + 15) // 16) * 16 + pad
    out = np.zeros(total, np.uint8)
    out[:pk.size] = pk
    return out
