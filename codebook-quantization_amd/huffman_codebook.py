"""Canonical Huffman streams for codebook indices (format producer + device prep).

Stream format of the reference (src/huffman_codebook.py:126-226): canonical
codes (RFC 1951 section 3.2.2: assigned in (length, symbol) order), written
MSB-first into bytes, exactly ceil(bits/8) bytes followed by 4 zero bytes;
alphabet 0..max(idx); per-row start bits `huff_row_bit_starts[r]` = start of
symbol r*K; the 12-bit GPU LUT and slow-path tables keep the reference's
meaning (src/huffman_codebook.py:353-423).

Differences, all additive:
  * code lengths come from package-merge (Larmore & Hirschberg 1990) with a
    length limit (default 24 bits), instead of an unlimited heap;
  * `huff_chunk_offsets` (uint64, bit offset of every 4096th symbol, plus the
    end) and `huff_sub_lens` (uint16, bits used by every 64-symbol
    sub-block) index the stream for chunk-parallel decoding.

The stream is built in the device's native order first (LSB-first words,
each code bit-reversed) and the reference byte stream is that with the bits
of every byte reversed.
"""
from __future__ import annotations

import ctypes
from typing import Dict, Optional, Tuple

import numpy as np

LUT_BITS = 12
LUT_SIZE = 1 << LUT_BITS
CHUNK_SYMBOLS = 4096
SUB_SYMBOLS = 64
DEFAULT_MAX_LEN = 24

REV8 = np.array([int(f"{i:08b}"[::-1], 2) for i in range(256)], np.uint8)


# ---------------------------------------------------------------------------
# Code lengths
# ---------------------------------------------------------------------------

def length_limited_code_lengths(freq, max_len: int = DEFAULT_MAX_LEN) -> np.ndarray:
    """Optimal prefix-code lengths with every length <= max_len.

    Package-merge: level lists Q_L = leaves, Q_j = merge(leaves, pairs(Q_{j+1}));
    the first 2n-2 items of Q_1 are selected, a selected package selects its
    two children one level down, and a leaf's length is the number of levels
    at which it is selected.  Leaves are ordered by (weight, symbol) and win
    ties against packages, which makes the result deterministic.
    """
    freq = np.asarray(freq, dtype=np.int64)
    lengths = np.zeros(len(freq), np.uint8)
    syms = np.nonzero(freq > 0)[0]
    n = len(syms)
    if n == 0:
        return lengths
    if n == 1:
        lengths[syms[0]] = 1
        return lengths
    if (1 << max_len) < n:
        raise ValueError(f"{n} symbols cannot be coded within {max_len} bits")
    order = np.lexsort((syms, freq[syms]))
    w = freq[syms][order]
    leaf_flags = []                      # per level, deepest first
    cur = w
    leaf_flags.append(np.ones(n, bool))
    for _ in range(max_len - 1):
        m = len(cur) // 2
        pk = cur[0:2 * m:2] + cur[1:2 * m:2]
        allw = np.concatenate([w, pk])
        isleaf = np.concatenate([np.ones(n, bool), np.zeros(m, bool)])
        o = np.argsort(allw, kind="stable")
        cur = allw[o]
        leaf_flags.append(isleaf[o])
    depth = np.zeros(n, np.int64)
    take = 2 * n - 2
    for flags in reversed(leaf_flags):   # level 1 .. max_len
        sel = flags[:take]
        a = int(sel.sum())
        depth[:a] += 1
        take = 2 * (take - a)
        if take == 0:
            break
    lengths[syms[order]] = depth.astype(np.uint8)
    return lengths


def canonical_codes(lengths) -> np.ndarray:
    """RFC 1951 section 3.2.2 codes (uint64 per symbol, 0 for unused)."""
    lengths = np.asarray(lengths, np.int64)
    codes = np.zeros(len(lengths), np.uint64)
    if len(lengths) == 0 or lengths.max() == 0:
        return codes
    mx = int(lengths.max())
    count = np.bincount(lengths[lengths > 0], minlength=mx + 1)
    first = np.zeros(mx + 2, np.int64)
    code = 0
    for L in range(1, mx + 1):
        code = (code + int(count[L - 1])) << 1
        first[L] = code
    used = np.nonzero(lengths > 0)[0]
    order = used[np.lexsort((used, lengths[used]))]
    Ls = lengths[order]
    # rank within each length (symbols already in (length, symbol) order)
    starts = np.searchsorted(Ls, Ls, side="left")
    rank = np.arange(len(order)) - starts
    codes[order] = (first[Ls] + rank).astype(np.uint64)
    return codes


def _bitrev(values: np.ndarray, nbits: np.ndarray) -> np.ndarray:
    v = values.astype(np.uint64)
    nb = nbits.astype(np.uint64)
    out = np.zeros_like(v)
    mx = int(nbits.max()) if len(nbits) else 0
    for i in range(mx):
        bit = (v >> np.uint64(i)) & np.uint64(1)
        dest = nb - np.uint64(1) - np.uint64(i)
        ok = np.uint64(i) < nb
        out |= np.where(ok, bit << np.where(ok, dest, np.uint64(0)), np.uint64(0))
    return out


# ---------------------------------------------------------------------------
# Reference-format decode tables (meaning of src/huffman_codebook.py:353-423)
# ---------------------------------------------------------------------------

def build_gpu_lut(lengths) -> Tuple[np.ndarray, np.ndarray]:
    """int32 lut_sym (-1 = no code of <= 12 bits ends in this prefix) and
    int32 lut_len, indexed by the first 12 stream bits (MSB-first)."""
    lengths = np.asarray(lengths, np.int64)
    codes = canonical_codes(lengths)
    lut_sym = np.full(LUT_SIZE, -1, np.int32)
    lut_len = np.zeros(LUT_SIZE, np.int32)
    for s in np.nonzero((lengths > 0) & (lengths <= LUT_BITS))[0]:
        L = int(lengths[s])
        lo = int(codes[s]) << (LUT_BITS - L)
        lut_sym[lo:lo + (1 << (LUT_BITS - L))] = s
        lut_len[lo:lo + (1 << (LUT_BITS - L))] = L
    return lut_sym, lut_len


def build_slow_tables(lengths):
    """int64 first code per length (-1 none), int32 offsets into sl_sym with a
    sentinel at [max+1], int32 symbols of codes > 12 bits in code order."""
    lengths = np.asarray(lengths, np.int64)
    mx = int(lengths.max()) if len(lengths) and lengths.max() > 0 else LUT_BITS
    codes = canonical_codes(lengths)
    first = np.full(mx + 2, -1, np.int64)
    base = np.zeros(mx + 2, np.int32)
    syms = []
    for L in range(LUT_BITS + 1, mx + 1):
        base[L] = len(syms)
        sel = np.nonzero(lengths == L)[0]
        if len(sel):
            sel = sel[np.argsort(codes[sel], kind="stable")]
            first[L] = int(codes[sel[0]])
            syms.extend(sel.tolist())
    base[mx + 1] = len(syms)
    return first, base, np.array(syms if syms else [0], np.int32)


# ---------------------------------------------------------------------------
# Encoder
# ---------------------------------------------------------------------------

def encode_device_words(idx: np.ndarray, lengths: np.ndarray, codes: np.ndarray):
    """Bit starts, total bits and the LSB-first uint64 word stream."""
    L = lengths.astype(np.int64)[idx]
    rev_of = _bitrev(codes, lengths.astype(np.int64))
    rv = rev_of[idx]
    n = len(idx)
    starts = np.zeros(n + 1, np.int64)
    np.cumsum(L, out=starts[1:])
    total = int(starts[-1])
    nwords = total // 64 + 2
    words = np.zeros(nwords, np.uint64)
    if n:
        st = starts[:-1]
        w = st >> 6
        sh = (st & 63).astype(np.uint64)
        lo = rv << sh
        seg = np.nonzero(np.r_[True, w[1:] != w[:-1]])[0]
        words[w[seg]] |= np.bitwise_or.reduceat(lo, seg)
        spill = (st & 63) + L > 64
        if spill.any():
            ws = w[spill] + 1
            hi = rv[spill] >> (np.uint64(64) - sh[spill])
            seg2 = np.nonzero(np.r_[True, ws[1:] != ws[:-1]])[0]
            words[ws[seg2]] |= np.bitwise_or.reduceat(hi, seg2)
    return starts, total, words


def huffman_encode_indices(indices, shape: Optional[tuple] = None,
                           max_len: int = DEFAULT_MAX_LEN,
                           lengths: Optional[np.ndarray] = None) -> Dict[str, np.ndarray]:
    """Encode a flat uint16 index array (the reference's data-dict keys plus
    the chunk / sub-block index).  `lengths` overrides the computed lengths."""
    idx = np.asarray(indices).reshape(-1).astype(np.int64)
    n = idx.size
    C = int(idx.max()) + 1 if n else 1
    if lengths is None:
        lengths = length_limited_code_lengths(np.bincount(idx, minlength=C), max_len)
    lengths = np.asarray(lengths, np.uint8)
    codes = canonical_codes(lengths)
    starts, total, words = encode_device_words(idx, lengths, codes)
    nbytes = (total + 7) // 8
    dev_bytes = words.view(np.uint8)[:nbytes]
    stream = np.concatenate([REV8[dev_bytes], np.zeros(4, np.uint8)])
    out = {
        "huff_lengths": lengths,
        "huff_stream": stream,
        "huff_n": np.array([n], np.int64),
        "huff_chunk_offsets": np.concatenate(
            [starts[:-1][::CHUNK_SYMBOLS], starts[-1:]]).astype(np.uint64),
        "huff_sub_lens": np.diff(np.concatenate(
            [starts[:-1][::SUB_SYMBOLS], starts[-1:]])).astype(np.uint16),
    }
    if shape is not None and len(shape) == 2:
        M, K = int(shape[0]), int(shape[1])
        out["huff_row_bit_starts"] = (starts[:-1][::K].astype(np.int64)
                                      if n and M * K == n else np.zeros(max(M, 1), np.int64))
        out["huff_lut_sym"], out["huff_lut_len"] = build_gpu_lut(lengths)
        (out["huff_sl_first_code"], out["huff_sl_base_offset"],
         out["huff_sl_sym"]) = build_slow_tables(lengths)
    return out


SPLIT_MAX_LEN = 7          # high-byte code limit of the split format


def split_tables(codebook, counts) -> Optional[Tuple[np.ndarray, np.ndarray, np.ndarray]]:
    """Symbol tables of the split device format (cbq_split_matrix,
    include/cbq_hip.h) for a bf16-exact codebook: symbol i stands for the
    value codebook[min(i, C-1)] (the reference's clamp); the high byte of
    its bf16 bits (sign and exponent bits 7..1) gets a canonical code of at
    most SPLIT_MAX_LEN bits from the high-byte histogram implied by `counts`
    (occurrences per symbol), and the low byte (exponent bit 0 and the 7
    mantissa bits) travels raw.  Returns (sym_code uint32: bit-reversed code
    | len << 24, sym_raw uint8: low byte, lut uint32[16384]: the next two
    codes for every 14 stream bits j, as hi1 << 24 | hi2 << 16 | (len1 +
    len2)), or None when a value is not bf16 or more than 128 high bytes
    occur.  Two codes of at most 7 bits always fit in 14 bits."""
    cb = np.ascontiguousarray(codebook, np.float32).reshape(-1)
    bits = cb.view(np.uint32)
    if cb.size == 0 or np.any(bits & 0xFFFF):
        return None
    counts = np.asarray(counts, np.int64).reshape(-1)
    n_sym = max(int(counts.size), int(cb.size))
    b16 = (bits[np.minimum(np.arange(n_sym), cb.size - 1)] >> 16).astype(np.int64)
    hi = b16 >> 8
    raw = (b16 & 0xFF).astype(np.uint8)
    cnt = np.zeros(n_sym, np.int64)
    cnt[:counts.size] = counts
    hcount = np.bincount(hi, weights=cnt, minlength=256).astype(np.int64)
    if np.count_nonzero(hcount) == 0:
        hcount[hi[0]] = 1
    if np.count_nonzero(hcount) > (1 << SPLIT_MAX_LEN):
        return None
    lengths = length_limited_code_lengths(hcount, SPLIT_MAX_LEN)
    rev = _bitrev(canonical_codes(lengths), lengths.astype(np.int64)).astype(np.uint32)
    sym_code = (rev[hi] | (lengths[hi].astype(np.uint32) << 24)).astype(np.uint32)
    one = np.zeros(1 << SPLIT_MAX_LEN, np.int64)          # next 7 bits -> hi << 24 | len
    filled = np.zeros(one.size, bool)
    for h in np.nonzero(lengths)[0]:
        L = int(lengths[h])
        j = int(rev[h]) + (np.arange(1 << (SPLIT_MAX_LEN - L)) << L)
        one[j] = (int(h) << 24) | L
        filled[j] = True
    if not filled.all():                     # incomplete code (one symbol): never read
        one[~filled] = one[filled][0]
    j = np.arange(1 << (2 * SPLIT_MAX_LEN), dtype=np.int64)
    e1 = one[j & 127]
    e2 = one[(j >> (e1 & 0xFF)) & 127]
    pair = (e1 & 0xFF000000) | ((e2 >> 8) & 0x00FF0000) | ((e1 & 0xFF) + (e2 & 0xFF))
    return sym_code, raw, pair.astype(np.uint32)


def device_words_from_stream(stream) -> np.ndarray:
    """Reference MSB-first byte stream -> LSB-first uint32 words, padded with
    >= 2 zero words (the device window reads word d and d + 1)."""
    b = REV8[np.asarray(stream, np.uint8)]
    nw = (b.size + 3) // 4 + 2
    out = np.zeros(nw * 4, np.uint8)
    out[:b.size] = b
    return out.view(np.uint32)


# ---------------------------------------------------------------------------
# Device tables through the C ABI's host builders
# ---------------------------------------------------------------------------

def _native():
    import cbq_native
    return cbq_native.load()


def device_luts(lengths, codebook: Optional[np.ndarray], C: int, value_payload: bool,
                clamp: bool = True):
    """lut1, lut2, canon[100], canon_pay for the chunked decoder."""
    lib = _native()
    lengths = np.ascontiguousarray(lengths, np.uint8)
    cb = None if codebook is None else np.ascontiguousarray(codebook, np.float32)
    n2 = ctypes.c_int(0)
    canon = np.zeros(100, np.int32)
    pay = np.zeros(max(1, int((lengths > 0).sum())), np.int32)
    cb_p = None if cb is None else cb.ctypes.data
    rc = lib.cbq_huff_build_luts(lengths.ctypes.data, len(lengths), cb_p, int(C),
                                 int(value_payload), int(clamp), None, None,
                                 ctypes.byref(n2), canon.ctypes.data, pay.ctypes.data)
    if rc:
        raise ValueError(f"invalid Huffman code lengths (cbq_huff_build_luts rc={rc})")
    lut1 = np.zeros(LUT_SIZE, np.uint32)
    lut2 = np.zeros(n2.value, np.uint32)
    rc = lib.cbq_huff_build_luts(lengths.ctypes.data, len(lengths), cb_p, int(C),
                                 int(value_payload), int(clamp), lut1.ctypes.data,
                                 lut2.ctypes.data, ctypes.byref(n2), canon.ctypes.data,
                                 pay.ctypes.data)
    if rc:
        raise ValueError(f"cbq_huff_build_luts rc={rc}")
    return lut1, lut2, canon, pay


def unified_luts(lengths, codebook: np.ndarray):
    """ulut1[4096], ulut2 for the column GEMV (bf16-value payloads, codes of
    at most 24 bits), or None when the code does not qualify."""
    lib = _native()
    lengths = np.ascontiguousarray(lengths, np.uint8)
    cb = np.ascontiguousarray(codebook, np.float32)
    n2 = ctypes.c_int(0)
    if lib.cbq_huff_build_ulut(lengths.ctypes.data, len(lengths), cb.ctypes.data, int(cb.size),
                               None, None, ctypes.byref(n2)):
        return None
    u1 = np.zeros(LUT_SIZE, np.uint32)
    u2 = np.zeros(n2.value, np.uint32)
    rc = lib.cbq_huff_build_ulut(lengths.ctypes.data, len(lengths), cb.ctypes.data, int(cb.size),
                                 u1.ctypes.data, u2.ctypes.data, ctypes.byref(n2))
    if rc:
        raise ValueError(f"cbq_huff_build_ulut rc={rc}")
    return u1, u2


def index_stream(stream, lengths, M: int, K: int, row_bit_starts=None,
                 threads: int = 0) -> Tuple[np.ndarray, np.ndarray]:
    """chunk offsets and sub-block lengths of a reference-format stream."""
    import os
    lib = _native()
    st = np.ascontiguousarray(stream, np.uint8)
    lengths = np.ascontiguousarray(lengths, np.uint8)
    N = int(M) * int(K)
    chunk = np.zeros((N + CHUNK_SYMBOLS - 1) // CHUNK_SYMBOLS + 1, np.uint64)
    sub = np.zeros((N + SUB_SYMBOLS - 1) // SUB_SYMBOLS, np.uint16)
    rbs = None if row_bit_starts is None else np.ascontiguousarray(row_bit_starts, np.int64)
    nthr = threads or min(16, os.cpu_count() or 1)
    rc = lib.cbq_huff_index_stream(st.ctypes.data, st.size, lengths.ctypes.data, len(lengths),
                                   None if rbs is None else rbs.ctypes.data, int(M), int(K),
                                   chunk.ctypes.data, sub.ctypes.data, nthr)
    if rc:
        raise ValueError("Huffman stream does not match its row starts / code lengths")
    return chunk, sub


def stage_words_for(chunk_offsets) -> int:
    """LDS words a wave needs to stage its largest chunk (rounded to 64)."""
    co = np.asarray(chunk_offsets, np.int64)
    if co.size < 2:
        return 64
    need = ((co[1:] + 31) >> 5) - (co[:-1] >> 5) + 2
    return int(((int(need.max()) + 63) // 64) * 64)
