"""Canonical-Huffman compressed linear / embedding on gfx950 (drop-in backends).

Same classes and constructor signatures as the reference
(src/gpu_huffman_functions.py:715-1002):

    HuffmanCodebookLinear(name, huff_stream, huff_lengths, huff_n, codebook,
                          shape, bits, huff_row_bit_starts=..., huff_lut_sym=...,
                          huff_lut_len=..., huff_sl_first_code=...,
                          huff_sl_base_offset=..., huff_sl_sym=...)

plus two optional keys written by this package's encoder,
`huff_chunk_offsets` and `huff_sub_lens`.  Where the reference decodes every
row into a transient int32 [M*K] buffer and then runs a GEMV (and decodes the
whole vocabulary for each embedding call), this backend keeps one compressed
format per matrix in HBM and decodes it chunk-parallel straight into the dot
product (one token) or into the requested embedding rows.

At construction the reference stream is turned into the device format: bytes
bit-reversed into LSB-first words, decode tables rebuilt from `huff_lengths`
(the reference's huff_lut_* / huff_sl_* arrays are derived from the same
lengths and are not needed), and - when the chunk index is absent - one host
pass over the stream (split at `huff_row_bit_starts`) computes it.  A linear
whose codebook allows it is then re-encoded on the device into the split
format and the stream is freed (HuffmanCodebookLinear's `layout`).
"""
from __future__ import annotations

import ctypes
import math
from typing import Optional, Tuple

import numpy as np
import torch

import cbq_native as nat
import cbq_ops
import huffman_codebook as hc

_BF16_PAYLOAD_MAX_C = 1 << 16
_SYMBOL_PAYLOAD_MAX_C = 16384     # fp32 codebook staged in LDS


def _is_bf16_exact(cb: np.ndarray) -> bool:
    return bool(np.all((cb.view(np.uint32) & 0xFFFF) == 0))


class _DeviceStream:
    """Device-resident chunked stream + decode tables for one tensor."""

    def __init__(self, name, huff_stream, huff_lengths, huff_n, codebook_f32: np.ndarray,
                 shape: Tuple[int, int], row_bit_starts=None, chunk_offsets=None,
                 sub_lens=None, device=None, raw_symbols=False):
        self.name = name
        M, K = shape
        n = int(huff_n)
        if n != M * K:
            raise ValueError(f"{name}: huff_n={n} != {M}x{K}")
        lengths = np.ascontiguousarray(huff_lengths, np.uint8)
        stream = np.ascontiguousarray(huff_stream, np.uint8)
        if chunk_offsets is None or sub_lens is None:
            chunk_offsets, sub_lens = hc.index_stream(stream, lengths, M, K, row_bit_starts)
        chunk_offsets = np.ascontiguousarray(chunk_offsets, np.uint64)
        sub_lens = np.ascontiguousarray(sub_lens, np.uint16)
        if chunk_offsets.size != (n + hc.CHUNK_SYMBOLS - 1) // hc.CHUNK_SYMBOLS + 1 or \
                sub_lens.size != (n + hc.SUB_SYMBOLS - 1) // hc.SUB_SYMBOLS:
            raise ValueError(f"{name}: chunk index does not match {n} symbols")
        if int(chunk_offsets[-1]) > 8 * stream.size:
            raise ValueError(f"{name}: chunk index points past the stream")
        self.C = int(codebook_f32.size)
        self.value_payload = (not raw_symbols) and _is_bf16_exact(codebook_f32) and self.C > 0
        if not self.value_payload and not raw_symbols and self.C > _SYMBOL_PAYLOAD_MAX_C:
            raise ValueError(f"{name}: non-bf16 codebook with {self.C} > "
                             f"{_SYMBOL_PAYLOAD_MAX_C} entries is not supported")
        lut1, lut2, canon, pay = hc.device_luts(lengths, codebook_f32 if self.C else None,
                                                self.C, self.value_payload,
                                                clamp=not raw_symbols)
        words = hc.device_words_from_stream(stream)
        dev = device or torch.device("cuda")
        self.words = torch.from_numpy(words.view(np.int32)).to(dev)
        self.chunk_off = torch.from_numpy(chunk_offsets.view(np.int64)).to(dev)
        self.sub_len = torch.from_numpy(sub_lens.view(np.int16)).to(dev)
        self.lut1 = torch.from_numpy(lut1.view(np.int32)).to(dev)
        self.lut2 = torch.from_numpy(lut2.view(np.int32)).to(dev)
        self.canon = torch.from_numpy(canon).to(dev)
        self.canon_pay = torch.from_numpy(pay).to(dev)
        self.value_cb = (None if (self.value_payload or raw_symbols)
                         else torch.from_numpy(np.ascontiguousarray(codebook_f32)).to(dev))
        self.stream_bytes = int(stream.size)
        self.table_bytes = int(chunk_offsets.nbytes + sub_lens.nbytes)
        self.desc = nat.HuffStream(
            words=self.words.data_ptr(), n_words=int(self.words.numel()),
            chunk_off=self.chunk_off.data_ptr(), sub_len=self.sub_len.data_ptr(),
            lut1=self.lut1.data_ptr(), lut2=self.lut2.data_ptr(), n_lut2=int(lut2.size),
            canon=self.canon.data_ptr(), canon_pay=self.canon_pay.data_ptr(),
            value_cb=None if self.value_cb is None else self.value_cb.data_ptr(),
            C=self.C, stage_words=hc.stage_words_for(chunk_offsets))

    def op_args(self):
        """The stream's tensors and sizes in torch.ops.cbq.huff_* argument order."""
        return (self.words, self.chunk_off, self.sub_len, self.lut1, self.lut2, self.canon,
                self.canon_pay, self.value_cb, self.C, int(self.desc.stage_words))


def stream_from_device(t) -> _DeviceStream:
    """_DeviceStream over a device_formats.HuffTensor's device arrays (the
    stream and chunk index already in HBM, e.g. loaded from a device image):
    no host stream, no host indexing."""
    tb = t.tables
    d = _DeviceStream.__new__(_DeviceStream)
    d.name = t.name
    d.C = int(tb["codebook"].numel())
    d.value_payload = True
    d.words, d.chunk_off, d.sub_len = t.words, t.chunk_off, t.sub_len
    d.lut1, d.lut2, d.canon, d.canon_pay = tb["lut1"], tb["lut2"], tb["canon"], tb["pay"]
    d.value_cb = None
    d.stream_bytes = (int(t.total_bits) + 7) // 8
    d.table_bytes = int(t.chunk_off.numel() * 8 + t.sub_len.numel() * 2)
    d.desc = nat.HuffStream(
        words=d.words.data_ptr(), n_words=int(d.words.numel()), chunk_off=d.chunk_off.data_ptr(),
        sub_len=d.sub_len.data_ptr(), lut1=d.lut1.data_ptr(), lut2=d.lut2.data_ptr(),
        n_lut2=int(d.lut2.numel()), canon=d.canon.data_ptr(), canon_pay=d.canon_pay.data_ptr(),
        value_cb=None, C=d.C, stage_words=int(tb["stage_words"]))
    return d


def build_columns(desc: "nat.HuffStream", n_sym: int, device, lengths=None,
                  codebook: Optional[np.ndarray] = None):
    """Column layout of a device stream (struct cbq_huff_columns): chunk c's
    64 sub-blocks side by side, built on the device; with the code lengths
    and the (bf16-exact) codebook also the unified decode tables when the
    code qualifies.  Returns the device tensors to keep alive and the
    descriptor."""
    lib = nat.load()
    n_chunks = (n_sym + hc.CHUNK_SYMBOLS - 1) // hc.CHUNK_SYMBOLS
    st = nat.stream_ptr(device)
    rows = torch.empty(n_chunks, dtype=torch.int32, device=device)
    nat.check(lib.cbq_huff_column_rows(ctypes.byref(desc), n_sym, rows.data_ptr(), st),
              "cbq_huff_column_rows")
    cum = torch.cumsum(rows.to(torch.int64), 0)
    total = int(cum[-1])
    if total + 4 >= 2 ** 31:
        raise ValueError(f"column layout of {total} rows exceeds the 32-bit row index")
    row_off = torch.zeros(n_chunks + 1, dtype=torch.int32, device=device)
    row_off[1:] = cum.to(torch.int32)
    cwords = torch.zeros((total + 4) * hc.SUB_SYMBOLS, dtype=torch.int32, device=device)
    nat.check(lib.cbq_huff_columnize(ctypes.byref(desc), n_sym, row_off.data_ptr(),
                                     cwords.data_ptr(), st), "cbq_huff_columnize")
    keep = [cwords, row_off]
    cols = nat.HuffColumns(cwords=cwords.data_ptr(), row_off=row_off.data_ptr(), n_chunks=n_chunks)
    if lengths is not None and codebook is not None:
        u = hc.unified_luts(lengths, codebook)
        if u is not None and u[1].size <= 8192:
            u1 = torch.from_numpy(u[0].view(np.int32)).to(device)
            u2 = torch.from_numpy(u[1].view(np.int32)).to(device)
            keep += [u1, u2]
            cols.ulut1, cols.ulut2, cols.n_ulut2 = u1.data_ptr(), u2.data_ptr(), int(u[1].size)
    return keep, cols


def build_split(indices: torch.Tensor, codebook: np.ndarray, device, counts=None):
    """Split format (struct cbq_split_matrix) of decoded symbols
    (int32 [n], n % 4096 == 0), built on the device; None when a codebook
    value is not bf16 or the exponents need codes longer than 7 bits.
    counts: the symbols' histogram when the caller has it.  Returns the
    device tensors to keep alive and the descriptor."""
    n = int(indices.numel())
    if n == 0 or n % hc.CHUNK_SYMBOLS:
        return None
    if counts is None:
        counts = torch.bincount(indices.reshape(-1).clamp_min(0).to(torch.int64)).cpu().numpy()
    t = hc.split_tables(codebook, counts)
    if t is None:
        return None
    sym_code, sym_raw, lut = t
    lib = nat.load()
    st = nat.stream_ptr(device)
    sc = torch.from_numpy(sym_code.view(np.int32)).to(device)
    sr = torch.from_numpy(sym_raw).to(device)
    lt = torch.from_numpy(lut.view(np.int32)).to(device)
    n_chunks = n // hc.CHUNK_SYMBOLS
    sub_bits = torch.empty(n // hc.SUB_SYMBOLS, dtype=torch.int32, device=device)
    nat.check(lib.cbq_split_bits(indices.data_ptr(), n, sc.data_ptr(), int(sym_code.size),
                                 sub_bits.data_ptr(), st), "cbq_split_bits")
    widest = sub_bits.view(n_chunks, hc.SUB_SYMBOLS).amax(1).to(torch.int64)
    cum = torch.cumsum(torch.clamp_min((widest + 31) // 32, 1), 0)
    total = int(cum[-1])
    if total >= 2 ** 31 // hc.SUB_SYMBOLS:
        raise ValueError(f"split layout of {total} rows exceeds the 32-bit row index")
    row_off = torch.zeros(n_chunks + 1, dtype=torch.int32, device=device)
    row_off[1:] = cum.to(torch.int32)
    cwords = torch.zeros((total + 3) * hc.SUB_SYMBOLS, dtype=torch.int32, device=device)
    raw = torch.empty(n, dtype=torch.uint8, device=device)
    nat.check(lib.cbq_split_pack(indices.data_ptr(), n, sc.data_ptr(), sr.data_ptr(),
                                 int(sym_code.size), row_off.data_ptr(), cwords.data_ptr(),
                                 raw.data_ptr(), st), "cbq_split_pack")
    desc = nat.SplitMatrix(cwords=cwords.data_ptr(), row_off=row_off.data_ptr(),
                           raw=raw.data_ptr(), lut=lt.data_ptr(), n_chunks=n_chunks)
    return [cwords, row_off, raw, lt], desc


def split_bytes(keep) -> int:
    """Bytes the split GEMV streams: column words, row offsets, raw bytes, table."""
    return sum(int(t.numel() * t.element_size()) for t in keep)


def split_eligible(M: int, K: int) -> bool:
    """Shapes the split GEMV serves: K % 1024 == 0 and whole 4096-symbol
    chunks (cbq_split_linear_f32)."""
    return M > 0 and K > 0 and K % 1024 == 0 and (M * K) % hc.CHUNK_SYMBOLS == 0


def index_exact(codebook: np.ndarray, counts: np.ndarray) -> bool:
    """True when the split format's values name their indices uniquely: every
    symbol that occurs is < C and the codebook's bf16 values are distinct, so
    decoding through split_inverse returns the stored indices exactly."""
    cb = np.ascontiguousarray(codebook, np.float32).reshape(-1)
    counts = np.asarray(counts).reshape(-1)
    if counts.size > cb.size and counts[cb.size:].any():
        return False
    pats = cb.view(np.uint32) >> 16
    return np.unique(pats).size == pats.size


class SymbolDecoder:
    """Symbol-payload decode tables over a device-format stream (words,
    chunk_off, sub_len as in _DeviceStream), built once; indices() decodes
    every symbol to int32 with cbq_huff_decode_indices."""

    def __init__(self, words: torch.Tensor, chunk_off: torch.Tensor, sub_len: torch.Tensor,
                 lengths: np.ndarray, device):
        lengths = np.ascontiguousarray(lengths, np.uint8)
        lut1, lut2, canon, pay = hc.device_luts(lengths, None, int(lengths.size), False,
                                                clamp=False)
        self.device = device
        self.n_sym = int(lengths.size)
        self._keep = [words, chunk_off, sub_len,
                      torch.from_numpy(lut1.view(np.int32)).to(device),
                      torch.from_numpy(lut2.view(np.int32)).to(device),
                      torch.from_numpy(canon).to(device), torch.from_numpy(pay).to(device)]
        k = self._keep
        self.desc = nat.HuffStream(
            words=words.data_ptr(), n_words=int(words.numel()), chunk_off=chunk_off.data_ptr(),
            sub_len=sub_len.data_ptr(), lut1=k[3].data_ptr(), lut2=k[4].data_ptr(),
            n_lut2=int(lut2.size), canon=k[5].data_ptr(), canon_pay=k[6].data_ptr(),
            value_cb=None, C=self.n_sym, stage_words=hc.stage_words_for(chunk_off.cpu().numpy()))

    def indices(self, n: int) -> torch.Tensor:
        out = torch.empty(n, dtype=torch.int32, device=self.device)
        nat.check(nat.load().cbq_huff_decode_indices(ctypes.byref(self.desc), out.data_ptr(), n,
                                                     nat.stream_ptr(self.device)),
                  "cbq_huff_decode_indices")
        return out


def decode_symbols(words: torch.Tensor, chunk_off: torch.Tensor, sub_len: torch.Tensor,
                   lengths: np.ndarray, n: int, device) -> torch.Tensor:
    """Decoded symbols (int32 [n]) of a device-format stream."""
    out = SymbolDecoder(words, chunk_off, sub_len, lengths, device).indices(n)
    torch.cuda.synchronize(device)
    return out


def prefill_bits(C: int) -> int:
    """Index width of the transient fixed-width stream (8, 10..13; 9 packs
    as 10), or 0 when C needs more than 13 bits."""
    bits = max(8, int(np.ceil(np.log2(max(C, 2)))))
    bits = 10 if bits == 9 else bits
    return bits if bits <= 13 else 0


_INVERSE: dict = {}


def split_inverse(codebook: np.ndarray, device) -> torch.Tensor:
    """uint16 [65536]: bf16 bit pattern -> an index of the codebook holding
    that value (the split format stores bf16 values; any index of an equal
    value gives the same product).  One device copy per (device, codebook),
    shared by every matrix of that codebook."""
    cb = np.ascontiguousarray(codebook, np.float32).reshape(-1)
    key = (str(torch.device(device)), cb.size, hash(cb.tobytes()))
    hit = _INVERSE.get(key)
    if hit is not None and np.array_equal(hit[0], cb):
        return hit[1]
    pats = (cb.view(np.uint32) >> 16).astype(np.int64)
    inv = np.zeros(1 << 16, np.uint16)
    inv[pats[::-1]] = np.arange(len(cb), dtype=np.uint16)[::-1]     # first index wins
    t = torch.from_numpy(inv.view(np.int16)).to(device)
    _INVERSE[key] = (cb.copy(), t)
    return t




def _packed_for_gemm(idx_or_split, n: int, C: int, dev, inv: Optional[torch.Tensor] = None):
    """(packed uint8 stream, bits) of n indices for ck_linear_f32: the
    LSB-first fixed-width stream (8, 10..13 bits; 16 bits = little-endian
    uint16 when C needs more), with the zero padding the GEMV's wide reads
    need.  idx_or_split: int32 indices on the device, or a split-format
    descriptor pair decoded through inv (cbq_split_to_packed)."""
    lib = nat.load()
    st = nat.stream_ptr(dev)
    bits = prefill_bits(C) or 16
    nb = (n * bits + 7) // 8
    packed = torch.empty(((nb + 15) // 16) * 16 + 16, dtype=torch.uint8, device=dev)
    packed[nb:].zero_()                            # the padding; the stream is written below
    if inv is not None:
        nat.check(lib.cbq_split_to_packed(ctypes.byref(idx_or_split[1]), inv.data_ptr(), bits,
                                          packed.data_ptr(), st), "cbq_split_to_packed")
        return packed, bits
    idx = idx_or_split
    if bits == 16:
        packed[:2 * n] = idx.clamp(0, 0xFFFF).to(torch.int32).to(torch.int16).view(torch.uint8)
        return packed, bits
    n32 = (n + 31) // 32 * 32
    if n32 != n:                                   # whole 32-index groups for the packer
        idx = torch.cat([idx, idx.new_zeros(n32 - n)])
    nat.check(lib.cbq_pack_indices(idx.data_ptr(), n32, bits, packed.data_ptr(), st),
              "cbq_pack_indices")
    return packed, bits


def linear_from_packed(x: torch.Tensor, packed: torch.Tensor, bits: int, M: int, K: int,
                       codebook: torch.Tensor) -> torch.Tensor:
    """y [T, M] = x [T, K] (fp32) @ W^T over a transient packed index stream:
    ck_linear_f32's kernels for every T (the fp32 matrix cores for T >= 64,
    with split K in a torch workspace)."""
    lib = nat.load()
    dev = x.device
    T = x.shape[0]
    C = int(codebook.numel())
    out = torch.empty(T, M, dtype=torch.float32, device=dev)
    nws = int(lib.cbq_linear_f32_workspace(T, M, K)) if T >= 64 else 0
    ws = torch.empty(max(1, nws // 4), dtype=torch.float32, device=dev) if nws else None
    nat.check(lib.cbq_linear_f32_ws(x.data_ptr(), packed.data_ptr(), codebook.data_ptr(),
                                    out.data_ptr(), T, M, K, C, bits,
                                    None if ws is None else ws.data_ptr(), nws,
                                    nat.stream_ptr(dev)), "cbq_linear_f32_ws")
    return out


def huffman_prefill(sym: "SymbolDecoder", x: torch.Tensor, M: int, K: int,
                    codebook: torch.Tensor) -> torch.Tensor:
    """y [T, M] for batched fp32 tokens from the stream: decoded to transient
    fixed-width indices (cbq_huff_decode_indices, cbq_pack_indices) and
    multiplied by ck_linear_f32's kernels."""
    idx = sym.indices(M * K)
    packed, bits = _packed_for_gemm(idx, M * K, int(codebook.numel()), x.device)
    del idx
    return linear_from_packed(x, packed, bits, M, K, codebook)


FEWTOK_MAX_T = 32       # up to two 16-token launches of the fused kernel


def split_fewtok_eligible(K: int) -> bool:
    """Shapes cbq_split_linear_fewtok_f32 takes (its tile geometry): K % 4096
    == 0, or K % 1024 == 0 with the rows of a chunk group tiling 16 waves in
    at most two MFMA passes (K = 1024, 2048, 3072, 5120, 6144, 7168)."""
    ch = hc.CHUNK_SYMBOLS
    if K <= 0 or K % 1024:
        return False
    if K % ch == 0:
        return True
    g = math.gcd(K, ch)
    gr, rch = ch // g, K // g
    gpt = 16 // rch
    per_row = K // 64
    tr = gpt * gr
    npairs = (tr + 15) // 16 * (per_row // 4)
    return gpt >= 1 and per_row % 16 == 0 and tr * per_row * 4 <= 4096 and 1 <= npairs <= 32


def split_prefill(split, inv: torch.Tensor, x: torch.Tensor, M: int, K: int,
                  codebook: torch.Tensor) -> torch.Tensor:
    """y [T, M] for batched fp32 tokens from the split format.  Up to 32
    tokens (and a shape it takes): one fused launch per 16 tokens
    (cbq_split_linear_fewtok_f32), every weight decoded once into LDS and
    multiplied on the matrix cores, no transient buffer.  Otherwise the
    format is decoded to a transient fixed-width stream (cbq_split_to_packed,
    one table read per two weights) and multiplied by ck_linear_f32's
    kernels."""
    T = int(x.shape[0])
    if 1 <= T <= FEWTOK_MAX_T and split_fewtok_eligible(K) and x.data_ptr() % 16 == 0:
        return split_fewtok([split], x, [M], K)[0]
    packed, bits = _packed_for_gemm(split, M * K, int(codebook.numel()), x.device, inv)
    return linear_from_packed(x, packed, bits, M, K, codebook)


def split_fewtok(splits, x: torch.Tensor, Ms, K: int):
    """[y_i [T, M_i]] for up to four split-format matrices sharing x [T, K]
    (fp32, 16-byte aligned), one fused launch per 16 tokens
    (cbq_split_linear_fewtok_f32; split_fewtok_eligible(K) must hold), x's
    bf16 parts staged in a transient workspace (96 K bytes) when it pays."""
    n = len(splits)
    T = int(x.shape[0])
    outs = [torch.empty(T, int(M), dtype=torch.float32, device=x.device) for M in Ms]
    mats = (ctypes.POINTER(nat.SplitMatrix) * n)(*[ctypes.pointer(sp[1]) for sp in splits])
    optr = (ctypes.c_void_p * n)(*[o.data_ptr() for o in outs])
    mptr = (ctypes.c_int * n)(*[int(M) for M in Ms])
    lib = nat.load()
    # x's bf16 parts staged once: from 5 tokens on (the in-GEMM split then
    # costs more than the extra launch) and for the two-pass tile shapes
    two_pass = K % hc.CHUNK_SYMBOLS != 0 and K not in (1024, 2048)
    wsb = int(lib.cbq_split_fewtok_ws_bytes(K)) if (T > 4 or two_pass) else 0
    ws = torch.empty(wsb, dtype=torch.uint8, device=x.device) if wsb else None
    nat.check(lib.cbq_split_linear_fewtok_f32(x.data_ptr(), T, n, mats, optr, mptr, K,
                                              ws.data_ptr() if ws is not None else None, wsb,
                                              nat.stream_ptr(x.device)),
              "cbq_split_linear_fewtok_f32")
    return outs


def split_indices(split, inv: torch.Tensor, n: int, device) -> torch.Tensor:
    """int32 [n] codebook indices of a split-format matrix (exact when
    index_exact held at build time)."""
    out = torch.empty(n, dtype=torch.int32, device=device)
    nat.check(nat.load().cbq_split_to_packed(ctypes.byref(split[1]), inv.data_ptr(), 32,
                                             out.data_ptr(), nat.stream_ptr(device)),
              "cbq_split_to_packed")
    return out


def stack_split(splits, codebook: np.ndarray, Ms, K: int, device):
    """One split-format matrix of the row-stacked matrices `splits` (same
    codebook, same K), coded with one table built from their combined
    high-byte counts, so a single launch (cbq_split_linear_glu_f32) serves
    them all.  Returns (keep, stacked descriptor, part descriptors) -- the
    part descriptors point into the stacked arrays (row offsets and raw
    bytes offset by the parts before them), so the stacked matrix is the
    only resident copy -- or None when the shared code would need codes
    longer than 7 bits."""
    inv = split_inverse(codebook, device)
    idx = torch.cat([split_indices(sp, inv, M * K, device) for sp, M in zip(splits, Ms)])
    st = build_split(idx, codebook, device)
    del idx
    if st is None:
        return None
    keep, desc = st
    cwords, row_off, raw, lut = keep
    parts = []
    c0 = 0
    for M in Ms:
        n_ch = M * K // hc.CHUNK_SYMBOLS
        parts.append(nat.SplitMatrix(cwords=cwords.data_ptr(), row_off=row_off.data_ptr() + 4 * c0,
                                     raw=raw.data_ptr() + c0 * hc.CHUNK_SYMBOLS,
                                     lut=lut.data_ptr(), n_chunks=n_ch))
        c0 += n_ch
    return keep, desc, parts


def columns_eligible(desc: "nat.HuffStream", K: int) -> bool:
    """The column GEMV serves T = 1 rows of whole 4096-symbol chunks with
    bf16-value payloads and a second table level that fits its LDS."""
    return K % hc.CHUNK_SYMBOLS == 0 and not desc.value_cb and 1 <= desc.n_lut2 <= 8192


def _cb_numpy(codebook) -> np.ndarray:
    if isinstance(codebook, torch.Tensor):
        return codebook.detach().to(torch.float32).cpu().numpy().reshape(-1)
    return np.ascontiguousarray(codebook, np.float32).reshape(-1)


class HuffmanCodebookLinear:
    """y = x @ W^T with W Huffman-coded in HBM.

    One device format per matrix (`layout`):

    - "split" (the default wherever it applies: a bf16 codebook with distinct
      values, every symbol < C, K % 1024 == 0, whole 4096-symbol chunks): the
      split format alone, ~11.5 bits per weight, built on the device from the
      stream, after which the stream is freed.  One token runs the split
      GEMV; batched tokens decode it to a transient fixed-width stream for
      ck_linear_f32's kernels; decode_indices() maps the values back to their
      indices.
    - "stream": the reference stream in device words plus its chunk index
      (~10.8 bits per weight).  Every call runs the fused stream kernels
      (cbq_huff_linear_f32); T >= 64, and every T when K % 64 != 0, decode
      to a transient fixed-width stream for ck_linear_f32.
    - "columns": the stream plus its column layout (two formats resident),
      for comparing the column GEMV; one token runs cbq_huff_linear_col_f32.

    layout="auto" picks "split" when it applies, else "stream"."""

    def __init__(self, name: str, huff_stream, huff_lengths, huff_n: int,
                 codebook, shape, bits: int,
                 huff_row_bit_starts: Optional[np.ndarray] = None,
                 huff_lut_sym: Optional[np.ndarray] = None,
                 huff_lut_len: Optional[np.ndarray] = None,
                 huff_sl_first_code: Optional[np.ndarray] = None,
                 huff_sl_base_offset: Optional[np.ndarray] = None,
                 huff_sl_sym: Optional[np.ndarray] = None,
                 huff_chunk_offsets: Optional[np.ndarray] = None,
                 huff_sub_lens: Optional[np.ndarray] = None,
                 layout: str = "auto"):
        if not torch.cuda.is_available():
            raise RuntimeError("the compressed GPU path needs a ROCm GPU (none visible)")
        if layout not in ("auto", "split", "stream", "columns"):
            raise ValueError(f"{name}: unknown layout {layout!r}")
        self.name = name
        self.shape = tuple(int(s) for s in shape)
        self.M, self.K = self.shape
        self.bits = int(bits)
        self._lib = nat.load()
        device = codebook.device if isinstance(codebook, torch.Tensor) and codebook.is_cuda \
            else torch.device("cuda")
        self.device = device
        self._cb_np = _cb_numpy(codebook)
        self._cb_dev = torch.from_numpy(self._cb_np).to(device)
        self._lengths = np.ascontiguousarray(huff_lengths, np.uint8)
        dev = _DeviceStream(name, huff_stream, huff_lengths, huff_n, self._cb_np,
                            self.shape, huff_row_bit_starts, huff_chunk_offsets,
                            huff_sub_lens, device)
        self.split = None
        self.cols = None
        self._inv = None
        if layout in ("auto", "split") and split_eligible(self.M, self.K):
            idx = SymbolDecoder(dev.words, dev.chunk_off, dev.sub_len, self._lengths,
                                device).indices(self.M * self.K)
            counts = torch.bincount(idx.clamp_min(0).to(torch.int64)).cpu().numpy()
            if index_exact(self._cb_np, counts):
                self.split = build_split(idx, self._cb_np, device, counts=counts)
            del idx
        if layout == "split" and self.split is None:
            raise ValueError(f"{name}: the split format does not apply to this matrix")
        if self.split is not None:
            self.dev = None                       # one resident format: the stream is freed
            self._inv = split_inverse(self._cb_np, device)
        else:
            self.dev = dev
            if self.K % hc.SUB_SYMBOLS == 0 and layout == "columns":
                if not columns_eligible(dev.desc, self.K):
                    raise ValueError(f"{name}: the column layout does not apply")
                self._col_keep, self.cols = build_columns(dev.desc, self.M * self.K, device,
                                                          self._lengths, self._cb_np)
                self._cwords, self._row_off = self._col_keep[0], self._col_keep[1]

    @classmethod
    def from_device(cls, name: str, t, bits: Optional[int] = None) -> "HuffmanCodebookLinear":
        """A matrix already in HBM in its device format: a
        device_formats.SplitTensor (split layout) or HuffTensor (stream
        layout), e.g. from cbq_image.load_image.  Nothing is re-encoded."""
        import device_formats as dfm
        self = cls.__new__(cls)
        self.name = name
        self.shape = tuple(int(s) for s in t.shape)
        self.M, self.K = self.shape
        cb = t.codebook if isinstance(t, dfm.SplitTensor) else t.tables["codebook"]
        self.bits = int(bits) if bits is not None else int(np.ceil(np.log2(max(cb.numel(), 2))))
        self._lib = nat.load()
        self.device = cb.device
        self._cb_dev = cb
        self._cb_np = cb.cpu().numpy()
        self._lengths = np.ascontiguousarray(t.lengths, np.uint8)
        self.cols = None
        if isinstance(t, dfm.SplitTensor):
            self.split = t.split
            self.dev = None
            self._inv = split_inverse(self._cb_np, self.device)
        elif isinstance(t, dfm.HuffTensor):
            self.split = None
            self._inv = None
            self.dev = stream_from_device(t)
        else:
            raise TypeError(f"{name}: not a Huffman device tensor ({type(t).__name__})")
        return self

    @property
    def resident_bytes(self) -> int:
        """Device bytes of the matrix's format(s), tables included."""
        if self.split is not None:
            return split_bytes(self.split[0])
        n = self.dev.stream_bytes + self.dev.table_bytes
        if self.cols is not None:
            n += split_bytes(self._col_keep)
        return n

    @property
    def compressed_bytes(self) -> int:
        return self.resident_bytes

    def _symbols(self) -> "SymbolDecoder":
        return SymbolDecoder(self.dev.words, self.dev.chunk_off, self.dev.sub_len,
                             self._lengths, self.device)

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        in_dtype = x.dtype
        x = x.to(self.device)
        lead = x.shape[:-1]
        if x.shape[-1] != self.K:
            raise ValueError(f"{self.name}: expected last dim {self.K}, got {x.shape[-1]}")
        T = int(x.numel() // self.K)
        xc = x.reshape(T, self.K).to(torch.float32).contiguous()
        st = nat.stream_ptr(self.device)
        if T == 0:
            out = torch.empty(0, self.M, dtype=torch.float32, device=self.device)
        elif self.split is not None and (T == 1 or (
                T <= FEWTOK_MAX_T and split_fewtok_eligible(self.K) and xc.data_ptr() % 16 == 0)):
            # one token: the split GEMV; up to 32: the fused few-token kernel
            cw, ro, raw, lut = self.split[0]
            out = cbq_ops.load().split_linear(xc, cw, ro, raw, lut, self.M)
        elif self.split is not None:
            out = split_prefill(self.split, self._inv, xc, self.M, self.K, self._cb_dev)
        elif T >= 64 or self.K % hc.SUB_SYMBOLS:
            out = huffman_prefill(self._symbols(), xc, self.M, self.K, self._cb_dev)
        elif T == 1 and self.cols is not None:
            out = torch.empty(1, self.M, dtype=torch.float32, device=self.device)
            nat.check(self._lib.cbq_huff_linear_col_f32(
                xc.data_ptr(), ctypes.byref(self.dev.desc), ctypes.byref(self.cols),
                out.data_ptr(), self.M, self.K, st), "cbq_huff_linear_col_f32")
        else:
            out = cbq_ops.load().huff_linear(xc, *self.dev.op_args(), self.M)
        out = out.reshape(*lead, self.M)
        return out if in_dtype == torch.float32 else out.to(in_dtype)

    def decode_indices(self) -> torch.Tensor:
        """All M*K decoded symbols (int32, unclamped): from the split format
        through the inverse table, or from the stream with the chunked
        decoder; bit-exact either way."""
        if self.split is not None:
            out = split_indices(self.split, self._inv, self.M * self.K, self.device)
        else:
            out = self._symbols().indices(self.M * self.K)
        return out.reshape(self.M, self.K)


class HuffmanCodebookEmbedding:
    """Embedding rows decoded on demand from the Huffman stream (float32)."""

    def __init__(self, name: str, huff_stream, huff_lengths, huff_n: int,
                 codebook, shape, bits: int,
                 huff_row_bit_starts: Optional[np.ndarray] = None,
                 huff_lut_sym: Optional[np.ndarray] = None,
                 huff_lut_len: Optional[np.ndarray] = None,
                 huff_sl_first_code: Optional[np.ndarray] = None,
                 huff_sl_base_offset: Optional[np.ndarray] = None,
                 huff_sl_sym: Optional[np.ndarray] = None,
                 huff_chunk_offsets: Optional[np.ndarray] = None,
                 huff_sub_lens: Optional[np.ndarray] = None):
        if not torch.cuda.is_available():
            raise RuntimeError("the compressed GPU path needs a ROCm GPU (none visible)")
        self.name = name
        self.shape = tuple(int(s) for s in shape)
        self.vocab, self.hidden = self.shape
        self.bits = int(bits)
        self._lib = nat.load()
        device = codebook.device if isinstance(codebook, torch.Tensor) and codebook.is_cuda \
            else torch.device("cuda")
        cb = _cb_numpy(codebook)
        self.dev = _DeviceStream(name, huff_stream, huff_lengths, huff_n, cb,
                                 self.shape, huff_row_bit_starts, huff_chunk_offsets,
                                 huff_sub_lens, device)
        self.device = device
        self._lengths = np.ascontiguousarray(huff_lengths, np.uint8)
        self._cb_dev = torch.from_numpy(cb).to(device)

    @classmethod
    def from_device(cls, name: str, t, bits: Optional[int] = None) -> "HuffmanCodebookEmbedding":
        """A table already in HBM as a device_formats.HuffTensor (e.g. from
        cbq_image.load_image)."""
        self = cls.__new__(cls)
        self.name = name
        self.shape = tuple(int(s) for s in t.shape)
        self.vocab, self.hidden = self.shape
        cb = t.tables["codebook"]
        self.bits = int(bits) if bits is not None else int(np.ceil(np.log2(max(cb.numel(), 2))))
        self._lib = nat.load()
        self.device = cb.device
        self.dev = stream_from_device(t)
        self._lengths = np.ascontiguousarray(t.lengths, np.uint8)
        self._cb_dev = cb
        return self

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        ids = x.to(self.device).reshape(-1).to(torch.int32).contiguous()
        T = int(ids.numel())
        out = torch.empty(T, self.hidden, dtype=torch.float32, device=self.device)
        if T and self.hidden % hc.SUB_SYMBOLS:
            # rows that do not start on a 64-symbol sub-block: decode the
            # whole table (as the reference does per call) and gather
            idx = SymbolDecoder(self.dev.words, self.dev.chunk_off, self.dev.sub_len,
                                self._lengths, self.device).indices(self.vocab * self.hidden)
            rows = ids.to(torch.int64).clamp(0, self.vocab - 1)
            sym = idx.view(self.vocab, self.hidden)[rows].to(torch.int64)
            out = self._cb_dev[sym.clamp(0, self._cb_dev.numel() - 1)]
        elif T:
            out = cbq_ops.load().huff_embedding(ids, *self.dev.op_args(), self.vocab, self.hidden)
        return out.reshape(*x.shape, self.hidden)
