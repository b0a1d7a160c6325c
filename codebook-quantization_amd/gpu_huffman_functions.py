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
whole vocabulary for each embedding call), this backend keeps only the
stream in HBM and decodes it chunk-parallel straight into the dot product or
into the requested embedding rows.

At construction the reference stream is turned into the device format: bytes
bit-reversed into LSB-first words, decode tables rebuilt from `huff_lengths`
(the reference's huff_lut_* / huff_sl_* arrays are derived from the same
lengths and are not needed), and - when the chunk index is absent - one host
pass over the stream (split at `huff_row_bit_starts`) computes it.
"""
from __future__ import annotations

import ctypes
from typing import Optional, Tuple

import numpy as np
import torch

import cbq_native as nat
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


def build_split(indices: torch.Tensor, codebook: np.ndarray, device):
    """Split format (struct cbq_split_matrix) of decoded symbols
    (int32 [n], n % 4096 == 0), built on the device; None when a codebook
    value is not bf16 or the exponents need codes longer than 7 bits.
    Returns the device tensors to keep alive and the descriptor."""
    n = int(indices.numel())
    if n == 0 or n % hc.CHUNK_SYMBOLS:
        return None
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


def huffman_prefill(sym: SymbolDecoder, x: torch.Tensor, M: int, K: int,
                    codebook: torch.Tensor) -> Optional[torch.Tensor]:
    """y [T, M] for T >= 64 fp32 tokens: the stream is decoded to transient
    fixed-width indices (cbq_huff_decode_indices, cbq_pack_indices) and
    multiplied on the fp32 matrix cores (cbq_linear_f32_ws).  None when the
    alphabet needs more than 13 bits or K % 32 != 0."""
    T = x.shape[0]
    C = int(codebook.numel())
    bits = max(8, int(np.ceil(np.log2(max(sym.n_sym, C, 2)))))
    bits = 10 if bits == 9 else bits
    if bits > 13 or K % 32 or (M * K) % 32:
        return None
    lib = nat.load()
    dev = sym.device
    st = nat.stream_ptr(dev)
    idx = sym.indices(M * K)
    packed = torch.empty(M * K * bits // 8 + 16, dtype=torch.uint8, device=dev)
    nat.check(lib.cbq_pack_indices(idx.data_ptr(), M * K, bits, packed.data_ptr(), st),
              "cbq_pack_indices")
    del idx
    out = torch.empty(T, M, dtype=torch.float32, device=dev)
    nws = int(lib.cbq_linear_f32_workspace(T, M, K))
    ws = torch.empty(max(1, nws // 4), dtype=torch.float32, device=dev) if nws else None
    nat.check(lib.cbq_linear_f32_ws(x.data_ptr(), packed.data_ptr(), codebook.data_ptr(),
                                    out.data_ptr(), T, M, K, C, bits,
                                    None if ws is None else ws.data_ptr(), nws, st),
              "cbq_linear_f32_ws")
    return out


def prefill_bits(C: int) -> int:
    """Index width of the transient fixed-width stream (8, 10..13; 9 packs
    as 10), or 0 when C needs more than 13 bits."""
    bits = max(8, int(np.ceil(np.log2(max(C, 2)))))
    bits = 10 if bits == 9 else bits
    return bits if bits <= 13 else 0


def split_inverse(codebook: np.ndarray, device) -> torch.Tensor:
    """uint16 [65536]: bf16 bit pattern -> an index of the codebook holding
    that value (the split format stores bf16 values; any index of an equal
    value gives the same product)."""
    cb = np.ascontiguousarray(codebook, np.float32).reshape(-1)
    pats = (cb.view(np.uint32) >> 16).astype(np.int64)
    inv = np.zeros(1 << 16, np.uint16)
    inv[pats[::-1]] = np.arange(len(cb), dtype=np.uint16)[::-1]     # first index wins
    return torch.from_numpy(inv.view(np.int16)).to(device)


def split_prefill(split, inv: torch.Tensor, x: torch.Tensor, M: int, K: int,
                  codebook: torch.Tensor) -> Optional[torch.Tensor]:
    """y [T, M] for T >= 64 fp32 tokens from the split format: decoded straight
    to a transient fixed-width stream (cbq_split_to_packed, one table read per
    two weights) and multiplied on the fp32 matrix cores (cbq_linear_f32_ws).
    None when the codebook needs more than 13 bits."""
    T = x.shape[0]
    C = int(codebook.numel())
    bits = prefill_bits(C)
    if not bits or K % 32 or (M * K) % 32:
        return None
    lib = nat.load()
    dev = x.device
    st = nat.stream_ptr(dev)
    packed = torch.empty(M * K * bits // 8 + 16, dtype=torch.uint8, device=dev)
    nat.check(lib.cbq_split_to_packed(ctypes.byref(split[1]), inv.data_ptr(), bits,
                                      packed.data_ptr(), st), "cbq_split_to_packed")
    out = torch.empty(T, M, dtype=torch.float32, device=dev)
    nws = int(lib.cbq_linear_f32_workspace(T, M, K))
    ws = torch.empty(max(1, nws // 4), dtype=torch.float32, device=dev) if nws else None
    nat.check(lib.cbq_linear_f32_ws(x.data_ptr(), packed.data_ptr(), codebook.data_ptr(),
                                    out.data_ptr(), T, M, K, C, bits,
                                    None if ws is None else ws.data_ptr(), nws, st),
              "cbq_linear_f32_ws")
    return out


def columns_eligible(desc: "nat.HuffStream", K: int) -> bool:
    """The column GEMV serves T = 1 rows of whole 4096-symbol chunks with
    bf16-value payloads and a second table level that fits its LDS."""
    return K % hc.CHUNK_SYMBOLS == 0 and not desc.value_cb and 1 <= desc.n_lut2 <= 8192


def _cb_numpy(codebook) -> np.ndarray:
    if isinstance(codebook, torch.Tensor):
        return codebook.detach().to(torch.float32).cpu().numpy().reshape(-1)
    return np.ascontiguousarray(codebook, np.float32).reshape(-1)


class HuffmanCodebookLinear:
    """y = x @ W^T with W Huffman-coded in HBM; decode fused into the GEMV."""

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
                 split_format: bool = True):
        if not torch.cuda.is_available():
            raise RuntimeError("the compressed GPU path needs a ROCm GPU (none visible)")
        self.name = name
        self.shape = tuple(int(s) for s in shape)
        self.M, self.K = self.shape
        self.bits = int(bits)
        if self.K % hc.SUB_SYMBOLS:
            raise ValueError(f"{name}: in_features {self.K} must be a multiple of "
                             f"{hc.SUB_SYMBOLS}")
        self._lib = nat.load()
        device = codebook.device if isinstance(codebook, torch.Tensor) and codebook.is_cuda \
            else torch.device("cuda")
        self._cb_np = _cb_numpy(codebook)
        self._src = (huff_stream, huff_lengths, int(huff_n), huff_row_bit_starts)
        self.dev = _DeviceStream(name, huff_stream, huff_lengths, huff_n, self._cb_np,
                                 self.shape, huff_row_bit_starts, huff_chunk_offsets,
                                 huff_sub_lens, device)
        self.device = device
        self._idx_dev = None
        self._sym = None                  # symbol tables (split format, batched tokens)
        self._cb_dev = torch.from_numpy(self._cb_np).to(device)
        # single-token GEMVs read the split format when the codebook
        # is bf16-exact, else the column layout when the shape allows
        self.cols = None
        self.split = None
        self._inv = None
        if split_format and self.K % hc.CHUNK_SYMBOLS == 0:
            self._sym = SymbolDecoder(self.dev.words, self.dev.chunk_off, self.dev.sub_len,
                                      np.asarray(huff_lengths, np.uint8), device)
            idx = self._sym.indices(self.M * self.K)
            self.split = build_split(idx, self._cb_np, device)
            del idx
        if self.split is None and columns_eligible(self.dev.desc, self.K):
            self._col_keep, self.cols = build_columns(
                self.dev.desc, self.M * self.K, device, np.asarray(huff_lengths, np.uint8),
                self._cb_np)
            self._cwords, self._row_off = self._col_keep[0], self._col_keep[1]

    @property
    def compressed_bytes(self) -> int:
        return self.dev.stream_bytes + self.dev.table_bytes

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        in_dtype = x.dtype
        x = x.to(self.device)
        lead = x.shape[:-1]
        if x.shape[-1] != self.K:
            raise ValueError(f"{self.name}: expected last dim {self.K}, got {x.shape[-1]}")
        T = int(x.numel() // self.K)
        xc = x.reshape(T, self.K).to(torch.float32).contiguous()
        out = torch.empty(T, self.M, dtype=torch.float32, device=self.device)
        st = nat.stream_ptr(self.device)
        if T >= 64 and self.split is not None:
            if self._inv is None:
                self._inv = split_inverse(self._cb_np, self.device)
            y = split_prefill(self.split, self._inv, xc, self.M, self.K, self._cb_dev)
            if y is not None:
                out = y.reshape(*lead, self.M)
                return out if in_dtype == torch.float32 else out.to(in_dtype)
        if T >= 64:
            if self._sym is None:
                self._sym = SymbolDecoder(self.dev.words, self.dev.chunk_off, self.dev.sub_len,
                                          np.asarray(self._src[1], np.uint8), self.device)
            y = huffman_prefill(self._sym, xc, self.M, self.K, self._cb_dev)
            if y is not None:
                out = y.reshape(*lead, self.M)
                return out if in_dtype == torch.float32 else out.to(in_dtype)
        if T == 1 and self.split is not None:
            nat.check(self._lib.cbq_split_linear_f32(
                xc.data_ptr(), None, None, 0, 0.0, 1,
                (ctypes.POINTER(nat.SplitMatrix) * 1)(ctypes.pointer(self.split[1])),
                (ctypes.c_void_p * 1)(out.data_ptr()), (ctypes.c_int * 1)(self.M), self.K, st),
                "cbq_split_linear_f32")
            T = 0
        elif T == 1 and self.cols is not None:
            nat.check(self._lib.cbq_huff_linear_col_f32(
                xc.data_ptr(), ctypes.byref(self.dev.desc), ctypes.byref(self.cols),
                out.data_ptr(), self.M, self.K, st), "cbq_huff_linear_col_f32")
            T = 0
        for t0 in range(0, T, 16):
            tt = min(16, T - t0)
            rc = self._lib.cbq_huff_linear_f32(
                xc.data_ptr() + t0 * self.K * 4, ctypes.byref(self.dev.desc),
                out.data_ptr() + t0 * self.M * 4, tt, self.M, self.K, st)
            nat.check(rc, "cbq_huff_linear_f32")
        out = out.reshape(*lead, self.M)
        return out if in_dtype == torch.float32 else out.to(in_dtype)

    def decode_indices(self) -> torch.Tensor:
        """All M*K decoded symbols (int32, unclamped) with the chunked kernel."""
        if self._idx_dev is None:
            s, l, n, rbs = self._src
            self._idx_dev = _DeviceStream(self.name, s, l, n, self._cb_np, self.shape, rbs,
                                          None, None, self.device, raw_symbols=True)
        out = torch.empty(self.M * self.K, dtype=torch.int32, device=self.device)
        rc = self._lib.cbq_huff_decode_indices(ctypes.byref(self._idx_dev.desc), out.data_ptr(),
                                               self.M * self.K, nat.stream_ptr(self.device))
        nat.check(rc, "cbq_huff_decode_indices")
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
        if self.hidden % hc.SUB_SYMBOLS:
            raise ValueError(f"{name}: hidden {self.hidden} must be a multiple of "
                             f"{hc.SUB_SYMBOLS}")
        self._lib = nat.load()
        device = codebook.device if isinstance(codebook, torch.Tensor) and codebook.is_cuda \
            else torch.device("cuda")
        self.dev = _DeviceStream(name, huff_stream, huff_lengths, huff_n, _cb_numpy(codebook),
                                 self.shape, huff_row_bit_starts, huff_chunk_offsets,
                                 huff_sub_lens, device)
        self.device = device

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        ids = x.to(self.device).reshape(-1).to(torch.int32).contiguous()
        T = int(ids.numel())
        out = torch.empty(T, self.hidden, dtype=torch.float32, device=self.device)
        if T:
            rc = self._lib.cbq_huff_embedding_f32(ids.data_ptr(), ctypes.byref(self.dev.desc),
                                                  out.data_ptr(), T, self.vocab, self.hidden,
                                                  nat.stream_ptr(self.device))
            nat.check(rc, "cbq_huff_embedding_f32")
        return out.reshape(*x.shape, self.hidden)
