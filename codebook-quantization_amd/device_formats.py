"""Device-resident formats of one compressed matrix and the GPU encoder that
produces them from codebook indices.

- FixedTensor: fixed-width b-bit indices, LSB-first packed (the reference's
  bitpack layout, src/bitpack.py:32-95), zero-padded to whole 16 bytes + 16,
  and the float32 codebook.
- HuffTensor: the canonical-Huffman stream as LSB-first 32-bit words (bit j
  of the reference's MSB-first stream byte i is bit 7 - j of byte i here,
  src/huffman_codebook.py:197-201), the chunk index (uint64 bit offset of
  every 4096th symbol plus the total) and the 64-symbol sub-block bit
  lengths, with the decode tables built from the code lengths.
- SplitTensor: the split format of a Huffman matrix (cbq_split_matrix):
  per 4096-symbol chunk the raw low byte of every weight's bf16 pattern and
  a <= 7-bit code of its high byte in 64 side-by-side columns.  What the
  decode-step GEMV streams; built on the GPU from the matrix's indices.

The encoder runs on whatever device the indices live on (torch integer ops
only: the same bits on the CPU and the GPU).
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import List, Optional, Tuple

import numpy as np
import torch

import codebook_builder as cbb
import huffman_codebook as hc


@dataclass
class FixedTensor:
    name: str
    shape: Tuple[int, int]
    bits: int
    category: str
    packed: torch.Tensor            # uint8, device, padded
    codebook: torch.Tensor          # float32, device

    @property
    def nbytes(self) -> int:
        return (self.shape[0] * self.shape[1] * self.bits + 7) // 8


@dataclass
class HuffTensor:
    name: str
    shape: Tuple[int, int]
    category: str
    lengths: np.ndarray
    words: torch.Tensor             # int32 view of LSB-first words
    chunk_off: torch.Tensor         # int64 (uint64 values)
    sub_len: torch.Tensor           # int16 (uint16 values)
    total_bits: int
    tables: dict = field(default_factory=dict)

    @property
    def nbytes(self) -> int:
        """Stream bytes + chunk table + sub-block table."""
        return (self.total_bits + 7) // 8 + self.chunk_off.numel() * 8 + self.sub_len.numel() * 2


@dataclass
class SplitTensor:
    name: str
    shape: Tuple[int, int]
    category: str
    lengths: np.ndarray             # the Huffman code lengths it was built from
    keep: List[torch.Tensor]        # cwords int32, row_off int32, raw uint8, lut int32
    desc: object                    # cbq_native.SplitMatrix over keep
    codebook: torch.Tensor          # float32, device

    @property
    def split(self):
        """(keep, desc), the pair gpu_huffman_functions.build_split returns."""
        return self.keep, self.desc

    @property
    def nbytes(self) -> int:
        return sum(int(t.numel() * t.element_size()) for t in self.keep)


def split_from_arrays(name, shape, category, lengths, cwords, row_off, raw, lut, codebook,
                      n_chunks: int) -> SplitTensor:
    """SplitTensor over device arrays already in the split layout."""
    import cbq_native as nat
    desc = nat.SplitMatrix(cwords=cwords.data_ptr(), row_off=row_off.data_ptr(),
                           raw=raw.data_ptr(), lut=lut.data_ptr(), n_chunks=int(n_chunks))
    return SplitTensor(name, tuple(shape), category, np.asarray(lengths, np.uint8),
                       [cwords, row_off, raw, lut], desc, codebook)


def stack_fixed(parts, name: str) -> Optional[FixedTensor]:
    """Row-stack fixed-width tensors that share K, the index width and the
    codebook (q/k/v, gate/up): when every part's index stream ends on a byte
    boundary, the concatenated bytes are exactly the packed stream of the
    stacked [sum M, K] matrix, so one GEMV launch computes all parts.
    None when the parts do not qualify."""
    K, bits, cb = parts[0].shape[1], parts[0].bits, parts[0].codebook
    for t in parts:
        if (t.shape[1] != K or t.bits != bits or t.codebook.data_ptr() != cb.data_ptr()
                or t.codebook.numel() != cb.numel() or (t.shape[0] * K * bits) % 8):
            return None
    M = sum(t.shape[0] for t in parts)
    nb = (M * K * bits) // 8
    packed = torch.zeros(((nb + 15) // 16) * 16 + 16, dtype=torch.uint8, device=cb.device)
    o = 0
    for t in parts:
        packed[o:o + t.nbytes] = t.packed[:t.nbytes]
        o += t.nbytes
    return FixedTensor(name, (M, K), bits, parts[0].category, packed, cb)


# ---- encoder ---------------------------------------------------------------

def huffman_encode_torch(idx: torch.Tensor, lengths: np.ndarray, row_len: int = 0):
    """Canonical-Huffman encoder on idx's device -> (int32 words, chunk_off,
    sub_len, total bits), plus the bit start of every row_len-th symbol
    (the reference's huff_row_bit_starts) when row_len > 0.

    Codes are bit-reversed and scattered LSB-first into 64-bit words; code
    fields never overlap, so integer adds of the shifted fields equal their OR.
    """
    dev = idx.device
    codes = hc.canonical_codes(lengths)
    rev = hc._bitrev(codes, lengths.astype(np.int64)).astype(np.int64)
    L_tab = torch.from_numpy(lengths.astype(np.int64)).to(dev)
    R_tab = torch.from_numpy(rev).to(dev)
    flat = idx.reshape(-1).to(torch.int64)
    L = L_tab[flat]
    starts = torch.cumsum(L, 0) - L
    total = int(starts[-1] + L[-1])
    words = torch.zeros(total // 64 + 3, dtype=torch.int64, device=dev)
    w = starts >> 6
    sh = starts & 63
    r = R_tab[flat]
    words.index_add_(0, w, r << sh)
    spill = (sh + L) > 64
    if bool(spill.any()):
        words.index_add_(0, w[spill] + 1, r[spill] >> (64 - sh[spill]))
    tot = torch.tensor([total], dtype=torch.int64, device=dev)
    chunk_off = torch.cat([starts[::hc.CHUNK_SYMBOLS], tot])
    sub_len = torch.diff(torch.cat([starts[::hc.SUB_SYMBOLS], tot])).to(torch.int16)
    if row_len > 0:
        return words.view(torch.int32), chunk_off, sub_len, total, starts[::row_len].clone()
    return words.view(torch.int32), chunk_off, sub_len, total


def huff_tables_host(lengths: np.ndarray, codebook_np: np.ndarray, codebook: torch.Tensor,
                     stage_words: int, device) -> dict:
    """Decode tables of a value-payload stream (lut1, lut2, canon, pay) from
    its code lengths and host codebook, its LDS staging size and the device
    codebook: HuffTensor.tables."""
    cb_np = np.ascontiguousarray(codebook_np, np.float32)
    lut1, lut2, canon, pay = hc.device_luts(lengths, cb_np, int(cb_np.size), value_payload=True)
    return dict(lut1=torch.from_numpy(lut1.view(np.int32)).to(device),
                lut2=torch.from_numpy(lut2.view(np.int32)).to(device),
                canon=torch.from_numpy(canon).to(device),
                pay=torch.from_numpy(pay).to(device),
                stage_words=int(stage_words), codebook=codebook)


def huff_tables(lengths: np.ndarray, codebook: torch.Tensor, chunk_off: torch.Tensor,
                device) -> dict:
    """huff_tables_host with the codebook and chunk index on the device."""
    return huff_tables_host(lengths, codebook.cpu().numpy(), codebook,
                            hc.stage_words_for(chunk_off.cpu().numpy()), device)


def encode_fixed(name: str, idx: torch.Tensor, codebook: torch.Tensor, shape, category: str
                 ) -> FixedTensor:
    """Fixed-width tensor of int indices (any integer dtype) into `codebook`
    at ceil(log2(max(C, 2))) bits (src/adaptive_compressor.py:109)."""
    bits = cbb.bits_for(codebook.numel())
    pk = cbb.pack_torch(idx.reshape(-1), bits)
    padded = torch.zeros(((pk.numel() + 15) // 16) * 16 + 16, dtype=torch.uint8,
                         device=idx.device)
    padded[:pk.numel()] = pk
    return FixedTensor(name, tuple(shape), bits, category, padded, codebook.contiguous())


def encode_huffman(name: str, idx: torch.Tensor, codebook: torch.Tensor, shape, category: str,
                   max_len: int = hc.DEFAULT_MAX_LEN, with_row_starts: bool = False):
    """Huffman tensor of int indices: lengths from this tensor's symbol
    counts (package-merge, <= max_len bits), the stream and its chunk index
    encoded on idx's device.  With with_row_starts also returns the bit
    start of every row (int64 tensor)."""
    M, K = shape
    flat = idx.reshape(-1).to(torch.int64)
    C = codebook.numel()
    counts = torch.bincount(flat, minlength=C).cpu().numpy()
    lengths = hc.length_limited_code_lengths(counts, max_len)
    enc = huffman_encode_torch(flat, lengths, K if with_row_starts else 0)
    words, chunk_off, sub_len, total = enc[:4]
    t = HuffTensor(name, (M, K), category, lengths, words, chunk_off, sub_len, total)
    t.tables = huff_tables(lengths, codebook, chunk_off, idx.device)
    t.tables["counts"] = counts
    return (t, enc[4]) if with_row_starts else t


def to_split(t: HuffTensor, indices: Optional[torch.Tensor] = None) -> Optional[SplitTensor]:
    """The split format of a Huffman tensor (None when its shape or codebook
    does not allow one).  indices: the tensor's decoded symbols when the
    caller has them (the encoder does); else the stream is decoded on the
    GPU."""
    from gpu_huffman_functions import SymbolDecoder, build_split, split_eligible
    M, K = t.shape
    if not split_eligible(M, K):
        return None
    dev = t.words.device
    if indices is None:
        indices = SymbolDecoder(t.words, t.chunk_off, t.sub_len, t.lengths, dev).indices(M * K)
    cb = t.tables["codebook"]
    sp = build_split(indices.reshape(-1).to(torch.int32), cb.cpu().numpy(), dev,
                     counts=t.tables.get("counts"))
    if sp is None:
        return None
    return SplitTensor(t.name, t.shape, t.category, t.lengths, sp[0], sp[1], cb)
