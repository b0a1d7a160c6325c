"""Lossless codebooks and index streams for bf16 weights (format producer).

The reference's lossless path (src/adaptive_compressor.py:85-136) takes the
unique bf16 values of a tensor as the codebook and stores each weight's
position in it as a ceil(log2(C))-bit index.  Here the codebook is ordered by
descending frequency (index 0 = most common value; ties by ascending bf16
bit pattern), the order the reference documents (README.md:26-29) and that
makes Huffman codes short for small indices; any order decodes identically.
Codebooks may be shared by a category of tensors (attention / mlp_ffn /
embedding, as classify_tensor in src/compressor.py:37-91).

numpy functions serve tests and small tensors; the *_torch functions run on
the GPU for multi-GB synthetic models.
"""
from __future__ import annotations

from typing import Iterable, Tuple

import numpy as np
import torch

import bitpack


def bits_for(C: int) -> int:
    """ceil(log2(max(C, 2))) (src/adaptive_compressor.py:109)."""
    return int(np.ceil(np.log2(max(int(C), 2))))


def classify_tensor(name: str) -> str:
    """Category of a parameter name for shared codebooks."""
    n = name.lower()
    if "norm" in n or "ln_" in n:
        return "layernorm"
    if "embed" in n or "lm_head" in n or "wte" in n:
        return "embedding"
    if "router" in n or ("gate" in n and "mlp" not in n and "expert" not in n):
        return "router"
    if "expert" in n or "block_sparse" in n:
        return "moe_expert"
    if "attn" in n:
        return "attention"
    return "mlp_ffn"


# ---------------------------------------------------------------------------
# numpy
# ---------------------------------------------------------------------------

def bf16_round(w) -> np.ndarray:
    """float32 -> nearest-even bf16 value, returned as float32."""
    u = np.ascontiguousarray(w, np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return (u.astype(np.uint32) << 16).view(np.float32)


def bf16_patterns(w) -> np.ndarray:
    return (np.ascontiguousarray(w, np.float32).view(np.uint32) >> 16).astype(np.int64)


def codebook_from_counts(counts: np.ndarray) -> Tuple[np.ndarray, np.ndarray]:
    """counts[65536] over bf16 patterns -> (codebook float32[C], lut[65536])."""
    present = np.nonzero(counts)[0]
    order = np.lexsort((present, -counts[present]))
    pats = present[order]
    lut = np.zeros(65536, np.int64)
    lut[pats] = np.arange(len(pats))
    return (pats.astype(np.uint32) << 16).view(np.float32), lut


def frequency_sorted_codebook(w) -> Tuple[np.ndarray, np.ndarray]:
    """(codebook float32[C], indices uint16 of w.ravel())."""
    pat = bf16_patterns(w).reshape(-1)
    cb, lut = codebook_from_counts(np.bincount(pat, minlength=65536))
    return cb, lut[pat].astype(np.uint16)


def shared_codebook(tensors: Iterable) -> Tuple[np.ndarray, np.ndarray]:
    counts = np.zeros(65536, np.int64)
    for w in tensors:
        counts += np.bincount(bf16_patterns(w).reshape(-1), minlength=65536)
    return codebook_from_counts(counts)


def compress_fixed(w, codebook=None, lut=None) -> dict:
    """Reference-format data dict for a lossless fixed-width tensor."""
    w = np.asarray(w, np.float32)
    if codebook is None:
        codebook, idx = frequency_sorted_codebook(w)
    else:
        idx = lut[bf16_patterns(w).reshape(-1)].astype(np.uint16)
    bits = bits_for(len(codebook))
    return {"mode": "direct_codebook", "shape": tuple(w.shape), "bits": bits,
            "codebook": np.asarray(codebook, np.float32),
            "indices": bitpack.pack_any_bits(idx, bits), "_raw_indices": idx}


# ---------------------------------------------------------------------------
# torch (GPU) versions for large synthetic models
# ---------------------------------------------------------------------------

def patterns_torch(w_bf16: torch.Tensor) -> torch.Tensor:
    return w_bf16.contiguous().view(torch.int16).to(torch.int32) & 0xFFFF


def counts_torch(w_bf16: torch.Tensor) -> torch.Tensor:
    return torch.bincount(patterns_torch(w_bf16).reshape(-1), minlength=65536)


def codebook_from_counts_torch(counts: torch.Tensor):
    """Descending count, ties ascending pattern -> (codebook f32, lut int64)."""
    pats = torch.arange(65536, device=counts.device, dtype=torch.int64)
    key = (counts.max() - counts.to(torch.int64)) * 65536 + pats
    present = counts > 0
    key = torch.where(present, key, torch.iinfo(torch.int64).max)
    order = torch.argsort(key)
    C = int(present.sum())
    sel = order[:C]
    lut = torch.zeros(65536, dtype=torch.int64, device=counts.device)
    lut[sel] = torch.arange(C, device=counts.device)
    cb = (sel.to(torch.int32) << 16).view(torch.float32)
    return cb, lut


def pack_torch(idx: torch.Tensor, bits: int) -> torch.Tensor:
    """LSB-first b-bit packing on the GPU -> uint8 tensor (bitpack layout).
    Index fields never overlap, so integer adds of the shifted fields equal
    their OR (int64 two's-complement, no carries)."""
    n = idx.numel()
    i64 = idx.reshape(-1).to(torch.int64) & ((1 << bits) - 1)
    pos = torch.arange(n, device=idx.device, dtype=torch.int64) * bits
    w = pos >> 6
    sh = pos & 63
    nwords = (n * bits + 63) // 64 + 1
    out = torch.zeros(nwords, dtype=torch.int64, device=idx.device)
    out.index_add_(0, w, i64 << sh)
    spill = (sh + bits) > 64
    if bool(spill.any()):
        out.index_add_(0, w[spill] + 1, i64[spill] >> (64 - sh[spill]))
    nbytes = (n * bits + 7) // 8
    return out.view(torch.uint8)[:nbytes]


def affine_form(codebook, bits: int):
    """(lo, w, remap) when the codebook's values are bf16 numbers whose
    nonzero magnitudes (bf16 bit patterns without sign) all lie in
    [lo, lo + w) with 2w + 1 <= 2^bits, else None.  remap[i] is the
    implicit-codebook index of entry i for cbq_linear_affine_f32: the
    magnitude offset for positive values, w + offset for negative ones, 2w
    for +-0."""
    cb = np.ascontiguousarray(codebook, np.float32).reshape(-1)
    u = cb.view(np.uint32)
    if cb.size == 0 or (u & 0xFFFF).any():
        return None
    v16 = (u >> 16).astype(np.int64)
    mag, sign = v16 & 0x7FFF, v16 >> 15
    nz = mag > 0
    if not nz.any():
        return None
    lo = int(mag[nz].min())
    w = int(mag[nz].max()) - lo + 1
    if 2 * w + 1 > (1 << bits) or lo + w > 0x8000:
        return None
    remap = np.where(nz, (mag - lo) + sign * w, 2 * w).astype(np.int64)
    return lo, w, remap
