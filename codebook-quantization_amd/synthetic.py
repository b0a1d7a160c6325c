"""Synthetic compressed decoders built on the GPU (bench and e2e workloads).

Weights are N(0, std) bf16 values drawn per tensor by a counter-based
integer generator (make_bf16): a 32-bit hash of (tensor seed, element index)
picks the bf16 value through an inverse-CDF table of the normal distribution
over bf16 rounding intervals.  Only integer operations touch the samples, so
the CPU (numpy or torch) and the GPU produce the same bits, and a CPU oracle
can rebuild exactly the model the GPU runs.  Lossless codebooks are shared
per category (attention / mlp_ffn / embedding) and frequency-sorted;
fixed-width tensors are packed LSB-first; Huffman tensors get their own 24-bit-limited canonical code
(lengths from that tensor's symbol counts, as the reference codes each
tensor, src/adaptive_compressor.py:111-127) and the chunk index.
"""
from __future__ import annotations

import zlib
from typing import Dict, List, Optional, Tuple

import numpy as np
import torch

import codebook_builder as cbb
import huffman_codebook as hc
from device_formats import (FixedTensor, HuffTensor, SplitTensor, encode_fixed,  # noqa: F401
                            encode_huffman, huffman_encode_torch, stack_fixed, to_split)

# (name, out_features, in_features) per decoder layer
def layer_shapes(hidden: int, inter: int, n_q: int, n_kv: int, head_dim: int):
    return [("self_attn.q_proj", n_q * head_dim, hidden),
            ("self_attn.k_proj", n_kv * head_dim, hidden),
            ("self_attn.v_proj", n_kv * head_dim, hidden),
            ("self_attn.o_proj", hidden, n_q * head_dim),
            ("mlp.gate_proj", inter, hidden),
            ("mlp.up_proj", inter, hidden),
            ("mlp.down_proj", hidden, inter)]


CONFIGS = {
    # benchmark config 5: Qwen3-8B-style, 36 layers
    "qwen3-8b": dict(layers=36, hidden=4096, inter=12288, n_q=32, n_kv=8, head_dim=128,
                     vocab=151936),
    # benchmark config 2: Qwen3-1.7B-style, 28 layers
    "qwen3-1.7b": dict(layers=28, hidden=2048, inter=6144, n_q=16, n_kv=8, head_dim=128,
                       vocab=151936),
}


def tensor_seed(name: str, base: int = 0) -> int:
    return (zlib.crc32(name.encode()) ^ (base * 0x9E3779B1)) & 0x7FFFFFFF


_M32 = 0xFFFFFFFF
_GEN_CHUNK = 1 << 26


def _mul32(x, c: int):
    """(x * c) mod 2^32 for x in [0, 2^32) held in int64 (torch or numpy):
    the constant is split in 16-bit halves so no product exceeds 2^49."""
    return (x * (c & 0xFFFF) + (((x * (c >> 16)) & 0xFFFF) << 16)) & _M32


def mix32(x):
    """Chris Wellons' "lowbias32" 32-bit integer hash (hash-prospector):
    x ^= x>>16; x *= 0x7feb352d; x ^= x>>15; x *= 0x846ca68b; x ^= x>>16."""
    x = x ^ (x >> 16)
    x = _mul32(x, 0x7FEB352D)
    x = x ^ (x >> 15)
    x = _mul32(x, 0x846CA68B)
    return x ^ (x >> 16)


def uniform32(i, seed: int):
    """Uniform 32-bit integers for element indices i (int64, < 2^32) of the
    stream `seed`: two hash rounds keyed by the seed."""
    a = (i + ((seed * 0x9E3779B9) & _M32)) & _M32
    return mix32(mix32(a) ^ ((seed * 0x85EBCA6B) & _M32))


_TABLES: Dict[float, Tuple[np.ndarray, np.ndarray]] = {}


def normal_bf16_table(std: float = 0.02) -> Tuple[np.ndarray, np.ndarray]:
    """(pats uint16 [n], thr int64 [n-1]): the bf16 values with nonzero
    probability under N(0, std) rounded to nearest bf16, in ascending order,
    and the upper ends of their intervals on the 2^32 grid.  A uniform u in
    [0, 2^32) draws pats[searchsorted(thr, u, side='right')].  Value j's
    interval is bounded by the midpoints to its neighbours (its rounding
    interval), so its probability is Phi(mid_hi/std) - Phi(mid_lo/std) to
    within 2^-32."""
    if std in _TABLES:
        return _TABLES[std]
    from scipy.special import ndtr
    pos = np.arange(1, 0x7F80, dtype=np.uint32)              # positive finite bf16
    pv = (pos << 16).view(np.float32).astype(np.float64)
    vals = np.concatenate([-pv[::-1], [0.0], pv])
    pats = np.concatenate([pos[::-1] | 0x8000, [0], pos]).astype(np.uint16)
    mids = 0.5 * (vals[1:] + vals[:-1])
    thr = np.floor(ndtr(mids / std) * 2.0 ** 32).astype(np.int64)
    lo = np.concatenate([[0], thr])
    hi = np.concatenate([thr, [1 << 32]])
    keep = hi > lo
    _TABLES[std] = (pats[keep], hi[keep][:-1].copy())
    return _TABLES[std]


def make_bf16(shape, name: str, std: float = 0.02, base_seed: int = 0,
              device="cuda") -> torch.Tensor:
    """N(0, std) bf16 weights of one tensor, identical bits on every device
    (see normal_bf16_table and uniform32)."""
    pats, thr = normal_bf16_table(std)
    dev = torch.device(device)
    pats_t = torch.from_numpy(pats.view(np.int16)).to(dev)
    thr_t = torch.from_numpy(thr).to(dev)
    seed = tensor_seed(name, base_seed)
    n = int(np.prod(shape))
    out = torch.empty(n, dtype=torch.int16, device=dev)
    step = n if dev.type == "cuda" else _GEN_CHUNK
    for s0 in range(0, n, step):
        s1 = min(n, s0 + step)
        u = uniform32(torch.arange(s0, s1, dtype=torch.int64, device=dev), seed)
        out[s0:s1] = pats_t[torch.searchsorted(thr_t, u, right=True)]
    return out.view(torch.bfloat16).reshape(shape)


class SyntheticDecoder:
    """All linear weights of a decoder (+ lm_head and embedding), compressed."""

    def __init__(self, config: str = "qwen3-8b", layers: Optional[int] = None,
                 base_seed: int = 0, device="cuda", log=print):
        c = dict(CONFIGS[config])
        if layers is not None:
            c["layers"] = layers
        self.cfg = c
        self.device = torch.device(device)
        self.base_seed = base_seed
        self.log = log
        shapes = layer_shapes(c["hidden"], c["inter"], c["n_q"], c["n_kv"], c["head_dim"])
        self.linears: List[Tuple[str, int, int]] = [
            (f"model.layers.{i}.{n}", M, K) for i in range(c["layers"]) for n, M, K in shapes]
        self.lm_head = ("lm_head", c["vocab"], c["hidden"])
        self.embed = ("model.embed_tokens", c["vocab"], c["hidden"])

    def all_linears(self, with_head=True):
        return self.linears + ([self.lm_head] if with_head else [])

    def _gen(self, name, M, K):
        return make_bf16((M, K), name, base_seed=self.base_seed, device=self.device)

    def category_codebooks(self, tensors) -> Dict[str, Tuple[torch.Tensor, torch.Tensor]]:
        counts: Dict[str, torch.Tensor] = {}
        for name, M, K in tensors:
            cat = cbb.classify_tensor(name)
            cnt = cbb.counts_torch(self._gen(name, M, K))
            counts[cat] = counts[cat] + cnt if cat in counts else cnt
        return {cat: cbb.codebook_from_counts_torch(cnt) for cat, cnt in counts.items()}

    def build_fixed(self, tensors) -> Dict[str, FixedTensor]:
        books = self.category_codebooks(tensors)
        out = {}
        for name, M, K in tensors:
            cat = cbb.classify_tensor(name)
            cb, lut = books[cat]
            idx = lut[cbb.patterns_torch(self._gen(name, M, K)).reshape(-1).to(torch.int64)]
            out[name] = encode_fixed(name, idx, cb, (M, K), cat)
        return out

    def build_huffman(self, tensors, max_len: int = hc.DEFAULT_MAX_LEN) -> Dict[str, HuffTensor]:
        books = self.category_codebooks(tensors)
        out = {}
        for name, M, K in tensors:
            cat = cbb.classify_tensor(name)
            cb, lut = books[cat]
            idx = lut[cbb.patterns_torch(self._gen(name, M, K)).reshape(-1).to(torch.int64)]
            out[name] = encode_huffman(name, idx, cb, (M, K), cat, max_len)
        return out


# ---- CPU (numpy) builder for small models: tests and golden fixtures --------

def make_bf16_cpu(shape, name: str, std: float = 0.02, base_seed: int = 0) -> np.ndarray:
    """N(0, std) rounded to bf16 (nearest even), from PCG64 seeded per tensor."""
    rng = np.random.default_rng(tensor_seed(name, base_seed))
    return cbb.bf16_round(rng.standard_normal(shape, dtype=np.float32) * np.float32(std))


def compress_model_cpu(cfg, base_seed: int = 0, encoding: str = "fixed",
                       huffman_max_len: int = hc.DEFAULT_MAX_LEN) -> Dict[str, dict]:
    """Every linear, the lm_head and the embedding of a decoder.DecoderConfig,
    compressed on the CPU as reference-format data dicts (shared
    per-category frequency-sorted codebooks, src/adaptive_compressor.py:870-969).
    Dense weights come back under "_dense" (bf16 values as float32) for the
    golden-fixture generator."""
    names = [(n, M, K) for n, M, K in cfg.linear_shapes()]
    names.append(("model.embed_tokens", cfg.vocab, cfg.hidden))
    dense = {n: make_bf16_cpu((M, K), n, base_seed=base_seed) for n, M, K in names}
    cats: Dict[str, list] = {}
    for n, _, _ in names:
        cats.setdefault(cbb.classify_tensor(n), []).append(n)
    books = {c: cbb.shared_codebook(dense[n] for n in ns) for c, ns in cats.items()}
    out: Dict[str, dict] = {}
    for n, M, K in names:
        cb, lut = books[cbb.classify_tensor(n)]
        if encoding == "huffman":
            idx = lut[cbb.bf16_patterns(dense[n]).reshape(-1)]
            enc = hc.huffman_encode_indices(idx, shape=(M, K), max_len=huffman_max_len)
            d = {"mode": "direct_codebook", "encoding": "huffman", "shape": (M, K),
                 "bits": cbb.bits_for(len(cb)), "codebook": cb}
            d.update(enc)
        else:
            d = cbb.compress_fixed(dense[n], codebook=cb, lut=lut)
        d["_dense"] = dense[n]
        out[n] = d
    return out
