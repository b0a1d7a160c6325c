"""Drop-in AdaptiveCodebookLinear / AdaptiveCodebookEmbedding for MI355X.

Same module API as the reference (src/compressed_modules.py:48-490):

    layer = AdaptiveCodebookLinear.from_compressed(name, data, global_codebooks,
                                                   use_gpu=True, use_mmap=False,
                                                   idx_file=None)
    y = layer(x)

`data` uses the reference's keys (src/compressor.py:144-196): mode, shape,
bits, indices (packed, no pad) or the Huffman keys (encoding='huffman',
huff_stream, huff_lengths, huff_n, huff_row_bit_starts, huff_lut_*, huff_sl_*),
codebook or codebook_type; this package's encoder may add huff_chunk_offsets
and huff_sub_lens.

Dispatch (src/compressed_modules.py:77-165, 317-376):
  * 'exact'          -> F.linear / F.embedding on the stored weight;
  * 'direct_codebook'-> fixed-width or Huffman gfx950 kernels (backends in
                        gpu_accelerated_functions / gpu_huffman_functions);
  * 'linear_quant'   -> idx * scale + v_min, then F.linear.
The compressed path always runs on the GPU: the reference's CPU C-kernel,
FastIndexManager and load-time-decode fallbacks are not part of this build,
so a layer that cannot get its GPU backend raises instead of silently
falling back.
"""
from __future__ import annotations

from pathlib import Path
from typing import Tuple

import numpy as np
import torch
import torch.nn as nn
import torch.nn.functional as F

from gpu_accelerated_functions import GPUAcceleratedEmbedding, GPUAcceleratedLinear
from gpu_huffman_functions import HuffmanCodebookEmbedding, HuffmanCodebookLinear

HIP_AVAILABLE = torch.cuda.is_available()

_HUFF_KEYS = ("huff_row_bit_starts", "huff_lut_sym", "huff_lut_len", "huff_sl_first_code",
              "huff_sl_base_offset", "huff_sl_sym", "huff_chunk_offsets", "huff_sub_lens")


def _exact_weight(raw: np.ndarray, shape) -> torch.Tensor:
    if raw.dtype == np.uint16:     # bf16 bit patterns (src/compressed_modules.py:176-179)
        w = (raw.astype(np.uint32) << 16).view(np.float32)
    else:
        w = raw.astype(np.float32)
    return torch.from_numpy(np.ascontiguousarray(w).reshape(shape))


def _resolve_codebook(data: dict, global_codebooks: dict, default_type=None):
    """Local per-tensor codebook first, then the global one named by
    codebook_type / type (src/compressed_modules.py:183-196)."""
    cb = data.get("codebook")
    if cb is not None and np.asarray(cb).size > 0:
        return torch.as_tensor(np.asarray(cb)).float()
    ttype = data.get("codebook_type") or data.get("type") or default_type
    if ttype and ttype in global_codebooks:
        g = global_codebooks[ttype]
        if isinstance(g, torch.Tensor):          # e.g. bf16, as the loader returns them
            return g.detach().to("cpu", torch.float32)
        return torch.as_tensor(np.asarray(g)).float()
    return None


def _packed_indices(data: dict, use_mmap: bool, idx_file):
    if data.get("indices") is not None:
        return data["indices"]
    if idx_file is not None and Path(idx_file).exists():
        # flat .idx file of packed bytes (src/adaptive_compressor.py:1254-1315)
        return np.memmap(idx_file, dtype=np.uint8, mode="r")
    raise KeyError("direct_codebook data has neither 'indices' nor a readable idx_file")


def _gpu_required(name: str, use_gpu: bool):
    if not use_gpu:
        raise RuntimeError(f"{name}: compressed execution here is GPU-only (use_gpu=False "
                           "has no CPU path in this build)")
    if not HIP_AVAILABLE:
        raise RuntimeError(f"{name}: no ROCm GPU visible for the compressed path")


def _huff_kwargs(data: dict) -> dict:
    return {k: (np.asarray(data[k]) if data.get(k) is not None else None) for k in _HUFF_KEYS}


class AdaptiveCodebookLinear(nn.Module):
    """Linear layer whose weight stays codebook-compressed."""

    def __init__(self, name: str, shape: Tuple[int, ...], mode: str = "exact"):
        super().__init__()
        self.name = name
        self.shape = tuple(int(s) for s in shape)
        self.mode = mode
        for buf in ("bias", "indices", "codebook", "weight", "packed", "scale", "v_min"):
            self.register_buffer(buf, None, persistent=False)
        self.bits = 8
        self._gpu_func = None

    def forward(self, x):
        if self.mode == "exact":
            w = self.weight if self.weight.dtype == x.dtype else self.weight.to(x.dtype)
            return F.linear(x, w, self.bias)
        if self.mode == "direct_codebook":
            if self._gpu_func is None:
                raise RuntimeError(f"{self.name}: no GPU backend bound")
            out = self._gpu_func(x).to(x.device)
            if self.bias is not None:
                out = out + self.bias.to(device=out.device, dtype=out.dtype)
            return out
        if self.mode == "linear_quant":
            w = (self.indices.float() * self.scale + self.v_min).reshape(self.shape)
            if x.dtype != torch.float32:
                w = w.to(x.dtype)
            return F.linear(x, w, self.bias)
        raise ValueError(f"Unsupported mode: {self.mode}")

    @classmethod
    def from_compressed(cls, name: str, data: dict, global_codebooks: dict,
                        use_gpu: bool = True, use_mmap: bool = False, idx_file=None):
        mode = data["mode"]
        shape = data["shape"]
        layer = cls(name, shape, mode)
        layer.bits = int(data.get("bits", 8))
        if mode == "exact":
            layer.weight = nn.Parameter(_exact_weight(np.asarray(data["data"]), shape),
                                        requires_grad=False)
        elif mode == "direct_codebook":
            cb = _resolve_codebook(data, global_codebooks)
            if cb is None:
                raise KeyError(f"{name}: no codebook (local or global) for direct_codebook")
            layer.register_buffer("codebook", cb, persistent=False)
            _gpu_required(name, use_gpu)
            if data.get("encoding") == "huffman":
                layer._gpu_func = HuffmanCodebookLinear(
                    name, np.asarray(data["huff_stream"], np.uint8),
                    np.asarray(data["huff_lengths"], np.uint8), int(np.asarray(data["huff_n"])[0]),
                    layer.codebook, shape, layer.bits, **_huff_kwargs(data))
            else:
                layer._gpu_func = GPUAcceleratedLinear(
                    name, _packed_indices(data, use_mmap, idx_file), layer.codebook, shape,
                    layer.bits)
        elif mode == "linear_quant":
            layer.register_buffer("indices", torch.as_tensor(np.asarray(data["indices"])))
            layer.register_buffer("scale", torch.tensor(data["scale"], dtype=torch.float32))
            layer.register_buffer("v_min", torch.tensor(data["v_min"], dtype=torch.float32))
        else:
            raise ValueError(f"Unsupported mode: {mode}")
        return layer


    @classmethod
    def from_device(cls, name: str, t) -> "AdaptiveCodebookLinear":
        """A weight already in HBM: a device_formats FixedTensor,
        SplitTensor or HuffTensor (e.g. from cbq_image.load_image; bound to
        the kernels as it is, nothing uploaded or re-encoded), or a dense
        tensor (mode 'exact')."""
        import device_formats as dfm
        if isinstance(t, torch.Tensor):
            layer = cls(name, tuple(t.shape), "exact")
            layer.weight = nn.Parameter(t, requires_grad=False)
            return layer
        layer = cls(name, t.shape, "direct_codebook")
        if isinstance(t, dfm.FixedTensor):
            layer._gpu_func = GPUAcceleratedLinear.from_device(name, t)
            cb = t.codebook
        else:
            layer._gpu_func = HuffmanCodebookLinear.from_device(name, t)
            cb = layer._gpu_func._cb_dev
        layer.bits = int(layer._gpu_func.bits)
        layer.register_buffer("codebook", cb, persistent=False)
        return layer


class AdaptiveCodebookEmbedding(nn.Module):
    """Embedding whose table stays codebook-compressed."""

    def __init__(self, name: str, shape: Tuple[int, ...], mode: str = "exact"):
        super().__init__()
        self.name = name
        self.shape = tuple(int(s) for s in shape)
        self.mode = mode
        for buf in ("indices", "codebook", "weight"):
            self.register_buffer(buf, None, persistent=False)
        self.bits = 8
        self._gpu_func = None
        # e.g. Gemma scales embeddings by sqrt(hidden) (src/compressed_modules.py:313-315)
        self.embed_scale: float = 1.0

    def forward(self, x):
        if self.mode == "exact":
            out = F.embedding(x, self.weight)
        elif self.mode == "direct_codebook":
            if self._gpu_func is None:
                raise RuntimeError(f"{self.name}: no GPU backend bound")
            target = self.codebook.dtype if self.codebook is not None else torch.bfloat16
            out = self._gpu_func(x).to(device=x.device, dtype=target)
        else:
            raise ValueError(f"Unsupported mode: {self.mode}")
        return out * self.embed_scale if self.embed_scale != 1.0 else out

    @classmethod
    def from_compressed(cls, name: str, data: dict, global_codebooks: dict,
                        use_gpu: bool = True, use_mmap: bool = False, idx_file=None):
        mode = data["mode"]
        shape = data["shape"]
        layer = cls(name, shape, mode)
        layer.bits = int(data.get("bits", 8))
        if mode == "exact":
            layer.weight = nn.Parameter(_exact_weight(np.asarray(data["data"]), shape),
                                        requires_grad=False)
        elif mode == "direct_codebook":
            cb = _resolve_codebook(data, global_codebooks, default_type="embedding")
            if cb is None:
                raise KeyError(f"{name}: no codebook (local or global) for direct_codebook")
            layer.register_buffer("codebook", cb, persistent=False)
            _gpu_required(name, use_gpu)
            if data.get("encoding") == "huffman":
                layer._gpu_func = HuffmanCodebookEmbedding(
                    name, np.asarray(data["huff_stream"], np.uint8),
                    np.asarray(data["huff_lengths"], np.uint8), int(np.asarray(data["huff_n"])[0]),
                    layer.codebook, shape, layer.bits, **_huff_kwargs(data))
            else:
                layer._gpu_func = GPUAcceleratedEmbedding(
                    name, _packed_indices(data, use_mmap, idx_file), layer.codebook, shape,
                    layer.bits)
        else:
            raise ValueError(f"Unsupported mode: {mode}")
        return layer

    @classmethod
    def from_device(cls, name: str, t) -> "AdaptiveCodebookEmbedding":
        """A table already in HBM: a device_formats FixedTensor or HuffTensor
        (stream), or a dense tensor (mode 'exact')."""
        import device_formats as dfm
        if isinstance(t, torch.Tensor):
            layer = cls(name, tuple(t.shape), "exact")
            layer.weight = nn.Parameter(t, requires_grad=False)
            return layer
        layer = cls(name, t.shape, "direct_codebook")
        if isinstance(t, dfm.FixedTensor):
            layer._gpu_func = GPUAcceleratedEmbedding.from_device(name, t)
            cb = t.codebook
        elif isinstance(t, dfm.HuffTensor):
            layer._gpu_func = HuffmanCodebookEmbedding.from_device(name, t)
            cb = t.tables["codebook"]
        else:
            raise TypeError(f"{name}: no embedding over a {type(t).__name__}")
        layer.bits = int(layer._gpu_func.bits)
        layer.register_buffer("codebook", cb, persistent=False)
        return layer
