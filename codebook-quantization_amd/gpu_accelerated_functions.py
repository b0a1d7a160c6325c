"""Fixed-width compressed linear / embedding on gfx950 (drop-in backends).

Same classes, constructor and call signatures as the reference
(src/gpu_accelerated_functions.py:871-1029):

    GPUAcceleratedLinear(name, indices_np, codebook, shape, bits)(x)
    GPUAcceleratedEmbedding(name, indices_np, codebook, shape, bits)(ids)

The packed indices (+ zero padding) and the float32 codebook are copied to
the device once, at construction.  Each call is one torch.ops.cbq op
(cbq_ops: libcbq_torch.so over libcbq_hip.so's C ABI) on torch's current
stream, with no synchronisation:
  * linear: out = x @ W^T with W[m, k] = codebook[min(idx, C-1)], fp32
    accumulate, output in x's dtype (bf16 x runs the bf16-I/O kernel
    directly; other dtypes go through fp32);
  * embedding: out[..., h] = codebook[idx[id * H + h]] as float32 (the module
    casts to the codebook dtype, src/compressed_modules.py:322-330).
There is no CPU fallback: construction fails without a GPU and the built
library.
"""
from __future__ import annotations

import numpy as np
import torch

import bitpack
import cbq_native as nat
import cbq_ops


def _device_for(codebook: torch.Tensor) -> torch.device:
    if not torch.cuda.is_available():
        raise RuntimeError("the compressed GPU path needs a ROCm GPU (none visible)")
    return codebook.device if codebook.is_cuda else torch.device("cuda")


def index_bytes(indices, bits: int) -> np.ndarray:
    """The packed index bytes of a stored 'indices' array.  The reference
    keeps 8- and 16-bit indices unpacked as uint16 arrays
    (src/adaptive_compressor.py:128-131): 8-bit values are the bytes
    themselves, 16-bit values their little-endian byte pairs (the 16-bit
    layout of src/bitpack.py).  Every other array already holds the bytes."""
    arr = indices if isinstance(indices, np.ndarray) else indices.detach().cpu().numpy()
    arr = np.ascontiguousarray(arr).reshape(-1)
    if arr.dtype in (np.uint16, np.int16) and bits == 16:
        return arr.astype("<u2", copy=False).view(np.uint8)
    return arr.astype(np.uint8, copy=False)


def _upload_packed(arr: np.ndarray, device) -> torch.Tensor:
    return torch.from_numpy(bitpack.device_padded(arr.reshape(-1))).to(device)


class GPUAcceleratedLinear:
    """Packed indices + codebook in HBM; fused unpack / gather / dot on call."""

    def __init__(self, name: str, indices_np, codebook: torch.Tensor, shape: tuple, bits: int):
        self.name = name
        self.shape = tuple(int(s) for s in shape)          # (out_features, in_features)
        self.M, self.K = self.shape
        self.bits = int(bits)
        if not 1 <= self.bits <= 16:
            raise ValueError(f"{name}: bits must be in [1, 16], got {bits}")
        self._lib = nat.load()
        device = _device_for(codebook)
        self.codebook = codebook.detach().to(device=device, dtype=torch.float32).contiguous()
        self.C = int(self.codebook.numel())
        need = bitpack.calculate_packed_size(self.M * self.K, self.bits)
        raw = index_bytes(indices_np, self.bits)
        if raw.size < need:
            raise ValueError(f"{name}: {raw.size} packed bytes < {need} needed for "
                             f"{self.M}x{self.K} at {self.bits} bits")
        self.packed = _upload_packed(raw, device)

    @classmethod
    def from_device(cls, name: str, t) -> "GPUAcceleratedLinear":
        """A device_formats.FixedTensor already in HBM (padded packed bytes
        and codebook, e.g. from cbq_image.load_image): no host copy."""
        self = cls.__new__(cls)
        self.name = name
        self.shape = tuple(int(s) for s in t.shape)
        self.M, self.K = self.shape
        self.bits = int(t.bits)
        self._lib = nat.load()
        self.codebook = t.codebook
        self.C = int(t.codebook.numel())
        self.packed = t.packed
        return self

    @property
    def compressed_bytes(self) -> int:
        return bitpack.calculate_packed_size(self.M * self.K, self.bits)

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        in_dtype = x.dtype
        dev = self.codebook.device
        x = x.to(dev)
        lead = x.shape[:-1]
        if x.shape[-1] != self.K:
            raise ValueError(f"{self.name}: expected last dim {self.K}, got {x.shape[-1]}")
        T = int(x.numel() // self.K)
        if T == 0:
            return torch.empty(*lead, self.M, dtype=in_dtype, device=dev)
        ops = cbq_ops.load()
        if in_dtype == torch.bfloat16:
            # bf16 I/O kernel (batched tokens: bf16 MFMA with fp32 accumulation)
            out = ops.linear(x.reshape(T, self.K).contiguous(), self.packed, self.codebook,
                             self.M, self.bits)
            return out.reshape(*lead, self.M)
        xc = x.reshape(T, self.K).to(torch.float32).contiguous()
        out = ops.linear(xc, self.packed, self.codebook, self.M, self.bits).reshape(*lead, self.M)
        return out if in_dtype == torch.float32 else out.to(in_dtype)


class GPUAcceleratedEmbedding:
    """Rows gathered straight from the packed table; float32 output."""

    def __init__(self, name: str, indices_np, codebook: torch.Tensor, shape: tuple, bits: int):
        self.name = name
        self.shape = tuple(int(s) for s in shape)          # (vocab, hidden)
        self.vocab, self.hidden = self.shape
        self.bits = int(bits)
        if not 1 <= self.bits <= 16:
            raise ValueError(f"{name}: bits must be in [1, 16], got {bits}")
        self._lib = nat.load()
        device = _device_for(codebook)
        self.codebook = codebook.detach().to(device=device, dtype=torch.float32).contiguous()
        self.C = int(self.codebook.numel())
        self.packed = _upload_packed(index_bytes(indices_np, self.bits), device)

    @classmethod
    def from_device(cls, name: str, t) -> "GPUAcceleratedEmbedding":
        """A device_formats.FixedTensor already in HBM: no host copy."""
        self = cls.__new__(cls)
        self.name = name
        self.shape = tuple(int(s) for s in t.shape)
        self.vocab, self.hidden = self.shape
        self.bits = int(t.bits)
        self._lib = nat.load()
        self.codebook = t.codebook
        self.C = int(t.codebook.numel())
        self.packed = t.packed
        return self

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        dev = self.codebook.device
        ids = x.to(dev).reshape(-1).to(torch.int32).contiguous()
        out = cbq_ops.load().embedding(ids, self.packed, self.codebook, self.vocab, self.bits,
                                       self.hidden)
        return out.reshape(*x.shape, self.hidden)
