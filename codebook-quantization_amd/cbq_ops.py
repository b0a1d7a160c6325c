"""torch.ops.cbq: the compressed entry points registered with torch's
dispatcher (libcbq_torch.so, built from csrc/cbq_torch_ops.cpp over the C
ABI of libcbq_hip.so).

    linear(x, packed, codebook, M, bits)              fixed-width GEMV / GEMM
    embedding(ids, packed, codebook, vocab, bits, H)  fixed-width row gather
    split_linear(x, cwords, row_off, raw, lut, M)     Huffman (split format): T = 1 the
                                                      GEMV, T >= 2 the fused few-token
                                                      kernel (K % 1024 == 0 shapes)
    huff_linear(x, words, chunk_off, sub_len, lut1, lut2, canon, canon_pay,
                value_cb, C, stage_words, M)           Huffman (stream format)
    huff_embedding(ids, <stream tensors>, C, stage_words, vocab, H)

The modules (compressed_modules via gpu_accelerated_functions and
gpu_huffman_functions) call these ops; they run on torch's current HIP
stream, allocate outputs and workspaces from torch's caching allocator and
can be captured in a torch.cuda.graph.  Loading fails loudly when the
library is not built: there is no CPU fallback behind the ops.
"""
from __future__ import annotations

import os

import torch

import cbq_native

HERE = os.path.dirname(os.path.abspath(__file__))
SO_PATH = os.path.join(HERE, "libcbq_torch.so")

_loaded = False


def load(path: str = SO_PATH):
    """Register torch.ops.cbq (once) and return the namespace."""
    global _loaded
    if not _loaded:
        if not os.path.exists(path):
            raise RuntimeError(
                f"{path} is not built: run `python codebook-quantization_amd/build_native.py` "
                "(or __graft_entry__.build()); the compressed path has no CPU fallback")
        cbq_native.load()              # libcbq_hip.so first, typed for the ctypes callers
        torch.ops.load_library(path)
        _loaded = True
    return torch.ops.cbq
