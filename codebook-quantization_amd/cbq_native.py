"""ctypes binding of libcbq_hip.so, the gfx950 C ABI (include/cbq_hip.h,
include/cbq_decode.h).

The library is loaded after torch so that it binds to the HIP runtime torch
already loaded (same SONAME), which makes torch's device pointers and
streams valid inside it.  Loading fails loudly: there is no CPU fallback
behind these calls.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional

import torch  # noqa: F401  (must be loaded first: shares its HIP runtime)

HERE = os.path.dirname(os.path.abspath(__file__))
SO_PATH = os.path.join(HERE, "libcbq_hip.so")

CK_SUCCESS, CK_ERR_HIP, CK_ERR_ARG = 0, 1, 2
ARGMAX_WORKSPACE = 8192                          # CBQ_ARGMAX_WORKSPACE of include/cbq_hip.h
XF_SILU, XF_ADD_RMS, XF_RMS = 1, 2, 3            # CBQ_XF_* of include/cbq_hip.h

_vp = ctypes.c_void_p
_i = ctypes.c_int
_i64 = ctypes.c_int64


class HuffStream(ctypes.Structure):
    """struct cbq_huff_stream (include/cbq_hip.h)."""
    _fields_ = [
        ("words", _vp), ("n_words", _i64),
        ("chunk_off", _vp), ("sub_len", _vp),
        ("lut1", _vp), ("lut2", _vp), ("n_lut2", ctypes.c_int32),
        ("canon", _vp), ("canon_pay", _vp),
        ("value_cb", _vp), ("C", ctypes.c_int32),
        ("stage_words", ctypes.c_int32),
    ]


class HuffColumns(ctypes.Structure):
    """struct cbq_huff_columns (include/cbq_hip.h)."""
    _fields_ = [("cwords", _vp), ("row_off", _vp), ("n_chunks", _i64),
                ("ulut1", _vp), ("ulut2", _vp), ("n_ulut2", ctypes.c_int32)]


class SplitMatrix(ctypes.Structure):
    """struct cbq_split_matrix (include/cbq_hip.h)."""
    _fields_ = [("cwords", _vp), ("row_off", _vp), ("raw", _vp), ("lut", _vp),
                ("n_chunks", _i64)]


class UploadPart(ctypes.Structure):
    """struct cbq_upload_part (include/cbq_hip.h)."""
    _fields_ = [("file_offset", _i64), ("nbytes", _i64), ("dst", _vp)]


# name -> (restype, argtypes); every symbol declared in include/*.h
SIGNATURES = {
    "ck_error_string": (ctypes.c_char_p, [_i]),
    "cbq_version": (ctypes.c_char_p, []),
    "cbq_timeline_read": (_i, [_vp, ctypes.c_size_t]),
    "cbq_prefill_timeline_read": (_i, [_vp, ctypes.c_size_t]),
    "cbq_split_timeline_read": (_i, [_vp, ctypes.c_size_t]),
    "ck_linear_f32": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp]),
    "ck_linear_bf16": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp]),
    "cbq_linear_bf16_workspace": (ctypes.c_size_t, [_i, _i, _i]),
    "cbq_linear_f32_workspace": (ctypes.c_size_t, [_i, _i, _i]),
    "cbq_linear_f32_ws": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp, ctypes.c_size_t,
                               _vp]),
    "cbq_linear_bf16_ws": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp, ctypes.c_size_t,
                                _vp]),
    "cbq_linear_affine_f32": (_i, [_vp, _vp, ctypes.c_uint32, ctypes.c_uint32, _vp, _i, _i, _i, _i,
                                   _vp]),
    "ck_embedding_f32": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp]),
    "cbq_embedding_f32": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp]),
    "huff_decode_to_i32": (_i, [_vp] * 8 + [_i, _i, _i, _vp]),
    "huff_i32_linear_f32": (_i, [_vp] * 4 + [_i] * 4 + [_vp]),
    "huff_i32_embedding_f32": (_i, [_vp] * 4 + [_i] * 3 + [_vp]),
    "cbq_huff_build_luts": (_i, [_vp, _i, _vp, _i, _i, _i, _vp, _vp, _vp, _vp, _vp]),
    "cbq_huff_index_stream": (_i, [_vp, _i64, _vp, _i, _vp, _i, _i, _vp, _vp, _i]),
    "cbq_huff_linear_f32": (_i, [_vp, ctypes.POINTER(HuffStream), _vp, _i, _i, _i, _vp]),
    "cbq_huff_embedding_f32": (_i, [_vp, ctypes.POINTER(HuffStream), _vp, _i, _i, _i, _vp]),
    "cbq_huff_decode_indices": (_i, [ctypes.POINTER(HuffStream), _vp, _i64, _vp]),
    "cbq_huff_column_rows": (_i, [ctypes.POINTER(HuffStream), _i64, _vp, _vp]),
    "cbq_huff_build_ulut": (_i, [_vp, _i, _vp, _i, _vp, _vp, _vp]),
    "cbq_huff_columnize": (_i, [ctypes.POINTER(HuffStream), _i64, _vp, _vp, _vp]),
    "cbq_huff_linear_col_f32": (_i, [_vp, ctypes.POINTER(HuffStream), ctypes.POINTER(HuffColumns),
                                     _vp, _i, _i, _vp]),
    "cbq_huff_linear_col_multi_f32": (_i, [_vp, _i, _vp, _vp, _vp, _vp, _i, _vp]),
    "cbq_huff_linear_col_xform_f32": (_i, [_vp, _vp, _vp, _i, ctypes.c_float, _i, _vp, _vp, _vp,
                                           _vp, _i, _vp]),
    "cbq_linear_xform_f32": (_i, [_vp, _vp, _vp, _i, ctypes.c_float, _vp, _vp, _vp, _i, _i, _i,
                                  _i, _vp]),
    "cbq_linear_xform_glu_f32": (_i, [_vp, _vp, _vp, _i, ctypes.c_float, _vp, _vp, _vp, _i, _i,
                                      _i, _i, _vp]),
    "cbq_split_bits": (_i, [_vp, _i64, _vp, _i, _vp, _vp]),
    "cbq_pack_indices": (_i, [_vp, _i64, _i, _vp, _vp]),
    "cbq_split_to_packed": (_i, [_vp, _vp, _i, _vp, _vp]),
    "cbq_split_linear_fewtok_f32": (_i, [_vp, _i, _i, _vp, _vp, _vp, _i, _vp, ctypes.c_size_t,
                                         _vp]),
    "cbq_split_fewtok_ws_bytes": (ctypes.c_size_t, [_i]),
    "cbq_split_pack": (_i, [_vp, _i64, _vp, _vp, _i, _vp, _vp, _vp, _vp]),
    "cbq_split_linear_f32": (_i, [_vp, _vp, _vp, _i, ctypes.c_float, _i, _vp, _vp, _vp, _i,
                                  _vp]),
    "cbq_split_linear_glu_f32": (_i, [_vp, _vp, _vp, _i, ctypes.c_float,
                                      ctypes.POINTER(SplitMatrix), _vp, _i, _i, _vp]),
    "cbq_linear_xform_argmax_f32": (_i, [_vp, _vp, _vp, _i, ctypes.c_float, _vp, _vp, _vp, _i,
                                         _i, _i, _i, _vp, ctypes.c_size_t, _vp, _vp, _vp, _i64,
                                         _i64, _vp]),
    "cbq_split_linear_argmax_f32": (_i, [_vp, _vp, _vp, _i, ctypes.c_float,
                                         ctypes.POINTER(SplitMatrix), _vp, _i, _i, _vp,
                                         ctypes.c_size_t, _vp, _vp, _vp, _i64, _i64, _vp]),
    "ck_upload_packed": (_vp, [_vp, ctypes.c_size_t]),
    "ck_upload_codebook": (_vp, [_vp, _i]),
    "cbq_file_upload": (_i, [ctypes.c_char_p, ctypes.POINTER(UploadPart), _i, ctypes.c_size_t,
                             _i]),
    # include/cbq_decode.h
    "cbq_add_rmsnorm_f32": (_i, [_vp, _vp, _vp, _vp, _i, _i, ctypes.c_float, _vp]),
    "cbq_head_norm_rope_f32": (_i, [_vp] * 11 + [_i] * 5 + [ctypes.c_float, _vp]),
    "cbq_attn_decode_f32": (_i, [_vp] * 5 + [_i] * 4 + [ctypes.c_float, _vp]),
    "cbq_attn_rope_decode_f32": (_i, [_vp] * 11 + [_i] * 4 + [ctypes.c_float] * 2 + [_vp]),
    "cbq_attn_rope_decode_workspace": (ctypes.c_size_t, [_i, _i, _i]),
    "cbq_attn_rope_decode_ws_f32": (_i, [_vp] * 11 + [_i] * 4 + [ctypes.c_float] * 2
                                    + [_vp, ctypes.c_size_t, _vp]),
    "cbq_attn_rope_decode_noalloc_f32": (_i, [_vp] * 11 + [_i] * 4 + [ctypes.c_float] * 2
                                         + [_vp]),
    "cbq_argmax_step": (_i, [_vp, _i, _vp, _vp, _vp, _vp, _i64, _i64, _vp]),
    "cbq_silu_mul_f32": (_i, [_vp, _vp, _vp, _i64, _vp]),
}

_lib: Optional[ctypes.CDLL] = None


def load(path: str = SO_PATH) -> ctypes.CDLL:
    """Load (once) and type the library; raises if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise RuntimeError(
            f"{path} is not built: run `python codebook-quantization_amd/build_native.py` "
            "(or __graft_entry__.build()); the compressed path has no CPU fallback")
    lib = ctypes.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def check(rc: int, what: str) -> None:
    if rc != CK_SUCCESS:
        msg = load().ck_error_string(rc).decode()
        raise RuntimeError(f"{what} returned error {rc} ({msg})")


def stream_ptr(device: Optional[torch.device] = None) -> int:
    """Raw hipStream_t of torch's current stream on `device`."""
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()
