"""libcbq_hip.so loads and exports every function include/*.h declares;
host-only entry points work and argument validation rejects bad calls before
any GPU work (no kernel is launched here)."""
import ctypes
import os
import re

import numpy as np
import pytest

INCLUDE = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include")


def _declared():
    names = set()
    for f in sorted(os.listdir(INCLUDE)):
        if not f.endswith(".h"):
            continue
        text = open(os.path.join(INCLUDE, f)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names |= set(re.findall(r"^\s*(?:const\s+)?[\w\s\*]+?\b(\w+)\s*\(", text, flags=re.M))
    return sorted(names)


@pytest.fixture(scope="module")
def lib():
    import cbq_native
    try:
        return cbq_native.load()
    except RuntimeError as e:
        pytest.fail(str(e))


def test_header_symbols_exported(lib):
    names = _declared()
    assert "ck_linear_f32" in names and "cbq_huff_linear_f32" in names
    assert "cbq_attn_decode_f32" in names
    for n in names:
        assert hasattr(lib, n), f"{n} declared in include/ but not exported"
    import cbq_native
    assert set(names) == set(cbq_native.SIGNATURES), "ctypes table out of sync with header"


def test_error_strings(lib):
    assert lib.ck_error_string(0) == b"success"
    assert lib.ck_error_string(2) == b"invalid argument"
    assert b"gfx950" in lib.cbq_version()


def test_argument_validation_before_launch(lib):
    # null pointers / bad sizes return CK_ERR_ARG without touching the GPU
    assert lib.ck_linear_f32(None, None, None, None, 1, 1, 32, 1, 13, None) == 2
    buf = ctypes.create_string_buffer(64)
    p = ctypes.addressof(buf)
    assert lib.ck_linear_f32(p, p, p, p, 0, 1, 32, 1, 13, None) == 2
    assert lib.ck_linear_f32(p, p, p, p, 1, 1, 32, 1, 17, None) == 2
    assert lib.ck_linear_bf16(p, p, p, p, 1, 1, 32, 0, 13, None) == 2
    assert lib.ck_embedding_f32(p, p, p, p, 1, 0, 4, 13, None) == 2
    assert lib.cbq_embedding_f32(p, p, p, p, 1, 0, 64, 4, 13, None) == 2
    assert lib.huff_decode_to_i32(None, p, p, p, p, p, p, p, 1, 1, 20, None) == 2
    assert lib.huff_i32_linear_f32(p, p, p, p, 1, 0, 1, 1, None) == 2
    assert lib.huff_i32_embedding_f32(p, p, p, p, 1, 1, 0, None) == 2
    import cbq_native
    hs = cbq_native.HuffStream()
    assert lib.cbq_huff_linear_f32(p, ctypes.byref(hs), p, 1, 4, 64, None) == 2   # empty desc
    assert lib.cbq_huff_linear_f32(p, ctypes.byref(hs), p, 17, 4, 64, None) == 2  # T > 16
    assert lib.cbq_huff_embedding_f32(p, ctypes.byref(hs), p, 1, 4, 60, None) == 2
    assert lib.cbq_huff_decode_indices(ctypes.byref(hs), p, 64, None) == 2
    # decoder glue (include/cbq_decode.h)
    assert lib.cbq_add_rmsnorm_f32(p, None, None, p, 1, 64, 1e-6, None) == 2     # out aliases h
    assert lib.cbq_add_rmsnorm_f32(p, None, None, None, 1, 64, 1e-6, None) == 2
    assert lib.cbq_head_norm_rope_f32(*([p] * 11), 1, 4, 2, 300, 16, 1e-6, None) == 2   # hd > 256
    assert lib.cbq_head_norm_rope_f32(*([p] * 11), 1, 4, 2, 7, 16, 1e-6, None) == 2     # odd hd
    assert lib.cbq_attn_decode_f32(p, p, p, p, p, 6, 4, 128, 16, 1.0, None) == 2        # 6 % 4
    assert lib.cbq_attn_decode_f32(p, p, p, p, p, 4, 2, 96, 16, 1.0, None) == 2         # hd 96
    assert lib.cbq_attn_decode_f32(p, p, p, p, p, 4, 2, 128, 40000, 1.0, None) == 2     # > 32768
    assert lib.cbq_silu_mul_f32(p, p, p, 0, None) == 2
    # GEMVs that stage x through the glue (XF_SILU 1, XF_ADD_RMS 2, XF_RMS 3)
    xf = lib.cbq_linear_xform_f32
    assert xf(p, p, None, 0, 1e-6, p, p, p, 64, 4096, 16, 13, None) == 2        # no transform
    assert xf(p, p, None, 4, 1e-6, p, p, p, 64, 4096, 16, 13, None) == 2        # unknown mode
    assert xf(p, None, None, 1, 1e-6, p, p, p, 64, 4096, 16, 13, None) == 2     # silu needs x1
    assert xf(p, None, None, 2, 1e-6, p, p, p, 64, 4096, 16, 13, None) == 2     # add needs x1
    assert xf(p, None, None, 3, 1e-6, p, p, p, 64, 32768, 16, 13, None) == 2    # norm K > 16384
    assert xf(p, p, None, 1, 1e-6, p, p, p, 64, 17408, 16, 13, None) == 2       # silu K > 16384
    ws = ctypes.create_string_buffer(8192)
    w = ctypes.addressof(ws)
    xa = lib.cbq_linear_xform_argmax_f32
    assert xa(p, p, None, 1, 1e-6, p, p, p, 64, 17408, 16, 13, w, 8192, p, p, p, 0, 1,
              None) == 2                                                        # silu K > 16384
    glu = lib.cbq_linear_xform_glu_f32
    assert glu(p, p, None, 1, 1e-6, p, p, p, 64, 4096, 16, 13, None) == 2       # input is not silu
    assert glu(p, None, None, 2, 1e-6, p, p, p, 64, 4096, 16, 13, None) == 2    # add needs x1
    assert glu(p, None, None, 3, 1e-6, p, p, p, 64, 32768, 16, 13, None) == 2   # norm K > 16384
    assert glu(p, None, None, 0, 1e-6, p, p, p, 64, 4096, 16, 9, None) == 2     # width 9
    assert glu(p, None, None, 0, 1e-6, p, p, p, 0, 4096, 16, 13, None) == 2     # no rows
    one =(ctypes.c_void_p * 1)(p)
    m1 = (ctypes.c_int * 1)(64)
    hxf = lib.cbq_huff_linear_col_xform_f32
    assert hxf(p, None, None, 1, 1e-6, 1, one, one, one, m1, 4096, None) == 2   # silu needs x1
    assert hxf(p, p, None, 5, 1e-6, 1, one, one, one, m1, 4096, None) == 2      # unknown mode
    assert hxf(p, None, None, 3, 1e-6, 1, one, one, one, m1, 20480, None) == 2  # norm K > 16384
    assert hxf(p, None, None, 3, 1e-6, 5, one, one, one, m1, 4096, None) == 2   # > 4 matrices
    # direct-to-device load: argument and file checks come before any HIP call
    part = (cbq_native.UploadPart * 1)(cbq_native.UploadPart(0, 64, p))
    up = lib.cbq_file_upload
    assert up(b"/nonexistent/cbq.img", part, 1, 1 << 20, 2) == 2
    assert up(__file__.encode(), part, 1, 100, 2) == 2                          # chunk < 4 KiB
    assert up(__file__.encode(), part, 1, 1 << 20, 0) == 2                      # no threads
    bad = (cbq_native.UploadPart * 1)(cbq_native.UploadPart(-1, 64, p))
    assert up(__file__.encode(), bad, 1, 1 << 20, 2) == 2                       # negative offset
    assert up(__file__.encode(), part, 0, 1 << 20, 2) == 0                      # nothing to copy
    assert lib.cbq_timeline_read(None, 0) == 2               # diagnostics: product build / no buffer
    assert lib.cbq_prefill_timeline_read(None, 0) == 2
    assert lib.cbq_split_timeline_read(None, 0) == 2


def test_build_luts_rejects_overfull(lib):
    lengths = np.array([1, 1, 1], np.uint8)             # Kraft sum 1.5
    n2 = ctypes.c_int(0)
    rc = lib.cbq_huff_build_luts(lengths.ctypes.data, 3, None, 0, 0, 0, None, None,
                                 ctypes.byref(n2), None, None)
    assert rc == 2


def test_build_luts_sizes(lib):
    import huffman_codebook as hc
    lengths = np.array([2, 2, 2, 3, 4, 14, 14] + [0] * 3, np.uint8)
    lut1, lut2, canon, pay = hc.device_luts(lengths, None, 0, value_payload=False, clamp=False)
    assert lut1.size == 4096 and lut2.size == 4     # one 14-bit prefix -> 2^2 subtable
    assert canon[33 + 14] == 2 and list(pay[:5]) == [0, 1, 2, 3, 4]


def test_upload_helpers_refuse_empty_sources(lib):
    # NULL / empty sources return NULL before any HIP call
    assert lib.ck_upload_packed(None, 16) is None
    buf = ctypes.create_string_buffer(16)
    assert lib.ck_upload_packed(ctypes.addressof(buf), 0) is None
    assert lib.ck_upload_codebook(ctypes.addressof(buf), 0) is None
    assert lib.ck_upload_codebook(None, 4) is None


def test_torch_ops_registered():
    """libcbq_torch.so loads without a GPU and registers torch.ops.cbq with the
    documented schemas; the meta kernels give the output shapes."""
    import torch
    import cbq_ops
    ops = cbq_ops.load()
    want = {"linear": "linear(Tensor x, Tensor packed, Tensor codebook, int M, int bits) -> Tensor",
            "embedding": "embedding(Tensor ids, Tensor packed, Tensor codebook, int vocab, "
                         "int bits, int H) -> Tensor",
            "split_linear": "split_linear(Tensor x, Tensor cwords, Tensor row_off, Tensor raw, "
                            "Tensor lut, int M) -> Tensor"}
    for name, schema in want.items():
        assert str(getattr(ops, name).default._schema) == "cbq::" + schema
    for name in ("huff_linear", "huff_embedding"):
        assert "Tensor? value_cb" in str(getattr(ops, name).default._schema)
    m = torch.device("meta")
    x = torch.empty(3, 64, device=m)
    pk = torch.empty(100, dtype=torch.uint8, device=m)
    cb = torch.empty(10, device=m)
    assert ops.linear(x, pk, cb, 7, 4).shape == (3, 7)
    assert ops.linear(x.bfloat16(), pk, cb, 7, 4).dtype == torch.bfloat16
    ids = torch.empty(5, dtype=torch.int32, device=m)
    assert ops.embedding(ids, pk, cb, 10, 4, 64).shape == (5, 64)
    # the CPU has no kernel behind the ops: they refuse host tensors
    with pytest.raises(NotImplementedError):
        ops.linear(torch.zeros(1, 64), torch.zeros(100, dtype=torch.uint8), torch.zeros(10), 7, 4)
