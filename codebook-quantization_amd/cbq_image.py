"""Device image: a model's compressed weights in their device formats, one
file, copied straight into HBM at load.

The reference loads a compressed model from one gzip .npz per tensor on a
thread pool (src/compressor.py:347-361) or from raw .idx files by mmap
(src/compressed_matmul_cpu.py:23-63), then pads and uploads each array
(src/gpu_accelerated_functions.py:860-864).  Here the encoder writes every
matrix already in the form the kernels read (device_formats: fixed-width
packed bytes, Huffman split format, Huffman stream with its chunk index),
and loading is one device allocation filled by cbq_file_upload: reader
threads, pinned staging, asynchronous copies, no host decode or re-index.

File layout (little-endian):

    [0, 8)        magic b"CBQIMG01"
    [8, 16)       header length H (uint64)
    [16, 16 + H)  header, JSON (UTF-8)
    ...           zero padding to data_offset (a multiple of 4096)
    payload       sections, each at a 4096-aligned offset from data_offset

Header keys: format, version, data_offset, payload_bytes, meta (free-form,
e.g. the decoder config), codebooks {id: {offset, nbytes}} (float32
arrays, stored once and shared by every tensor that names them), tensors
{name: {kind, shape, category, codebook, sections {key: [offset, nbytes,
dtype]}, ...}} with kind

    fixed   bits; sections packed (uint8, zero-padded to 16 bytes + 16)
    split   n_chunks; sections cwords, row_off (int32), raw (uint8),
            lut (int32), lengths (uint8)
    stream  total_bits, stage_words; sections words (int32), chunk_off
            (int64), sub_len (int16), lengths (uint8)
    dense   no codebook; section data (the tensor's own dtype)
"""
from __future__ import annotations

import json
import os
import struct
import time
from typing import Dict, Optional, Tuple

import numpy as np
import torch

import device_formats as dfm

MAGIC = b"CBQIMG01"
ALIGN = 4096
VERSION = 1
_DTYPES = {"uint8": torch.uint8, "int16": torch.int16, "int32": torch.int32,
           "int64": torch.int64, "float32": torch.float32, "bfloat16": torch.bfloat16,
           "float16": torch.float16}


def _align(n: int) -> int:
    return (n + ALIGN - 1) // ALIGN * ALIGN


def _dtype_name(t) -> str:
    if isinstance(t, np.ndarray):
        return np.dtype(t.dtype).name
    return str(t.dtype).replace("torch.", "")


def _sections_of(t) -> Tuple[str, dict, Dict[str, object]]:
    """(kind, scalar fields, {section key: array}) of one device tensor."""
    if isinstance(t, dfm.FixedTensor):
        return "fixed", {"bits": int(t.bits)}, {"packed": t.packed}
    if isinstance(t, dfm.SplitTensor):
        cwords, row_off, raw, lut = t.keep
        return "split", {"n_chunks": int(t.desc.n_chunks)}, {
            "cwords": cwords, "row_off": row_off, "raw": raw, "lut": lut,
            "lengths": np.ascontiguousarray(t.lengths, np.uint8)}
    if isinstance(t, dfm.HuffTensor):
        return "stream", {"total_bits": int(t.total_bits),
                          "stage_words": int(t.tables["stage_words"])}, {
            "words": t.words, "chunk_off": t.chunk_off, "sub_len": t.sub_len,
            "lengths": np.ascontiguousarray(t.lengths, np.uint8)}
    raise TypeError(f"no device-image form for {type(t).__name__}")


def _codebook_of(t) -> torch.Tensor:
    return t.tables["codebook"] if isinstance(t, dfm.HuffTensor) else t.codebook


def _nbytes(a) -> int:
    return int(a.nbytes) if isinstance(a, np.ndarray) else int(a.numel() * a.element_size())


def _host_bytes(a) -> memoryview:
    if isinstance(a, np.ndarray):
        return memoryview(np.ascontiguousarray(a)).cast("B")
    return memoryview(a.detach().contiguous().reshape(-1).view(torch.uint8).cpu().numpy())


def write_image(path, tensors: Dict[str, object], meta: Optional[dict] = None,
                dense: Optional[Dict[str, torch.Tensor]] = None) -> dict:
    """Write `tensors` (FixedTensor / HuffTensor / SplitTensor) to a device
    image at `path`, and `dense` tensors (norm weights and the like) as they
    are; returns the header.  Codebooks are stored once per distinct device
    tensor (or equal contents)."""
    cb_ids: Dict[int, str] = {}
    cb_by_bytes: Dict[bytes, str] = {}
    plan = []                                    # arrays in file order
    off = 0
    header = {"format": "cbq-device-image", "version": VERSION, "meta": meta or {},
              "codebooks": {}, "tensors": {}}
    for name, t in tensors.items():
        cb = _codebook_of(t)
        cid = cb_ids.get(id(cb))
        if cid is None:
            data = cb.detach().float().contiguous().cpu().numpy().tobytes()
            cid = cb_by_bytes.get(data)
            if cid is None:
                cid = f"cb{len(cb_by_bytes)}"
                cb_by_bytes[data] = cid
                header["codebooks"][cid] = {"offset": off, "nbytes": len(data)}
                plan.append(cb)
                off += _align(len(data))
            cb_ids[id(cb)] = cid
        kind, fields, secs = _sections_of(t)
        entry = {"kind": kind, "shape": [int(s) for s in t.shape], "category": t.category,
                 "codebook": cid, **fields, "sections": {}}
        for key, a in secs.items():
            n = _nbytes(a)
            entry["sections"][key] = [off, n, _dtype_name(a)]
            plan.append(a)
            off += _align(n)
        header["tensors"][name] = entry
    for name, a in (dense or {}).items():
        n = _nbytes(a)
        header["tensors"][name] = {"kind": "dense", "shape": [int(x) for x in a.shape],
                                   "sections": {"data": [off, n, _dtype_name(a)]}}
        plan.append(a)
        off += _align(n)
    header["payload_bytes"] = off
    # data_offset depends on the header's own length: settle it by iterating
    data_offset = 0
    while True:
        header["data_offset"] = data_offset
        hb = json.dumps(header, separators=(",", ":")).encode()
        need = _align(16 + len(hb))
        if need == data_offset:
            break
        data_offset = need
    with open(path, "wb") as f:
        f.write(MAGIC + struct.pack("<Q", len(hb)) + hb)
        f.write(b"\0" * (data_offset - 16 - len(hb)))
        for a in plan:
            mv = _host_bytes(a)
            f.write(mv)
            f.write(b"\0" * (_align(len(mv)) - len(mv)))
    return header


def read_header(path) -> dict:
    with open(path, "rb") as f:
        head = f.read(16)
        if len(head) != 16 or head[:8] != MAGIC:
            raise ValueError(f"{path}: not a device image (bad magic)")
        (n,) = struct.unpack("<Q", head[8:])
        if n > (1 << 30):
            raise ValueError(f"{path}: header length {n} out of range")
        h = json.loads(f.read(n).decode())
    if h.get("format") != "cbq-device-image" or h.get("version") != VERSION:
        raise ValueError(f"{path}: unsupported image {h.get('format')} v{h.get('version')}")
    return h


_ELEM = {"uint8": 1, "int16": 2, "int32": 4, "int64": 8, "float32": 4, "bfloat16": 2,
         "float16": 2}


def validate_header(h: dict, file_size: int) -> None:
    """Check an image header against its file and the invariants the kernels
    rely on (the descriptors built from it are trusted by the kernels):
    sections aligned, typed and inside the payload, sized for the tensor's
    shape and format.  Raises ValueError.  The values inside the arrays
    (row offsets, chunk offsets) are checked after upload by load_image."""
    import huffman_codebook as hc
    D, P = int(h.get("data_offset", -1)), int(h.get("payload_bytes", -1))
    if D < 16 or D % ALIGN or P < 0 or P % ALIGN or D + P != file_size:
        raise ValueError(f"image payload [{D}, {D + P}) does not match the file size {file_size}")

    def sec(where, s, dtype=None, at_least=0, exact=None):
        if not (isinstance(s, list) and len(s) == 3):
            raise ValueError(f"{where}: malformed section {s!r}")
        off, n, dt = s
        if dt not in _ELEM or (dtype is not None and dt != dtype):
            raise ValueError(f"{where}: dtype {dt!r}, expected {dtype}")
        if off < 0 or off % ALIGN or n < 0 or n % _ELEM[dt] or off + n > P:
            raise ValueError(f"{where}: section [{off}, {off + n}) outside the payload")
        cnt = n // _ELEM[dt]
        if cnt < at_least or (exact is not None and cnt != exact):
            raise ValueError(f"{where}: {cnt} elements, expected "
                             f"{exact if exact is not None else '>= %d' % at_least}")
        return cnt

    cbn = {}
    for cid, c in h.get("codebooks", {}).items():
        cbn[cid] = sec(f"codebook {cid}", [c.get("offset"), c.get("nbytes"), "float32"],
                       "float32", at_least=1)
    for name, e in h.get("tensors", {}).items():
        kind, shape, s = e.get("kind"), e.get("shape"), e.get("sections", {})
        if kind == "dense":
            cnt = sec(f"{name}.data", s.get("data"))
            if cnt != int(np.prod(shape)):
                raise ValueError(f"{name}: {cnt} values for shape {shape}")
            continue
        if not (isinstance(shape, list) and len(shape) == 2 and min(shape) > 0):
            raise ValueError(f"{name}: bad shape {shape!r}")
        M, K = int(shape[0]), int(shape[1])
        n = M * K
        if e.get("codebook") not in cbn:
            raise ValueError(f"{name}: unknown codebook {e.get('codebook')!r}")
        if kind == "fixed":
            bits = int(e.get("bits", 0))
            if not 1 <= bits <= 16:
                raise ValueError(f"{name}: bits {bits}")
            # the writer pads the stream to 16-byte pieces plus 16 bytes: the
            # streaming kernels load whole 16-byte pieces past the last word
            sec(f"{name}.packed", s.get("packed"), "uint8",
                at_least=((n * bits + 7) // 8 + 15) // 16 * 16 + 16)
        elif kind == "split":
            nch = int(e.get("n_chunks", -1))
            if n % hc.CHUNK_SYMBOLS or nch != n // hc.CHUNK_SYMBOLS:
                raise ValueError(f"{name}: {nch} chunks for {M}x{K}")
            sec(f"{name}.row_off", s.get("row_off"), "int32", exact=nch + 1)
            sec(f"{name}.raw", s.get("raw"), "uint8", exact=n)
            sec(f"{name}.lut", s.get("lut"), "int32", exact=1 << 14)
            sec(f"{name}.cwords", s.get("cwords"), "int32", at_least=3 * hc.SUB_SYMBOLS)
            sec(f"{name}.lengths", s.get("lengths"), "uint8", at_least=1)
        elif kind == "stream":
            tb = int(e.get("total_bits", -1))
            sec(f"{name}.chunk_off", s.get("chunk_off"), "int64",
                exact=(n + hc.CHUNK_SYMBOLS - 1) // hc.CHUNK_SYMBOLS + 1)
            sec(f"{name}.sub_len", s.get("sub_len"), "int16",
                exact=(n + hc.SUB_SYMBOLS - 1) // hc.SUB_SYMBOLS)
            sec(f"{name}.words", s.get("words"), "int32", at_least=max(tb, 0) // 32 + 2)
            nl = sec(f"{name}.lengths", s.get("lengths"), "uint8", at_least=1)
            if tb < 0 or nl > cbn[e["codebook"]] + (1 << 16):
                raise ValueError(f"{name}: total_bits {tb}, {nl} code lengths")
        else:
            raise ValueError(f"{name}: unknown kind {kind!r}")


def _host_array(path, h: dict, off: int, n: int, dtype) -> np.ndarray:
    with open(path, "rb") as f:
        f.seek(h["data_offset"] + off)
        return np.frombuffer(f.read(n), dtype=dtype).copy()


def load_image(path, device="cuda", threads: int = 8, chunk_mb: int = 64):
    """Every tensor of the image, in HBM on `device` -> (tensors, header,
    stats).  The payload is one device allocation filled by
    cbq_file_upload; tensors are views into it (kept alive by them).
    stats: upload seconds, total seconds, bytes and upload GB/s."""
    import cbq_native as nat
    import huffman_codebook as hc
    t0 = time.perf_counter()
    h = read_header(path)
    dev = torch.device(device)
    total = int(h["payload_bytes"])
    validate_header(h, os.path.getsize(path))
    buf = torch.empty(max(total, 1), dtype=torch.uint8, device=dev)
    # the allocation may reuse memory that queued work still touches: the
    # upload's own streams must not overtake it
    torch.cuda.synchronize(dev)
    n_copy = total
    t1 = time.perf_counter()
    part = (nat.UploadPart * 1)(nat.UploadPart(h["data_offset"], n_copy, buf.data_ptr()))
    with torch.cuda.device(dev):
        nat.check(nat.load().cbq_file_upload(os.fsencode(str(path)), part, 1,
                                             int(chunk_mb) << 20, int(threads)),
                  "cbq_file_upload")
    t2 = time.perf_counter()

    def view(sec):
        off, n, dt = sec
        return buf[off:off + n].view(_DTYPES[dt])

    cbs = {cid: buf[c["offset"]:c["offset"] + c["nbytes"]].view(torch.float32)
           for cid, c in h["codebooks"].items()}
    out: Dict[str, object] = {}
    checks = []                                    # (name, device bool) of the array values
    for name, e in h["tensors"].items():
        shape = tuple(e["shape"])
        s = e["sections"]
        if e["kind"] == "dense":
            out[name] = view(s["data"]).reshape(shape)
            continue
        cb = cbs[e["codebook"]]
        if e["kind"] == "fixed":
            out[name] = dfm.FixedTensor(name, shape, int(e["bits"]), e["category"],
                                        view(s["packed"]), cb)
        elif e["kind"] == "split":
            lengths = _host_array(path, h, s["lengths"][0], s["lengths"][1], np.uint8)
            ro, cw = view(s["row_off"]), view(s["cwords"])
            # rows per chunk in [1, 14] (the kernels' slot), 3 readable rows after
            d = ro[1:] - ro[:-1]
            checks.append((name, (ro[0] == 0) & (d.min() >= 1) & (d.max() <= 14)
                           & ((ro[-1] + 3) * 64 <= cw.numel())))
            out[name] = dfm.split_from_arrays(name, shape, e["category"], lengths, cw, ro,
                                              view(s["raw"]), view(s["lut"]), cb,
                                              int(e["n_chunks"]))
        elif e["kind"] == "stream":
            lengths = _host_array(path, h, s["lengths"][0], s["lengths"][1], np.uint8)
            t = dfm.HuffTensor(name, shape, e["category"], lengths, view(s["words"]),
                               view(s["chunk_off"]), view(s["sub_len"]), int(e["total_bits"]))
            # chunk offsets from 0 to total_bits, each chunk's sub-block
            # lengths adding up to it, the words covering the stream
            co, sl = t.chunk_off, t.sub_len.to(torch.int64) & 0xFFFF
            nch = co.numel() - 1
            per = torch.zeros(nch * hc.SUB_SYMBOLS, dtype=torch.int64, device=dev)
            per[:sl.numel()] = sl
            per = per.view(nch, hc.SUB_SYMBOLS).sum(1)
            checks.append((name, (co[0] == 0) & (co[-1] == t.total_bits)
                           & (co[1:] - co[:-1] == per).all()
                           & (t.total_bits + 64 <= 32 * t.words.numel())))
            c = h["codebooks"][e["codebook"]]
            t.tables = dfm.huff_tables_host(
                lengths, _host_array(path, h, c["offset"], c["nbytes"], np.float32), cb,
                int(e["stage_words"]), dev)
            out[name] = t
        else:
            raise ValueError(f"{path}: {name} has unknown kind {e['kind']!r}")
    if checks:
        ok = torch.stack([c for _, c in checks]).cpu()
        bad = [n for (n, _), v in zip(checks, ok.tolist()) if not v]
        if bad:
            raise ValueError(f"{path}: inconsistent format arrays in {bad[:4]}")
    t3 = time.perf_counter()
    stats = {"bytes": n_copy, "upload_s": t2 - t1, "total_s": t3 - t0,
             "upload_GB/s": n_copy / max(t2 - t1, 1e-9) / 1e9, "threads": int(threads),
             "chunk_mb": int(chunk_mb)}
    return out, h, stats
