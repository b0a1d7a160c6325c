"""CPU parity oracle for the always-compressed matmul path.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker.  The product path
(codebook-quantization_amd/) never imports it.

Two halves:

* ctypes bindings of ``libcbq_oracle.so`` (``cbq_oracle.c``), the C
  restatement of /root/reference/src/compressed_matmul.c, and of the
  reference's own compiled kernel in ``_ref/`` when that was built, with the
  reference wrapper's calling conventions
  (/root/reference/src/compressed_matmul_cpu.py:279-343, 431-609): pad the
  stream, zero ``out``, walk 256-row chunks.
* numpy / pure-Python restatements of the reference's format producers:
  LSB-first packing (src/bitpack.py:32-157), heap Huffman code lengths
  (src/huffman_codebook.py:42-86), RFC 1951 canonical codes (:89-119), the
  MSB-first stream and row starts (:126-226), the 12-bit GPU LUT (:394-423)
  and slow-path tables (:353-391).

How each part is pinned (tests/test_oracle.py):
  - C kernels: bit-identical to the compiled reference C on the committed
    golden fixtures (tests/golden/), plus dense recomputation.
  - packing: closed form (index i at bits [i*b, (i+1)*b)), nibble-order KAT
    (tests/test_bitpack.py:50-55 of the reference), brute-force bit loops.
  - canonical codes / tables / stream: the hand-derived KAT of
    diagnostics/test_huffman_gpu.py:30-35 (stream D3 93 1B 1B), Kraft
    equality, prefix-freeness, brute-force decode, and decoding by the
    compiled reference C back to the input indices.
  - heap code lengths and the stream encoder: equal to the reference's own
    Python encoder on the fixtures of tests/golden/heap_golden.npz (tied
    large alphabets, the 32-bit cap, one-symbol and empty alphabets, stream
    bytes and tables; tests/test_heap_golden.py), plus optimal cost against
    an independent brute-force / package-merge optimum on small alphabets.
"""
from __future__ import annotations

import ctypes
import heapq
import os
from typing import Dict, Optional, Tuple

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "libcbq_oracle.so")
REF_SO = os.path.join(HERE, "_ref", "libref_compressed_matmul.so")
# the same source built with -march=x86-64-v4 (oracle/Makefile), for hosts with AVX-512
REF_SO_AVX512 = os.path.join(HERE, "_ref", "libref_compressed_matmul_avx512.so")
_AVX512 = ("avx512f", "avx512bw", "avx512cd", "avx512dq", "avx512vl")


def host_has_avx512() -> bool:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("flags"):
                    flags = set(line.split(":", 1)[1].split())
                    return all(x in flags for x in _AVX512)
    except OSError:
        pass
    return False
CHUNK_ROWS = 256          # src/compressed_matmul_cpu.py:276
LUT_BITS = 12             # src/huffman_codebook.py:349
LUT_SIZE = 1 << LUT_BITS

_f32p = ctypes.POINTER(ctypes.c_float)
_u8p = ctypes.POINTER(ctypes.c_uint8)
_u16p = ctypes.POINTER(ctypes.c_uint16)
_i32p = ctypes.POINTER(ctypes.c_int32)
_i64p = ctypes.POINTER(ctypes.c_int64)
_I = ctypes.c_int


def build(ref: bool = True) -> None:
    """Compile libcbq_oracle.so (and _ref/ when the reference tree exists)."""
    import subprocess
    subprocess.check_call(["make", "-s", "-C", HERE, "all" if ref else "oracle"])


def _p(arr, typ):
    return arr.ctypes.data_as(typ)


class _Lib:
    """ctypes view of either library; `names` maps roles to symbol names."""

    def __init__(self, path: str, names: Dict[str, str]):
        self.path = path
        lib = ctypes.CDLL(path)
        self.fixed_rows = getattr(lib, names["fixed_rows"])
        self.fixed_rows.restype = None
        self.fixed_rows.argtypes = [_f32p, _u8p, _f32p, _f32p] + [_I] * 7
        self.huff_rows = getattr(lib, names["huff_rows"])
        self.huff_rows.restype = None
        self.huff_rows.argtypes = [_f32p, _u8p, _u16p, _u8p, _i64p, _i32p, _u16p,
                                   _i64p, _f32p, _f32p] + [_I] * 7
        self.huff_emb = getattr(lib, names["huff_emb"])
        self.huff_emb.restype = None
        self.huff_emb.argtypes = [_i32p, _u8p, _u16p, _u8p, _i64p, _i32p, _u16p,
                                  _i64p, _f32p, _f32p] + [_I] * 4
        self.huff_dec = getattr(lib, names["huff_dec"])
        self.huff_dec.restype = None
        self.huff_dec.argtypes = [_u8p, _u16p, _u8p, _i64p, _i32p, _u16p, _i64p,
                                  _f32p, _f32p] + [_I] * 4
        self.lib = lib


_ORACLE_NAMES = dict(fixed_rows="oracle_fixed_gemv_rows", huff_rows="oracle_huff_gemv_rows",
                     huff_emb="oracle_huff_embedding_rows", huff_dec="oracle_huff_decode_weights")
# Symbol names of the reference's compiled kernel (src/compressed_matmul.c).
_REF_NAMES = dict(fixed_rows="compressed_matmul_f32_chunk", huff_rows="huffman_matmul_f32_chunk",
                  huff_emb="huffman_embedding_f32_rows", huff_dec="huffman_decode_to_weights_f32")

_cache: Dict[str, _Lib] = {}


def lib(kind: str = "oracle") -> _Lib:
    """The restated oracle ('oracle') or the compiled reference ('ref')."""
    if kind not in _cache:
        if kind == "oracle":
            if not os.path.exists(ORACLE_SO):
                build(ref=False)
            _cache[kind] = _Lib(ORACLE_SO, _ORACLE_NAMES)
            extra = _cache[kind].lib
            extra.oracle_fixed_embedding.restype = None
            extra.oracle_fixed_embedding.argtypes = [_i32p, _u8p, _f32p, _f32p] + [_I] * 4
            extra.oracle_unpack_indices.restype = None
            extra.oracle_unpack_indices.argtypes = [_u8p, ctypes.c_int64, _I, _i32p]
            extra.oracle_huff_decode_indices.restype = None
            extra.oracle_huff_decode_indices.argtypes = [_u8p, _u16p, _u8p, _i64p, _i32p,
                                                         _u16p, _i64p, _i32p] + [_I] * 3
        elif kind == "ref":
            if not os.path.exists(REF_SO):
                raise FileNotFoundError(f"{REF_SO} not built (reference tree absent?)")
            _cache[kind] = _Lib(REF_SO, _REF_NAMES)
        elif kind == "ref_native":
            # the wrapper's -march=native as nearly as this gcc builds it:
            # the AVX-512 build on hosts that run it, else the x86-64-v3 one
            path = REF_SO_AVX512 if (host_has_avx512() and os.path.exists(REF_SO_AVX512)) \
                else REF_SO
            if not os.path.exists(path):
                raise FileNotFoundError(f"{path} not built (reference tree absent?)")
            _cache[kind] = _Lib(path, _REF_NAMES)
        else:
            raise ValueError(kind)
    return _cache[kind]


def ref_available() -> bool:
    return os.path.exists(REF_SO)


# ---------------------------------------------------------------------------
# Fixed-width GEMV / embedding (as called by the reference wrapper)
# ---------------------------------------------------------------------------

def fixed_gemv(x, packed, codebook, M, K, bits, C=None, chunk_rows=CHUNK_ROWS,
               kind="oracle", threads: Optional[int] = None):
    """y[T, M] = x[T, K] @ W^T, W = codebook[idx]; restates compressed_matmul
    (src/compressed_matmul_cpu.py:279-343): pads the stream with 2 zero bytes
    when it is exactly ceil(M*K*b/8) long, zeroes out, calls the C kernel per
    `chunk_rows` rows (None = one call over all rows)."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, K)
    cb = np.ascontiguousarray(codebook, dtype=np.float32)
    pk = np.ascontiguousarray(packed, dtype=np.uint8)
    need = (M * K * bits + 7) // 8
    if len(pk) < need + 4:
        if len(pk) < need + 2:
            pk = np.concatenate([pk, np.zeros(2, np.uint8)])
        # The C read is a 4-byte window, one byte past the wrapper's 2-byte pad
        # for b <= 7 (src/compressed_matmul.c:330-347); keep that byte readable.
        pk = np.concatenate([pk, np.zeros(2, np.uint8)])
    T = x.shape[0]
    out = np.zeros((T, M), np.float32)
    C = len(cb) if C is None else int(C)
    L = lib(kind)
    step = M if not chunk_rows else int(chunk_rows)
    with _omp_threads(threads):
        for r in range(0, M, step):
            L.fixed_rows(_p(x, _f32p), _p(pk, _u8p), _p(cb, _f32p), _p(out, _f32p),
                         T, M, K, C, bits, r, min(r + step, M))
    return out


def fixed_gemv_serial(x, packed, codebook, M, K, bits, C=None):
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, K)
    cb = np.ascontiguousarray(codebook, dtype=np.float32)
    pk = np.concatenate([np.asarray(packed, np.uint8), np.zeros(4, np.uint8)])
    out = np.zeros((x.shape[0], M), np.float32)
    f = lib("oracle").lib.oracle_fixed_gemv_serial
    f.restype = None
    f.argtypes = [_f32p, _u8p, _f32p, _f32p] + [_I] * 5
    f(_p(x, _f32p), _p(pk, _u8p), _p(cb, _f32p), _p(out, _f32p), x.shape[0], M, K,
      len(cb) if C is None else int(C), bits)
    return out


def fixed_embedding(ids, packed, codebook, H, bits, C=None):
    """out[t, h] = codebook[min(idx[ids[t]*H + h], C-1)] (float32)."""
    ids = np.ascontiguousarray(ids, dtype=np.int32).reshape(-1)
    cb = np.ascontiguousarray(codebook, dtype=np.float32)
    pk = np.ascontiguousarray(packed, np.uint8)
    if len(ids) and len(pk) < ((int(ids.max()) + 1) * H * bits + 7) // 8 + 4:
        pk = np.concatenate([pk, np.zeros(4, np.uint8)])
    out = np.zeros((len(ids), H), np.float32)
    lib("oracle").lib.oracle_fixed_embedding(
        _p(ids, _i32p), _p(pk, _u8p), _p(cb, _f32p), _p(out, _f32p), len(ids), H,
        len(cb) if C is None else int(C), bits)
    return out


def unpack_indices_c(packed, bits, n):
    pk = np.concatenate([np.asarray(packed, np.uint8), np.zeros(4, np.uint8)])
    out = np.empty(n, np.int32)
    lib("oracle").lib.oracle_unpack_indices(_p(pk, _u8p), n, bits, _p(out, _i32p))
    return out


class _omp_threads:
    """Temporarily set the OpenMP team size for the C calls."""

    def __init__(self, n):
        self.n = n

    def __enter__(self):
        if self.n:
            try:
                gomp = ctypes.CDLL("libgomp.so.1")
                self._get = gomp.omp_get_max_threads()
                gomp.omp_set_num_threads(int(self.n))
                self._gomp = gomp
            except OSError:
                self._gomp = None
        return self

    def __exit__(self, *a):
        if self.n and getattr(self, "_gomp", None) is not None:
            self._gomp.omp_set_num_threads(self._get)


# ---------------------------------------------------------------------------
# Huffman GEMV / embedding / decode (as called by the reference wrapper)
# ---------------------------------------------------------------------------

def huff_cpu_tables(enc: dict) -> dict:
    """The dtype coercion of src/compressed_modules.py:240-249 and
    src/compressed_matmul_cpu.py:431-443 (lut_sym -> uint16 so -1 becomes
    0xFFFF, lut_len -> uint8, +4 zero bytes on the stream)."""
    lens = np.asarray(enc["huff_lengths"], np.uint8)
    mx = int(lens.max()) if lens.size and lens.max() > 0 else 1
    return dict(
        stream=np.concatenate([np.asarray(enc["huff_stream"], np.uint8), np.zeros(4, np.uint8)]),
        lut_sym=np.ascontiguousarray(np.asarray(enc["huff_lut_sym"]).astype(np.uint16)),
        lut_len=np.ascontiguousarray(np.asarray(enc["huff_lut_len"]).astype(np.uint8)),
        sl_first=np.ascontiguousarray(enc["huff_sl_first_code"], np.int64),
        sl_base=np.ascontiguousarray(enc["huff_sl_base_offset"], np.int32),
        sl_sym=np.ascontiguousarray(np.asarray(enc["huff_sl_sym"]).astype(np.uint16)),
        rbs=np.ascontiguousarray(enc["huff_row_bit_starts"], np.int64),
        max_len=mx)


def _tab_args(t):
    return (_p(t["stream"], _u8p), _p(t["lut_sym"], _u16p), _p(t["lut_len"], _u8p),
            _p(t["sl_first"], _i64p), _p(t["sl_base"], _i32p), _p(t["sl_sym"], _u16p),
            _p(t["rbs"], _i64p))


def huff_gemv(x, enc, codebook, M, K, C=None, chunk_rows=CHUNK_ROWS, kind="oracle",
              threads: Optional[int] = None):
    """Restates huffman_matmul (src/compressed_matmul_cpu.py:446-506)."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, K)
    cb = np.ascontiguousarray(codebook, dtype=np.float32)
    t = huff_cpu_tables(enc)
    T = x.shape[0]
    out = np.zeros((T, M), np.float32)
    C = len(cb) if C is None else int(C)
    L = lib(kind)
    step = M if not chunk_rows else int(chunk_rows)
    with _omp_threads(threads):
        for r in range(0, M, step):
            L.huff_rows(_p(x, _f32p), *_tab_args(t), _p(cb, _f32p), _p(out, _f32p),
                        T, M, K, C, r, min(r + step, M), t["max_len"])
    return out


def huff_embedding(ids, enc, codebook, H, C=None, kind="oracle"):
    """Restates huffman_embedding (src/compressed_matmul_cpu.py:509-560)."""
    ids = np.ascontiguousarray(ids, dtype=np.int32).reshape(-1)
    cb = np.ascontiguousarray(codebook, dtype=np.float32)
    t = huff_cpu_tables(enc)
    out = np.zeros((len(ids), H), np.float32)
    lib(kind).huff_emb(_p(ids, _i32p), *_tab_args(t), _p(cb, _f32p), _p(out, _f32p),
                       len(ids), H, len(cb) if C is None else int(C), t["max_len"])
    return out


def huff_decode_weights(enc, codebook, M, K, C=None, kind="oracle"):
    """Restates huffman_decode_weights (src/compressed_matmul_cpu.py:563-609)."""
    cb = np.ascontiguousarray(codebook, dtype=np.float32)
    t = huff_cpu_tables(enc)
    out = np.empty((M, K), np.float32)
    lib(kind).huff_dec(*_tab_args(t), _p(cb, _f32p), _p(out, _f32p), M, K,
                       len(cb) if C is None else int(C), t["max_len"])
    return out


def huff_decode_indices(enc, M, K, kind="oracle"):
    """Bit-exact decoded indices [M, K] (int32).  'oracle' calls the restated
    decoder directly; 'ref' uses the reference's decode-to-weights with an
    identity codebook (exact for indices < 2^24)."""
    if kind == "ref":
        C = 1 << 16
        w = huff_decode_weights(enc, np.arange(C, dtype=np.float32), M, K, C=C, kind="ref")
        return w.astype(np.int32)
    t = huff_cpu_tables(enc)
    out = np.empty((M, K), np.int32)
    lib("oracle").lib.oracle_huff_decode_indices(*_tab_args(t), _p(out, _i32p), M, K,
                                                 t["max_len"])
    return out


# ---------------------------------------------------------------------------
# Fixed-width format (src/bitpack.py)
# ---------------------------------------------------------------------------

def pack_lsb(indices, bits: int) -> np.ndarray:
    """Index i occupies stream bits [i*b, (i+1)*b), stream bit j is bit j%8 of
    byte j//8; exactly ceil(N*b/8) bytes (src/bitpack.py:32-95: 8-bit bytes,
    4-bit low nibble first and 16-bit little-endian are the same layout)."""
    idx = np.asarray(indices).reshape(-1).astype(np.uint32)
    n = idx.size
    nbytes = (n * bits + 7) // 8
    if n == 0:
        return np.zeros(0, np.uint8)
    shifts = np.arange(bits, dtype=np.uint32)
    bitmat = ((idx[:, None] >> shifts[None, :]) & 1).astype(np.uint8).reshape(-1)
    pad = (-bitmat.size) % 8
    if pad:
        bitmat = np.concatenate([bitmat, np.zeros(pad, np.uint8)])
    return np.packbits(bitmat, bitorder="little")[:nbytes]


def unpack_lsb(packed, bits: int, n: int) -> np.ndarray:
    """Inverse of pack_lsb (src/bitpack.py:97-157)."""
    pk = np.asarray(packed, np.uint8)
    need = (n * bits + 7) // 8
    if pk.size < need:
        pk = np.concatenate([pk, np.zeros(need - pk.size, np.uint8)])
    bitarr = np.unpackbits(pk[:need], bitorder="little")[: n * bits].reshape(n, bits)
    weights = (1 << np.arange(bits, dtype=np.uint32))
    return (bitarr.astype(np.uint32) * weights[None, :]).sum(axis=1).astype(np.uint16)


# ---------------------------------------------------------------------------
# Canonical Huffman (src/huffman_codebook.py)
# ---------------------------------------------------------------------------

def heap_code_lengths(freq) -> np.ndarray:
    """Code lengths from a binary heap of (frequency, node id) pairs: leaves
    have id = symbol, merged nodes take ids n, n+1, ... in creation order;
    one active symbol gets length 1; lengths are capped at 32
    (src/huffman_codebook.py:42-86)."""
    freq = np.asarray(freq)
    n = len(freq)
    lengths = np.zeros(n, np.uint8)
    heap = [(int(freq[s]), s) for s in range(n) if freq[s] > 0]
    if not heap:
        return lengths
    if len(heap) == 1:
        lengths[heap[0][1]] = 1
        return lengths
    heapq.heapify(heap)
    parent: Dict[int, int] = {}
    next_id = n
    while len(heap) > 1:
        fa, a = heapq.heappop(heap)
        fb, b = heapq.heappop(heap)
        parent[a] = parent[b] = next_id
        heapq.heappush(heap, (fa + fb, next_id))
        next_id += 1
    root = heap[0][1]
    depth_of: Dict[int, int] = {root: 0}

    def depth(node):
        chain = []
        while node not in depth_of:
            chain.append(node)
            node = parent[node]
        d = depth_of[node]
        for nd in reversed(chain):
            d += 1
            depth_of[nd] = d
        return depth_of[chain[0]] if chain else d

    for s in range(n):
        if freq[s] > 0:
            lengths[s] = min(depth(s), 32)
    return lengths


def canonical_codes(lengths) -> Dict[int, Tuple[int, int]]:
    """RFC 1951 section 3.2.2: codes assigned in (length, symbol) order;
    first code of length L is (first[L-1] + count[L-1]) << 1
    (src/huffman_codebook.py:89-119).  Returns {symbol: (code, length)}."""
    lengths = np.asarray(lengths)
    if lengths.size == 0 or lengths.max() == 0:
        return {}
    mx = int(lengths.max())
    count = np.bincount(lengths[lengths > 0].astype(np.int64), minlength=mx + 1)
    nxt = [0] * (mx + 2)
    code = 0
    for L in range(1, mx + 1):          # count[0] == 0: unused symbols excluded
        code = (code + int(count[L - 1])) << 1
        nxt[L] = code
    out = {}
    for s in range(len(lengths)):
        L = int(lengths[s])
        if L:
            out[s] = (nxt[L], L)
            nxt[L] += 1
    return out


def gpu_lut(lengths) -> Tuple[np.ndarray, np.ndarray]:
    """12-bit table: every 12-bit MSB-first prefix that starts with a code of
    length <= 12 maps to (symbol, length); others (-1, 0)
    (src/huffman_codebook.py:394-423; int32 both)."""
    lut_sym = np.full(LUT_SIZE, -1, np.int32)
    lut_len = np.zeros(LUT_SIZE, np.int32)
    for s, (code, L) in canonical_codes(lengths).items():
        if L <= LUT_BITS:
            lo = code << (LUT_BITS - L)
            hi = lo + (1 << (LUT_BITS - L))
            lut_sym[lo:hi] = s
            lut_len[lo:hi] = L
    return lut_sym, lut_len


def slow_tables(lengths):
    """For lengths > 12: first canonical code per length (-1 if none), the
    offset of each length's symbols in sl_sym, sentinel at [max+1]; sl_sym in
    code order, [0] when empty (src/huffman_codebook.py:353-391)."""
    lengths = np.asarray(lengths)
    mx = int(lengths.max()) if lengths.size and lengths.max() > 0 else LUT_BITS
    first = np.full(mx + 2, -1, np.int64)
    base = np.zeros(mx + 2, np.int32)
    by_len: Dict[int, list] = {}
    for s, (code, L) in canonical_codes(lengths).items():
        if L > LUT_BITS:
            by_len.setdefault(L, []).append((code, s))
    syms = []
    for L in range(LUT_BITS + 1, mx + 1):
        base[L] = len(syms)
        if L in by_len:
            group = sorted(by_len[L])
            first[L] = group[0][0]
            syms.extend(s for _, s in group)
    base[mx + 1] = len(syms)
    return first, base, np.array(syms if syms else [0], np.int32)


def huffman_encode(indices, shape=None, lengths=None) -> dict:
    """Stream of canonical codes, MSB-first in each byte, exactly
    ceil(bits/8) bytes then 4 zero bytes; alphabet 0..max(idx); with a 2-D
    shape also row starts (bit start of symbol r*K) and the GPU tables
    (src/huffman_codebook.py:126-226).  `lengths` overrides the heap
    lengths (used to feed length-limited codes through the same encoder)."""
    idx = np.asarray(indices).reshape(-1).astype(np.int64)
    n = idx.size
    C = int(idx.max()) + 1 if n else 1
    if lengths is None:
        lengths = heap_code_lengths(np.bincount(idx, minlength=C))
    lengths = np.asarray(lengths, np.uint8)
    codes = canonical_codes(lengths)
    code_of = np.zeros(len(lengths), np.uint64)
    len_of = np.zeros(len(lengths), np.int64)
    for s, (c, L) in codes.items():
        code_of[s] = c
        len_of[s] = L
    lens = len_of[idx]
    starts = np.zeros(n, np.int64)
    if n:
        starts[1:] = np.cumsum(lens[:-1])
    total = int(starts[-1] + lens[-1]) if n else 0
    bitarr = np.zeros(total + 8, np.uint8)
    mxl = int(lens.max()) if n else 0
    cv = code_of[idx]
    for b in range(mxl):
        sel = lens > b
        pos = starts[sel] + b
        sh = (lens[sel] - 1 - b).astype(np.uint64)
        bitarr[pos] = ((cv[sel] >> sh) & np.uint64(1)).astype(np.uint8)
    nbytes = (total + 7) // 8
    stream = np.concatenate([np.packbits(bitarr)[:nbytes], np.zeros(4, np.uint8)])
    out = {"huff_lengths": lengths, "huff_stream": stream,
           "huff_n": np.array([n], np.int64)}
    if shape is not None and len(shape) == 2:
        M, K = int(shape[0]), int(shape[1])
        if n and M * K == n:
            out["huff_row_bit_starts"] = starts[::K].astype(np.int64)
        else:
            out["huff_row_bit_starts"] = np.zeros(max(M, 1), np.int64)
        out["huff_lut_sym"], out["huff_lut_len"] = gpu_lut(lengths)
        (out["huff_sl_first_code"], out["huff_sl_base_offset"],
         out["huff_sl_sym"]) = slow_tables(lengths)
    return out


def huffman_decode_bitserial(stream, lengths, n) -> np.ndarray:
    """Independent decoder: read one bit at a time and look the (code,
    length) pair up in the inverse canonical map; no LUTs.  Small n only."""
    inv = {(c, L): s for s, (c, L) in canonical_codes(lengths).items()}
    bits = np.unpackbits(np.asarray(stream, np.uint8))
    out = np.zeros(n, np.int32)
    pos = 0
    mx = int(np.asarray(lengths).max()) if len(lengths) else 0
    for i in range(n):
        code = 0
        for L in range(1, mx + 1):
            code = (code << 1) | int(bits[pos + L - 1])
            if (code, L) in inv:
                out[i] = inv[(code, L)]
                pos += L
                break
        else:
            out[i] = 0
            pos += 1
    return out
