#!/usr/bin/env python3
"""Compressed-GEMV benchmark on one MI355X.

A step is one batch-1 pass over every linear weight of a random-init
36-layer Qwen3-8B-shape decoder (q/k/v/o/gate/up/down x 36 + lm_head), i.e.
the weight stream of one decode token, with the weights held as lossless
13-bit codebook indices (per-category shared, frequency-sorted codebooks)
and x resident in HBM.  The launches are the decoder's: per layer the q/k/v
rows stacked into one matrix and gate/up into one (same codebook, so the
packed streams concatenate exactly), o and down, then the lm_head: 145
launches, captured once into a HIP graph and replayed.

value = algorithmic compressed bytes per step / step time (GB/s).  "roofline"
is the dominant kernel (the stacked gate+up GEMV): algorithmic bytes per
launch / its mean launch time from HIP events around back-to-back launches
over all 36 layers' distinct weights (so the 256 MB MALL cannot serve
repeats).  Further keys:

- "breakdown": every unstacked 9B shape timed the same way;
- "batch_stacked_gate_up": the stacked gate+up launch with 2..16 tokens;
- "huffman": the same sweep with canonical-Huffman weights held in the split
  format alone (the decoder's format; each matrix's stream is decoded on the
  GPU, re-encoded and freed), with its resident bits per weight;
- "qwen3_1_7b": benchmark configs 2 and 3, the 28-layer 1.7B shapes at 1, 4
  and 16 tokens, fixed-width and Huffman;
- "prefill": the bf16 MFMA GEMM at T = 512 and 2048 (config 4);
- "e2e": greedy decode of the whole 36-layer model (config 5), both encodings,
  tokens checked against the CPU oracle's golden run when the prompt matches;
- "cpu_baseline": the reference's own C kernels (oracle/_ref, compiled from
  src/compressed_matmul.c) on config 1 on the host cores.
"""
import os

# The CPU baseline's OpenMP team binds to neighbouring cores; set before any
# OpenMP runtime is loaded (torch loads one).
os.environ.setdefault("OMP_PROC_BIND", "close")
# threads this process may run on, read before any OpenMP runtime binds the
# main thread to one core (OMP_PROC_BIND=close does, once it starts)
try:
    USABLE_THREADS = len(os.sched_getaffinity(0))
except (AttributeError, OSError):
    USABLE_THREADS = None

import argparse  # noqa: E402
import json  # noqa: E402
import re  # noqa: E402
import sys  # noqa: E402
import time  # noqa: E402

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "codebook-quantization_amd"))

METRIC = "compressed GEMV HBM GB/s (% of peak) + decode tok/s, batch 1, 9B-scale shapes"
HBM_PEAK_GBPS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0      # MI355X dense bf16
GOLDEN_E2E = os.path.join(ROOT, "tests", "golden", "e2e_qwen3_8b_golden.npz")


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


class mark:
    """A named range around a bench section (roctx through torch.cuda.nvtx),
    so a `rocprofv3 --kernel-trace --marker-trace` run attributes every
    kernel dispatch to the section that launched it."""

    def __init__(self, name):
        self.name = name

    def __enter__(self):
        import torch
        torch.cuda.nvtx.range_push("bench:" + self.name)
        return self

    def __exit__(self, *exc):
        import torch
        torch.cuda.nvtx.range_pop()
        return False


def fixed_bytes(M, K, bits, C, T=1):
    return (M * K * bits + 7) // 8 + 4 * C + T * K * 4 + T * M * 4


def timed_graph(torch, fn, reps, warmup):
    """Capture fn() into a graph; return mean ms per replay (HIP events on
    the replay stream) over `reps` replays after `warmup` replays."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()                                    # eager warm-up outside capture
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    st = torch.cuda.current_stream()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(st)
    for _ in range(reps):
        g.replay()
    e1.record(st)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps, g


PREFILL_PROFILE = "fixed_prefill_kernel_qwen3-8b_T512_T2048.md"


def read_profile_value(name, pattern, scale=1.0):
    """A figure from a committed rocprofv3 summary, if any."""
    p = os.path.join(ROOT, "profiles", name)
    if not os.path.exists(p):
        return None
    m = re.search(pattern, open(p).read())
    return round(float(m.group(1)) * scale, 4) if m else None


def read_traffic(name):
    """HBM bytes per launch from a committed rocprofv3 PMC summary, if any."""
    p = os.path.join(ROOT, "profiles", name)
    if not os.path.exists(p):
        return None
    m = re.search(r"traffic_bytes_per_launch:\s*([0-9.eE+]+)", open(p).read())
    return float(m.group(1)) if m else None


# ---- decoder launch lists ----------------------------------------------------

def step_plan(dec, with_head=True):
    """The decoder's launches for one token: per layer the stacked q/k/v,
    o, the stacked gate/up and down; then the lm_head.  Entries are a
    name or a tuple of part names (one stacked / grouped launch)."""
    plan = []
    for i in range(dec.cfg["layers"]):
        p = f"model.layers.{i}."
        plan.append(tuple(p + n for n in ("self_attn.q_proj", "self_attn.k_proj",
                                          "self_attn.v_proj")))
        plan.append(p + "self_attn.o_proj")
        plan.append(tuple(p + n for n in ("mlp.gate_proj", "mlp.up_proj")))
        plan.append(p + "mlp.down_proj")
    if with_head:
        plan.append("lm_head")
    return plan


def fixed_launches(torch, nat, lib, dev, synthetic, fixed, plan):
    """(launch list, outputs) of a step plan over fixed-width tensors, the
    stacked parts concatenated into one matrix (synthetic.stack_fixed)."""
    mats = []
    for e in plan:
        if isinstance(e, tuple):
            st = synthetic.stack_fixed([fixed[n] for n in e], e[0] + "+stacked")
            if st is None:
                mats += [fixed[n] for n in e]
            else:
                mats.append(st)
        else:
            mats.append(fixed[e])
    return mats


def run_fixed(torch, nat, lib, dev, mats, xs, outs, T=1):
    st = nat.stream_ptr(dev)
    for t in mats:
        M, K = t.shape
        rc = lib.ck_linear_f32(xs[K].data_ptr(), t.packed.data_ptr(), t.codebook.data_ptr(),
                               outs[id(t)].data_ptr(), T, M, K, t.codebook.numel(), t.bits, st)
        if rc:
            raise RuntimeError(f"ck_linear_f32 rc={rc} on {t.name}")


def fixed_sweep(torch, nat, lib, dev, mats, T, steps, warmup):
    """Graph-replayed step over `mats` with T tokens -> (ms, algorithmic bytes)."""
    xs, outs = {}, {}
    for t in mats:
        M, K = t.shape
        if K not in xs:
            xs[K] = torch.randn(T, K, device=dev)
        outs[id(t)] = torch.empty(T, M, device=dev)
    ms, _ = timed_graph(torch, lambda: run_fixed(torch, nat, lib, dev, mats, xs, outs, T),
                        steps, warmup)
    nbytes = sum(fixed_bytes(t.shape[0], t.shape[1], t.bits, t.codebook.numel(), T)
                 for t in mats)
    return ms, nbytes


# ---- Huffman: split format only ------------------------------------------------

def build_split_formats(torch, dev, huff, names):
    """The split format of every Huffman tensor in `names`, decoded from its
    stream on the GPU; the stream is then dropped (the split format is the
    matrix's only resident format).  Returns {name: (keep, desc)} and the
    streams' byte counts (reference stream + chunk index)."""
    from gpu_huffman_functions import build_split, decode_symbols, split_eligible
    splits, stream_bytes = {}, {}
    for n in names:
        t = huff[n]
        M, K = t.shape
        stream_bytes[n] = t.nbytes
        if split_eligible(M, K):
            idx = decode_symbols(t.words, t.chunk_off, t.sub_len, t.lengths, M * K, dev)
            sp = build_split(idx, t.tables["codebook"].cpu().numpy(), dev)
            del idx
            if sp is not None:
                splits[n] = sp
                t.words = t.chunk_off = t.sub_len = None     # stream freed
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return splits, stream_bytes


def stack_gate_up(torch, dev, huff, splits, plan):
    """Every layer's gate/up pair re-coded as one stacked split matrix under
    a shared table (the decoder's format for the gate/up launch with the SiLU
    epilogue); the pair's entries in `splits` become descriptors into it and
    the stacked pair is stored under ("glu", gate name)."""
    import numpy as np
    from gpu_huffman_functions import stack_split
    for e in plan:
        if not (isinstance(e, tuple) and e[0].endswith("mlp.gate_proj")):
            continue
        g, u = e
        M, K = huff[g].shape
        cb = huff[g].tables["codebook"].cpu().numpy()
        if K % 4096 or huff[u].shape != (M, K) or g not in splits or u not in splits or \
                not np.array_equal(cb, huff[u].tables["codebook"].cpu().numpy()):
            continue
        st = stack_split([splits[g], splits[u]], cb, [M, M], K, dev)
        if st is None:
            continue
        keep, sdesc, parts = st
        splits[g], splits[u] = (keep, parts[0]), (keep, parts[1])
        splits[("glu", g)] = (keep, sdesc)
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


def stream_gate_up(torch, nat, lib, dev, huff, plan, steps, warmup, layers=8):
    """The config-3 stream format's fused kernel (cbq_huff_linear_f32, T = 1)
    on the gate and up matrices of the first `layers` layers, before their
    streams are freed: mean us per matrix launch and GB/s on the stream's
    bytes (stream + chunk offsets + sub-block lengths + x + y)."""
    import ctypes
    pairs = [e for e in plan if isinstance(e, tuple) and e[0].endswith("mlp.gate_proj")][:layers]
    mats = [n for e in pairs for n in e]
    descs, outs = {}, {}
    for n in mats:
        t = huff[n]
        tb = t.tables
        descs[n] = nat.HuffStream(words=t.words.data_ptr(), n_words=t.words.numel(),
                                  chunk_off=t.chunk_off.data_ptr(), sub_len=t.sub_len.data_ptr(),
                                  lut1=tb["lut1"].data_ptr(), lut2=tb["lut2"].data_ptr(),
                                  n_lut2=tb["lut2"].numel(), canon=tb["canon"].data_ptr(),
                                  canon_pay=tb["pay"].data_ptr(), value_cb=None,
                                  C=tb["codebook"].numel(), stage_words=tb["stage_words"])
        outs[n] = torch.empty(1, t.shape[0], device=dev)
    K = huff[mats[0]].shape[1]
    x = torch.randn(1, K, device=dev)

    def run():
        for n in mats:
            M = huff[n].shape[0]
            rc = lib.cbq_huff_linear_f32(x.data_ptr(), ctypes.byref(descs[n]), outs[n].data_ptr(),
                                         1, M, K, nat.stream_ptr(dev))
            if rc:
                raise RuntimeError(f"cbq_huff_linear_f32 rc={rc}")
    ms, _ = timed_graph(torch, run, steps, warmup)
    nb = sum(huff[n].nbytes + 4 * K + 4 * huff[n].shape[0] for n in mats)
    us = ms * 1e3 / len(mats)
    return {"kernel": "cbq_huff_linear_f32 (stream format, huff_tile_fast_kernel), gate or up "
                      f"{K}->{huff[mats[0]].shape[0]}",
            "us_per_launch": round(us, 2), "bytes_per_launch": nb // len(mats),
            "GB/s": round(nb / (ms * 1e-3) / 1e9, 1),
            "frac": round(nb / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4), "matrices": len(mats)}


def split_launch_args(nat, splits, huff, ns, outs):
    import ctypes
    k = len(ns)
    return (k, (ctypes.POINTER(nat.SplitMatrix) * k)(*[ctypes.pointer(splits[n][1]) for n in ns]),
            (ctypes.c_void_p * k)(*[outs[n].data_ptr() for n in ns]),
            (ctypes.c_int * k)(*[huff[n].shape[0] for n in ns]), huff[ns[0]].shape[1])


def huffman_sweep(torch, nat, lib, dev, huff, splits, plan, steps, warmup):
    """Graph-replayed split-format step (grouped q/k/v and gate/up) ->
    (ms, bytes the kernels stream, per-launch args)."""
    import ctypes
    from gpu_huffman_functions import split_bytes
    outs, xs, launches = {}, {}, []
    nbytes = 0
    for e in plan:
        ns = list(e) if isinstance(e, tuple) else [e]
        missing = [n for n in ns if n not in splits]
        if missing:
            raise RuntimeError(f"no split format for {missing}")
        M, K = huff[ns[0]].shape
        if K not in xs:
            xs[K] = torch.randn(1, K, device=dev)
        glu = splits.get(("glu", ns[0])) if len(ns) == 2 else None
        if glu is not None:                       # gate/up: one launch, SiLU in the epilogue
            out = torch.empty(1, M, device=dev)
            outs[ns[0]] = out
            launches.append(("glu", glu, out, M, K))
            nbytes += split_bytes(glu[0]) + 4 * M + 4 * K
            continue
        for n in ns:
            outs[n] = torch.empty(1, huff[n].shape[0], device=dev)
        launches.append(("split",) + split_launch_args(nat, splits, huff, ns, outs))
        keeps = {id(splits[n][0]): splits[n][0] for n in ns}
        nbytes += sum(split_bytes(k) for k in keeps.values())
        nbytes += sum(4 * huff[n].shape[0] for n in ns) + 4 * K

    def run():
        for a in launches:
            if a[0] == "glu":
                _, glu, out, M, K = a
                rc = lib.cbq_split_linear_glu_f32(xs[K].data_ptr(), None, None, 0, 0.0,
                                                  ctypes.byref(glu[1]), out.data_ptr(), M, K,
                                                  nat.stream_ptr(dev))
            else:
                _, k, mats, out_a, m_a, K = a
                rc = lib.cbq_split_linear_f32(xs[K].data_ptr(), None, None, 0, 0.0, k, mats,
                                              out_a, m_a, K, nat.stream_ptr(dev))
            if rc:
                raise RuntimeError(f"split GEMV rc={rc}")
    ms, _ = timed_graph(torch, run, steps, warmup)
    return ms, nbytes


# ---- sections ------------------------------------------------------------------

def xf_bytes(T, K):
    """Bytes of the fragment-order copy of x at the front of the
    cbq_linear_bf16_ws workspace (the rest holds split-K partials: whole
    small grids, or the tiles left after the last full round of CUs)."""
    return ((T + 15) // 16 * 16 * K * 2 + 255) // 256 * 256


def prefill_section(torch, nat, lib, dev, fixed, kinds, args):
    """benchmark config 4: bf16 MFMA prefill over the same fixed-width weights,
    T = 512 and 2048 tokens of bf16 N(0, 1) activations; per shape the mean
    time of one cbq_linear_bf16_ws call (the x fragment-order copy, the GEMM
    and, when K is split, the partial sum) over 8 layers' distinct weights
    (graph-replayed)."""
    out = {"peak_tflops": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s", "shapes": {}}
    for T in (512, 2048):
        for kind in ("q_proj", "k_proj", "gate_proj", "down_proj"):
            ns = kinds[kind][:8]
            t0 = fixed[ns[0]]
            M, K = t0.shape
            x = torch.randn(T, K, device=dev).bfloat16()
            o = torch.empty(T, M, device=dev, dtype=torch.bfloat16)
            nws = int(lib.cbq_linear_bf16_workspace(T, M, K))
            ws = torch.empty(max(1, nws // 4), dtype=torch.float32, device=dev)

            def run(ns=ns, x=x, o=o, ws=ws, nws=nws):
                st = nat.stream_ptr(dev)
                for n in ns:
                    t = fixed[n]
                    rc = lib.cbq_linear_bf16_ws(x.data_ptr(), t.packed.data_ptr(),
                                                t.codebook.data_ptr(), o.data_ptr(), T, M, K,
                                                t.codebook.numel(), t.bits, ws.data_ptr(), nws, st)
                    if rc:
                        raise RuntimeError(f"cbq_linear_bf16_ws rc={rc} on {n}")
            ms, _ = timed_graph(torch, run, max(2, args.steps // 4), 1)
            us = ms * 1e3 / len(ns)
            tf = 2.0 * T * M * K / (us * 1e-6) / 1e12
            out["shapes"][f"T{T}_{kind}"] = {"shape": f"{K}->{M}", "us_per_launch": round(us, 1),
                                             "split_partials_MB": round((nws - xf_bytes(T, K)) / 1e6, 1),
                                             "TFLOP/s": round(tf, 1),
                                             "frac": round(tf / MFMA_BF16_PEAK_TFLOPS, 4)}
    g = out["shapes"]["T2048_gate_proj"]
    out["roofline"] = {"bound": "mfma", "achieved": g["TFLOP/s"], "peak": MFMA_BF16_PEAK_TFLOPS,
                       "unit": "TFLOP/s", "frac": g["frac"],
                       "kernel": "fixed_prefill_kernel<13> gate/up 4096->12288, T=2048",
                       "mfma_busy_rocprof_full_round_launch": read_profile_value(
                           PREFILL_PROFILE, r"\*\*MFMA busy ([0-9.]+) %\*\*", 0.01),
                       "profile": "profiles/" + PREFILL_PROFILE}
    return out


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_ids():
    """Family / model / stepping numbers of the host CPU (a virtualised host
    may report only a generic model name; the numbers still give the core
    generation) and the threads this process may run on."""
    out = {}
    try:
        for line in open("/proc/cpuinfo"):
            k, _, v = line.partition(":")
            k = k.strip()
            if k in ("cpu family", "model", "stepping", "cache size") and k not in out:
                out[k] = v.strip()
            if not line.strip() and out:
                break
    except OSError:
        pass
    out["logical_cpus"] = os.cpu_count()
    if USABLE_THREADS is not None:
        out["usable_threads_at_start"] = USABLE_THREADS
    return out


def config5_cpu_record():
    """Config 5 on the CPU: the golden run's own timing (the 36-layer model
    decoded by oracle/cpu_decoder.py with every GEMV on the reference's
    compiled C kernel, tests/golden/gen_e2e_full_golden.py), recorded beside
    the fixture.  Measured on the host that generated the fixture, not on the
    GPU box (the run takes ~35 minutes)."""
    path = os.path.join(ROOT, "tests", "golden", "e2e_qwen3_8b_cpu_timing.json")
    try:
        with open(path) as f:
            return json.load(f)
    except (OSError, ValueError):
        return None


def cpu_baseline(np, seconds):
    """benchmark config 1 on the host cores with the reference's own C kernels
    (oracle/_ref; the restatement when that is not built): W [6144, 2048]
    N(0, 0.02) bf16 (synthetic.make_bf16, seed "config1"), frequency-sorted
    lossless codebook, 13-bit fixed-width indices and the canonical-Huffman
    stream of the same indices; T = 1, 4, 16; each timed as the reference
    wrapper calls it (256-row chunks, stream copied to pad it every call,
    src/compressed_matmul_cpu.py:276-343, 446-507) and as one call over all
    rows (tables prepared once).  Median of >= 7 runs after one warm-up, with
    the box's CPU share of OpenMP threads bound close.  GB/s on the same
    algorithmic bytes as the GPU figures."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import cbq_oracle as O
    import codebook_builder as cbb
    import huffman_codebook as hc
    import synthetic
    kind = "reference" if O.ref_available() else "port"
    lk = "ref_native" if kind == "reference" else "oracle"
    threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or min(16, os.cpu_count() or 1)
    threads = min(threads, os.cpu_count() or threads)
    M, K = 6144, 2048
    w = synthetic.make_bf16((M, K), "config1", device="cpu").float().numpy()
    cb, idx = cbb.frequency_sorted_codebook(w)
    bits = cbb.bits_for(len(cb))
    import bitpack
    packed = bitpack.pack_any_bits(idx, bits)
    enc = hc.huffman_encode_indices(idx, shape=(M, K))
    C = len(cb)
    L = O.lib(lk)
    march = "x86-64-v4 (AVX-512)" if L.path.endswith("_avx512.so") else "x86-64-v3 (AVX2+FMA)"
    pk_pad = np.concatenate([packed, np.zeros(4, np.uint8)])
    tabs = O.huff_cpu_tables(enc)
    stream_b = len(enc["huff_stream"])
    rng = np.random.default_rng(1)
    budget = max(1.0, seconds) / 12.0                  # per (mode, encoding, T) cell
    res = {}

    def timed(fn):
        fn()
        ts = []
        t_end = time.perf_counter() + budget
        while len(ts) < 7 or (time.perf_counter() < t_end and len(ts) < 200):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        return float(np.median(ts)), len(ts)

    for T in (1, 4, 16):
        x = rng.standard_normal((T, K)).astype(np.float32)
        out = np.zeros((T, M), np.float32)
        fb = fixed_bytes(M, K, bits, C, T)
        hb = stream_b + 8 * M + 4 * C + T * K * 4 + T * M * 4   # + row starts (reference tables)

        def fixed_single():
            out[:] = 0
            with O._omp_threads(threads):
                L.fixed_rows(O._p(x, O._f32p), O._p(pk_pad, O._u8p), O._p(cb, O._f32p),
                             O._p(out, O._f32p), T, M, K, C, bits, 0, M)

        def huff_single():
            out[:] = 0
            with O._omp_threads(threads):
                L.huff_rows(O._p(x, O._f32p), *O._tab_args(tabs), O._p(cb, O._f32p),
                            O._p(out, O._f32p), T, M, K, C, 0, M, tabs["max_len"])

        cells = {
            "fixed_single": (fixed_single, fb),
            "fixed_as_called": (lambda: O.fixed_gemv(x, packed, cb, M, K, bits, kind=lk,
                                                     chunk_rows=256, threads=threads), fb),
            "huffman_single": (huff_single, hb),
            "huffman_as_called": (lambda: O.huff_gemv(x, enc, cb, M, K, kind=lk, chunk_rows=256,
                                                      threads=threads), hb),
        }
        for name, (fn, nb) in cells.items():
            med, n = timed(fn)
            res[f"T{T}_{name}"] = {"ms": round(med * 1e3, 3), "GB/s": round(nb / med / 1e9, 3),
                                   "runs": n}
    # configs 2 / 3: every distinct linear shape of the 28-layer 1.7B decoder
    # at T = 1, 4, 16, one call over all rows, fixed width and Huffman; the
    # per-step figure sums a layer's seven linears x 28
    shapes = {"q_o": (2048, 2048), "k_v": (1024, 2048), "gate_up": (6144, 2048),
              "down": (2048, 6144)}
    per_layer = {"q_o": 2, "k_v": 2, "gate_up": 2, "down": 1}
    budget = max(0.2, seconds / 60.0)
    small = {}
    for sname, (Ms, Ks) in shapes.items():
        ws = w if (Ms, Ks) == (M, K) else \
            synthetic.make_bf16((Ms, Ks), f"config2.{sname}", device="cpu").float().numpy()
        cbs, idxs = cbb.frequency_sorted_codebook(ws)
        bs = cbb.bits_for(len(cbs))
        pks = np.concatenate([bitpack.pack_any_bits(idxs, bs), np.zeros(4, np.uint8)])
        encs = hc.huffman_encode_indices(idxs, shape=(Ms, Ks))
        tbs = O.huff_cpu_tables(encs)
        Cs = len(cbs)
        for T in (1, 4, 16):
            x = rng.standard_normal((T, Ks)).astype(np.float32)
            out = np.zeros((T, Ms), np.float32)

            def fx():
                out[:] = 0
                with O._omp_threads(threads):
                    L.fixed_rows(O._p(x, O._f32p), O._p(pks, O._u8p), O._p(cbs, O._f32p),
                                 O._p(out, O._f32p), T, Ms, Ks, Cs, bs, 0, Ms)

            def hf():
                out[:] = 0
                with O._omp_threads(threads):
                    L.huff_rows(O._p(x, O._f32p), *O._tab_args(tbs), O._p(cbs, O._f32p),
                                O._p(out, O._f32p), T, Ms, Ks, Cs, 0, Ms, tbs["max_len"])
            for enc_name, fn in (("fixed", fx), ("huffman", hf)):
                fn()
                ts = []
                t_end = time.perf_counter() + budget
                while len(ts) < 3 or (time.perf_counter() < t_end and len(ts) < 50):
                    t0 = time.perf_counter()
                    fn()
                    ts.append(time.perf_counter() - t0)
                small[f"{sname}_T{T}_{enc_name}"] = round(float(np.median(ts)) * 1e3, 3)
    steps = {}
    for enc_name in ("fixed", "huffman"):
        for T in (1, 4, 16):
            ms = 28 * sum(n * small[f"{k}_T{T}_{enc_name}"] for k, n in per_layer.items())
            steps[f"{enc_name}_T{T}"] = {"ms_per_step": round(ms, 1),
                                         "tok_per_s": round(1000.0 * T / ms, 2)}
    res["qwen3_1_7b_linears_ms"] = small
    res["qwen3_1_7b_steps"] = steps
    head = res["T1_fixed_single"]
    return {"value": head["GB/s"], "unit": "GB/s", "cores": threads, "kind": kind,
            "sample": (f"config 1 (K={K} -> M={M}, 13-bit fixed width, T=1): one call over all "
                       f"rows of src/compressed_matmul.c compressed_matmul_f32_chunk "
                       f"(gcc -O3 -march={march.split()[0]} -fopenmp, {threads} threads, OMP_PROC_BIND="
                       f"{os.environ.get('OMP_PROC_BIND')}), median of {head['runs']} runs = "
                       f"{head['ms']} ms on {cpu_model()}; every mode, encoding and T in "
                       f"cpu_baseline_detail")}, \
        {"cpu": cpu_model(), "cpu_ids": cpu_ids(), "threads": threads, "omp_proc_bind": os.environ.get("OMP_PROC_BIND"),
         "kind": kind, "march": march,
         "march_note": "the reference wrapper builds with -march=native "
                       "(src/compressed_matmul_cpu.py:88-91); gcc 11 here has no znver5 target, "
                       "so AVX-512 hosts run the x86-64-v4 build and others the x86-64-v3 one",
         "codebook": C, "bits": bits,
         "config5_cpu_decode": config5_cpu_record(),
         "huffman_bits_per_weight": round(8.0 * stream_b / (M * K), 3), "cells": res}


def sweep_1p7b(torch, nat, lib, dev, synthetic, args):
    """benchmark configs 2 and 3: every layer linear of the 28-layer 1.7B-shape
    decoder (no lm_head), decoder launch order, at 1, 4 and 16 tokens;
    fixed-width 13-bit indices, and the same weights Huffman-coded in the
    split format (one token on the split GEMV; 4 and 16 tokens through the
    transient fixed-width stream and ck_linear_f32)."""
    from gpu_huffman_functions import (split_bytes, split_fewtok, split_fewtok_eligible,
                                       split_inverse, split_prefill)
    dec = synthetic.SyntheticDecoder("qwen3-1.7b", log=log)
    tensors = dec.all_linears(with_head=False)
    names = [n for n, _, _ in tensors]
    plan = step_plan(dec, with_head=False)
    out = {"layers": dec.cfg["layers"], "shapes": "q 2048->2048, k/v 2048->1024, o 2048->2048, "
                                                   "gate/up 2048->6144, down 6144->2048"}
    fixed = dec.build_fixed(tensors)
    mats = fixed_launches(torch, nat, lib, dev, synthetic, fixed, plan)
    fx = {}
    for T in (1, 4, 16):
        with mark(f"1p7b:fixed:sweep:T{T}"):
            ms, nb = fixed_sweep(torch, nat, lib, dev, mats, T, args.steps, args.warmup)
        fx[f"T{T}"] = {"ms_per_step": round(ms, 4), "GB/s": round(nb / (ms * 1e-3) / 1e9, 1),
                       "pct_of_hbm_peak": round(100 * nb / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 1)}
    per = {}
    for kind, sel in (("q_proj", "self_attn.q_proj"), ("k_proj", "self_attn.k_proj"),
                      ("o_proj", "self_attn.o_proj"), ("gate_proj", "mlp.gate_proj"),
                      ("down_proj", "mlp.down_proj")):
        ms_k = [fixed[n] for n in names if n.endswith(sel)]
        with mark(f"1p7b:fixed:{kind}"):
            ms, nb = fixed_sweep(torch, nat, lib, dev, ms_k, 1, max(3, args.steps // 2), 1)
        t = ms_k[0]
        per[kind] = {"shape": f"{t.shape[1]}->{t.shape[0]}",
                     "us_per_launch": round(ms * 1e3 / len(ms_k), 2),
                     "GB/s": round(nb / (ms * 1e-3) / 1e9, 1)}
    # the config's dominant launch: stacked gate+up (2 x 2048->6144), one token
    gu = [m for m in mats if m.shape[0] == 2 * dec.cfg["inter"] and "+stacked" in m.name]
    with mark("1p7b:fixed:gate_up_stacked"):
        ms, nb = fixed_sweep(torch, nat, lib, dev, gu, 1, args.steps, args.warmup)
    us = ms * 1e3 / len(gu)
    ach = nb / len(gu) / (us * 1e-6) / 1e9
    roof = {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
            "frac": round(ach / HBM_PEAK_GBPS, 4),
            "kernel": f"fixed_stream_kernel<{gu[0].bits},1,f32> stacked gate+up "
                      f"{gu[0].shape[1]}->{gu[0].shape[0]}",
            "bytes_per_launch": nb // len(gu), "us_per_launch": round(us, 2)}
    out["fixed"] = {"sweep": fx, "per_shape_T1": per, "roofline": roof}
    del fixed, mats
    torch.cuda.empty_cache()

    huff = dec.build_huffman(tensors)
    splits, stream_bytes = build_split_formats(torch, dev, huff, names)
    with mark("1p7b:huffman:sweep:T1"):
        ms1, nb1 = huffman_sweep(torch, nat, lib, dev, huff, splits, plan, args.steps,
                                 args.warmup)
    n_w = sum(huff[n].shape[0] * huff[n].shape[1] for n in names)
    res_b = sum(split_bytes(k) for k in {id(splits[n][0]): splits[n][0] for n in names}.values())
    hu = {"T1": {"ms_per_step": round(ms1, 4), "GB/s": round(nb1 / (ms1 * 1e-3) / 1e9, 1),
                 "pct_of_hbm_peak": round(100 * nb1 / (ms1 * 1e-3) / 1e9 / HBM_PEAK_GBPS, 1),
                 "stream_equivalent_GB/s": round(sum(stream_bytes.values()) / (ms1 * 1e-3) / 1e9,
                                                 1)}}
    per_h = {}
    for kind, sel in (("qkv_grouped", "self_attn.q_proj"), ("o_proj", "self_attn.o_proj"),
                      ("gate_up_grouped", "mlp.gate_proj"), ("down_proj", "mlp.down_proj")):
        sub = [e for e in plan if (e[0] if isinstance(e, tuple) else e).endswith(sel)]
        with mark(f"1p7b:huffman:{kind}"):
            ms_k, nb_k = huffman_sweep(torch, nat, lib, dev, huff, splits, sub,
                                       max(3, args.steps // 2), 1)
        e0 = sub[0]
        ns0 = list(e0) if isinstance(e0, tuple) else [e0]
        per_h[kind] = {"shape": " + ".join(f"{huff[n].shape[1]}->{huff[n].shape[0]}"
                                           for n in ns0),
                       "us_per_launch": round(ms_k * 1e3 / len(sub), 2),
                       "GB/s": round(nb_k / (ms_k * 1e-3) / 1e9, 1)}
        if kind == "gate_up_grouped":
            ach = nb_k / len(sub) / (ms_k * 1e3 / len(sub) * 1e-6) / 1e9
            hu["roofline"] = {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBPS,
                              "unit": "GB/s", "frac": round(ach / HBM_PEAK_GBPS, 4),
                              "kernel": "split_gemv_kernel grouped gate+up (2 x 2048->6144, "
                                        "row groups of 2)",
                              "bytes_per_launch": nb_k // len(sub),
                              "us_per_launch": round(ms_k * 1e3 / len(sub), 2)}
    hu["per_shape_T1"] = per_h
    invs = {}
    for T in (4, 16):
        xs = {}
        for n in names:
            K = huff[n].shape[1]
            if K not in xs:
                xs[K] = torch.randn(T, K, device=dev)
            cbt = huff[n].tables["codebook"]
            if id(cbt) not in invs:
                invs[id(cbt)] = split_inverse(cbt.cpu().numpy(), dev)

        def run(T=T, xs=xs):
            # the decoder's launches: q/k/v and gate/up grouped (one fused
            # launch each, matrices sharing x); a shape the fused kernel does
            # not take would go through split_prefill's transient stream
            for e in plan:
                ns = list(e) if isinstance(e, tuple) else [e]
                M0, K = huff[ns[0]].shape
                if split_fewtok_eligible(K):
                    split_fewtok([splits[n] for n in ns], xs[K], [huff[n].shape[0] for n in ns], K)
                    continue
                for n in ns:
                    t = huff[n]
                    split_prefill(splits[n], invs[id(t.tables["codebook"])], xs[K], t.shape[0],
                                  K, t.tables["codebook"])
        with mark(f"1p7b:huffman:sweep:T{T}"):
            ms, _ = timed_graph(torch, run, max(3, args.steps // 2), 1)
        hu[f"T{T}"] = {"ms_per_step": round(ms, 3),
                       "vs_T1": round(ms / ms1, 3),
                       "note": "the decoder's launch list straight from the split format on "
                               "the matrix cores (cbq_split_linear_fewtok_f32; q/k/v and gate/up "
                               "one launch each, down in row groups of 2); graph-replayed"}
    out["huffman"] = {"sweep": hu, "bits_per_weight_resident": round(8.0 * res_b / n_w, 3),
                      "bits_per_weight_stream_incl_index":
                          round(8.0 * sum(stream_bytes.values()) / n_w, 3)}
    del huff, splits
    torch.cuda.empty_cache()
    return out


def image_roundtrip(torch, tensors, enc, meta):
    """The direct-to-device load path on the e2e model: write `tensors` as a
    device image under $TMPDIR, empty `tensors` (the caller's dict: its
    device memory is freed), drop the file from the page cache
    (fsync + POSIX_FADV_DONTNEED), load it back (cold: from the disk), free
    that copy, load again (warm: from the page cache).  Returns the warm
    load's tensors and the timings."""
    import shutil
    import tempfile
    import cbq_image
    dev = torch.device("cuda:0")
    d = tempfile.mkdtemp(prefix="cbq_img_", dir=os.environ.get("TMPDIR", "/tmp"))
    path = os.path.join(d, f"{enc}.cbq")
    try:
        need = sum(int(t.numel() * t.element_size()) for t in torch_tensors_of(tensors))
        if shutil.disk_usage(d).free < 1.5 * need:
            return tensors, {"skipped": f"less than 1.5 x {need} bytes free under {d}"}
        t0 = time.perf_counter()
        hdr = cbq_image.write_image(path, tensors, meta)
        fd = os.open(path, os.O_RDONLY)
        os.fsync(fd)
        write_s = time.perf_counter() - t0
        tensors.clear()
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
        os.posix_fadvise(fd, 0, 0, os.POSIX_FADV_DONTNEED)
        os.close(fd)
        _, _, cold = cbq_image.load_image(path, dev, threads=8)
        torch.cuda.empty_cache()
        loaded, _, warm = cbq_image.load_image(path, dev, threads=8)
        size = hdr["data_offset"] + hdr["payload_bytes"]
        kinds = {}
        for e in hdr["tensors"].values():
            kinds[e["kind"]] = kinds.get(e["kind"], 0) + 1
        log(f"image {enc}: {size / 1e9:.2f} GB, write+fsync {write_s:.1f}s, cold load "
            f"{cold['total_s']:.2f}s ({cold['upload_GB/s']:.1f} GB/s), warm "
            f"{warm['total_s']:.2f}s ({warm['upload_GB/s']:.1f} GB/s)")
        return loaded, {"image_GB": round(size / 1e9, 3), "tensor_kinds": kinds,
                        "write_fsync_s": round(write_s, 2),
                        "cold_load_s": round(cold["total_s"], 3),
                        "cold_upload_GB/s": round(cold["upload_GB/s"], 2),
                        "warm_load_s": round(warm["total_s"], 3),
                        "warm_upload_GB/s": round(warm["upload_GB/s"], 2),
                        "threads": warm["threads"], "chunk_MiB": warm["chunk_mb"],
                        "note": "cold: file dropped from the page cache after fsync, read "
                                "from the box's disk; warm: the same file again from the page "
                                "cache; load = header + one device allocation + "
                                "cbq_file_upload + descriptor set-up, no host decode"}
    finally:
        shutil.rmtree(d, ignore_errors=True)


def torch_tensors_of(tensors):
    """Every device tensor the image would store for `tensors`."""
    import synthetic
    out = []
    for t in tensors.values():
        if isinstance(t, synthetic.FixedTensor):
            out.append(t.packed)
        elif isinstance(t, synthetic.SplitTensor):
            out += list(t.keep)
        elif isinstance(t, synthetic.HuffTensor):
            out += [t.words, t.chunk_off, t.sub_len]
    return out


def e2e_section(torch, dec, args):
    """benchmark config 5: always-compressed greedy decode of the random-init
    36-layer Qwen3-8B-shape decoder at batch 1: all linears, the lm_head and
    the embedding Huffman-coded (24-bit canonical codes, 4096-symbol chunks;
    linears re-encoded to the split format, their streams freed); 128-token
    uniform random prompt, then args.e2e_tokens greedy tokens (EOS ignored).
    tok/s over the decode steps, which are captured once as a HIP graph and
    replayed.  The same model with fixed-width 13-bit indices (the same
    weights) runs too; both encodings' tokens are compared with the CPU
    oracle's golden tokens (tests/golden/e2e_qwen3_8b_golden.npz) when the
    prompt is the golden's.  Unless --no-load, each model is written as a
    device image and the decoder runs from the image loaded back
    (image_roundtrip)."""
    import numpy as np
    import decoder as D
    import synthetic
    c = dec.cfg
    cfg = D.DecoderConfig(layers=c["layers"], hidden=c["hidden"], inter=c["inter"], n_q=c["n_q"],
                          n_kv=c["n_kv"], head_dim=c["head_dim"], vocab=c["vocab"])
    names = dec.all_linears() + [dec.embed]
    prompt = [int(t) for t in np.random.default_rng(2).integers(0, cfg.vocab, 128)]
    golden = None
    if os.path.exists(GOLDEN_E2E):
        g = np.load(GOLDEN_E2E, allow_pickle=False)
        if [int(t) for t in g["prompt"]] == prompt and c["layers"] == 36:
            golden = [int(t) for t in g["tokens"]]
    n_new = args.e2e_tokens
    out = {"prompt_tokens": len(prompt), "new_tokens": n_new, "batch": 1}
    toks = {}
    n_w = sum(M * K for n, M, K in dec.all_linears())
    for enc in ("huffman", "fixed"):
        t0 = time.time()
        tensors = dec.build_huffman(names) if enc == "huffman" else dec.build_fixed(names)
        if enc == "huffman":                # linears in the split format, embedding's stream
            tensors = {n: t if n == dec.embed[0] else (synthetic.to_split(t) or t)
                       for n, t in tensors.items()}
        torch.cuda.synchronize()
        build_s = time.time() - t0
        load = None
        if not args.no_load:
            tensors, load = image_roundtrip(torch, tensors, enc, {"config": dict(c),
                                                                  "encoding": enc})
        model = D.from_synthetic(cfg, tensors, max_len=len(prompt) + n_new)
        del tensors                                # the model holds what it streams
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
        prefill = []                         # first call (allocator and module warm-up), then steady
        for _ in range(2):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            model.reset()
            model.forward(torch.tensor(prompt))
            torch.cuda.synchronize()
            prefill.append(time.perf_counter() - t0)
        prefill_s = prefill[1]
        timing = {}
        toks[enc] = model.generate_graph(prompt, n_new, timing)
        step_bytes = sum(model.linear_bytes.values())
        tps = timing["decode_steps"] / timing["decode_s"]
        out[enc] = {"decode_tok_per_s": round(tps, 2),
                    "ms_per_token": round(1e3 / tps, 3),
                    "weight_GB_per_token": round(step_bytes / 1e9, 3),
                    "weight_GB/s": round(step_bytes * tps / 1e9, 1),
                    "bits_per_weight_resident": round(8.0 * step_bytes / n_w, 3),
                    "prefill_ms_128_tokens": round(prefill_s * 1e3, 1),
                    "prefill_ms_first_call": round(prefill[0] * 1e3, 1),
                    "build_s": round(build_s, 1), "first_tokens": toks[enc][:8]}
        if load is not None:
            out[enc]["load_from_device_image"] = load
        if golden is not None:
            k = min(len(golden), n_new)
            out[enc]["tokens_equal_oracle_golden"] = toks[enc][:k] == golden[:k]
            out[enc]["golden_tokens_compared"] = k
        log(f"e2e {enc}: {tps:.1f} tok/s")
        del model
        torch.cuda.empty_cache()
    out["tokens_equal_huffman_vs_fixed"] = toks["huffman"] == toks["fixed"]
    return out


def roofline_only(torch, nat, lib, dev, dec, tensors, names, plan, mats, args):
    """The two roofline launches alone, for counter runs: the fixed-width
    stacked gate+up graph (36 launches) and the Huffman stacked gate+up graph
    with the SiLU epilogue (36 launches); prints their mean times."""
    gus = [m for m in mats if m.shape[0] == 2 * dec.cfg["inter"] and "+stacked" in m.name]
    with mark("fixed:gate_up_stacked:T1"):
        ms_gu, nb = fixed_sweep(torch, nat, lib, dev, gus, 1, args.steps, args.warmup)
    out = {"fixed_gate_up_us": round(ms_gu * 1e3 / len(gus), 2),
           "fixed_gate_up_bytes": nb // len(gus), "fixed_launches": len(gus)}
    del mats, gus
    torch.cuda.empty_cache()
    huff = dec.build_huffman(tensors)
    splits, _ = build_split_formats(torch, dev, huff, names)
    stack_gate_up(torch, dev, huff, splits, plan)
    gate_up = [e for e in plan if isinstance(e, tuple) and e[0].endswith("mlp.gate_proj")]
    with mark("huffman:gate_up_glu"):
        ms_gg, b_gg = huffman_sweep(torch, nat, lib, dev, huff, splits, gate_up, args.steps,
                                    args.warmup)
    out.update({"huffman_gate_up_glu_us": round(ms_gg * 1e3 / len(gate_up), 2),
                "huffman_gate_up_glu_bytes": b_gg // len(gate_up),
                "huffman_launches": len(gate_up)})
    print(json.dumps(out), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="qwen3-8b")
    ap.add_argument("--layers", type=int, default=None)
    ap.add_argument("--no-huffman", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-e2e", action="store_true")
    ap.add_argument("--no-load", action="store_true",
                    help="e2e: skip the device-image write / load round trip")
    ap.add_argument("--no-1p7b", action="store_true")
    ap.add_argument("--e2e-tokens", type=int, default=256)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--prefill-only", action="store_true",
                    help="build the fixed-width weights, run only the prefill section and "
                         "print its JSON (for counter runs)")
    ap.add_argument("--cpu-seconds", type=float, default=20.0)
    ap.add_argument("--copy-probe", type=int, default=0,
                    help="only run a plain device copy of this many MiB (PMC calibration)")
    ap.add_argument("--roofline-only", action="store_true",
                    help="only the two roofline launches (fixed-width stacked gate+up, Huffman "
                         "stacked gate+up with the SiLU epilogue) and their JSON (PMC runs)")
    ap.add_argument("--only-1p7b", action="store_true",
                    help="only the configs 2/3 (1.7B) sweeps and their JSON")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (got --gpus {args.gpus}); the compressed GEMV "
              "path is measured per GPU and multi-GPU scaling is not part of this build",
              file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch
    import cbq_native as nat
    import synthetic

    dev = torch.device("cuda:0")
    lib = nat.load()
    if args.copy_probe:
        a = torch.empty(args.copy_probe << 20, dtype=torch.uint8, device=dev).fill_(1)
        b = torch.empty_like(a)
        for _ in range(3):
            b.copy_(a)
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_bytes": a.numel()}))
        return

    if args.only_1p7b:
        print(json.dumps({"qwen3_1_7b": sweep_1p7b(torch, nat, lib, dev, synthetic, args)}),
              flush=True)
        return

    dec = synthetic.SyntheticDecoder(args.config, layers=args.layers, log=log)
    tensors = dec.all_linears()
    names = [n for n, _, _ in tensors]
    t0 = time.time()
    fixed = dec.build_fixed(tensors)
    torch.cuda.synchronize()
    log(f"built {len(fixed)} fixed-width tensors in {time.time() - t0:.1f}s")

    if args.prefill_only:
        kinds = {}
        for n in names:
            kinds.setdefault(n.split(".")[-1] if "layers" in n else n, []).append(n)
        print(json.dumps({"prefill": prefill_section(torch, nat, lib, dev, fixed, kinds, args)}),
              flush=True)
        return

    plan = step_plan(dec)
    mats = fixed_launches(torch, nat, lib, dev, synthetic, fixed, plan)
    if args.roofline_only:
        roofline_only(torch, nat, lib, dev, dec, tensors, names, plan, mats, args)
        return
    with mark("fixed:sweep:T1"):
        ms_step, step_bytes = fixed_sweep(torch, nat, lib, dev, mats, 1, args.steps,
                                          args.warmup)
    log(f"fixed sweep: {ms_step:.3f} ms/step, {step_bytes / 1e9:.2f} GB/step, "
        f"{len(mats)} launches")

    # per-shape mean launch time (each shape over all layers' distinct weights)
    kinds = {}
    for n in names:
        kinds.setdefault(n.split(".")[-1] if "layers" in n else n, []).append(n)
    stacked = {"qkv_proj": [m for m in mats if m.shape[0] == dec.cfg["n_q"] * dec.cfg["head_dim"]
                            + 2 * dec.cfg["n_kv"] * dec.cfg["head_dim"] and "+stacked" in m.name],
               "gate_up_proj": [m for m in mats if m.shape[0] == 2 * dec.cfg["inter"]
                                and "+stacked" in m.name]}
    breakdown = {}
    groups = {k: [fixed[n] for n in ns] for k, ns in kinds.items()}
    groups.update({k: v for k, v in stacked.items() if v})
    for kind, ts in groups.items():
        with mark(f"fixed:{kind}"):
            ms, nb = fixed_sweep(torch, nat, lib, dev, ts, 1, max(3, args.steps // 2), 1)
        t = ts[0]
        breakdown[kind] = {"shape": f"{t.shape[1]}->{t.shape[0]}", "bits": t.bits,
                           "us_per_launch": round(ms * 1e3 / len(ts), 2),
                           "GB/s": round(nb / (ms * 1e-3) / 1e9, 1)}
    gus = stacked["gate_up_proj"] or groups["gate_proj"] + groups["up_proj"]
    with mark("fixed:gate_up_stacked:T1"):
        ms_gu, _ = fixed_sweep(torch, nat, lib, dev, gus, 1, args.steps, args.warmup)
    t = gus[0]
    b_gu = fixed_bytes(t.shape[0], t.shape[1], t.bits, t.codebook.numel())
    us_gu = ms_gu * 1e3 / len(gus)
    achieved = b_gu / (us_gu * 1e-6) / 1e9
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS,
                "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4),
                "traffic": read_traffic("fixed_stream_kernel_gate_up_stacked_qwen3-8b_pmc.md"),
                "kernel": (f"fixed_stream_kernel<13,1,f32> stacked gate+up "
                           f"{t.shape[1]}->{t.shape[0]}"),
                "bytes_per_launch": b_gu, "us_per_launch": round(us_gu, 2)}

    # config 2's batch 4 / 16 (and 2, 8) on the 9B stacked gate+up: every
    # weight is read once for all T rows of x
    batch = {}
    for T in (2, 4, 8, 16):
        with mark(f"fixed:gate_up_stacked:T{T}"):
            ms_T, nb = fixed_sweep(torch, nat, lib, dev, gus, T, args.steps, args.warmup)
        us_T = ms_T * 1e3 / len(gus)
        batch[f"T{T}"] = {"us_per_launch": round(us_T, 2),
                          "GB/s": round(nb / len(gus) / (us_T * 1e-6) / 1e9, 1),
                          "vs_T1": round(us_T / us_gu, 3),
                          "GFLOP/s": round(2.0 * T * t.shape[0] * t.shape[1] / (us_T * 1e-6) / 1e9,
                                           1)}
    log(f"stacked gate+up at T=2/4/8/16: {batch}")

    result = {
        "metric": METRIC, "value": round(step_bytes / (ms_step * 1e-3) / 1e9, 1), "unit": "GB/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_step, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic: random-init N(0,0.02) bf16 weights (counter-based generator, "
                "identical on CPU and GPU), lossless per-category codebooks",
        "config": {"workload": f"{args.config} decode-step GEMV sweep, batch 1, fixed-width",
                   "layers": dec.cfg["layers"], "linears_per_step": len(names),
                   "launches_per_step": len(mats),
                   "stacking": "per layer q/k/v rows in one matrix, gate/up in one",
                   "bytes_per_step": step_bytes, "pct_of_hbm_peak":
                       round(100 * step_bytes / (ms_step * 1e-3) / 1e9 / HBM_PEAK_GBPS, 1),
                   "weight_stream_tok_per_s": round(1000.0 / ms_step, 1)},
        "roofline": roofline,
        "breakdown": breakdown,
        "batch_stacked_gate_up": batch,
    }

    if not args.no_prefill:
        with mark("prefill"):
            result["prefill"] = prefill_section(torch, nat, lib, dev, fixed, kinds, args)
    del fixed, mats, gus, groups, stacked
    torch.cuda.empty_cache()

    if not args.no_cpu_baseline:
        result["cpu_baseline"], result["cpu_baseline_detail"] = cpu_baseline(np, args.cpu_seconds)
        log(f"cpu baseline: {result['cpu_baseline']['value']} GB/s")

    if not args.no_huffman:
        from gpu_huffman_functions import split_bytes
        t0 = time.time()
        huff = dec.build_huffman(tensors)
        with mark("huffman:stream_format:gate_up"):
            stream_k = stream_gate_up(torch, nat, lib, dev, huff, plan, args.steps, args.warmup)
        log(f"stream-format gate/up: {stream_k['us_per_launch']} us per matrix, "
            f"{stream_k['GB/s']} GB/s")
        splits, stream_bytes = build_split_formats(torch, dev, huff, names)
        stack_gate_up(torch, dev, huff, splits, plan)
        log(f"built {len(huff)} Huffman tensors, {len(splits)} split formats, in "
            f"{time.time() - t0:.1f}s")
        with mark("huffman:sweep:T1"):
            ms_h, sbytes = huffman_sweep(torch, nat, lib, dev, huff, splits, plan, args.steps,
                                         args.warmup)
        hbytes = sum(stream_bytes.values())
        n_w = sum(h.shape[0] * h.shape[1] for h in huff.values())
        res_b = sum(split_bytes(k) for k in {id(splits[n][0]): splits[n][0]
                                            for n in names}.values())
        gate_up = [e for e in plan if isinstance(e, tuple) and e[0].endswith("mlp.gate_proj")]
        with mark("huffman:gate_up_glu"):
            ms_gg, b_gg = huffman_sweep(torch, nat, lib, dev, huff, splits, gate_up, args.steps,
                                        args.warmup)
        us_gg = ms_gg * 1e3 / len(gate_up)
        b_gg //= len(gate_up)
        s_gg = sum(stream_bytes[n] for n in gate_up[0]) + 4 * (
            huff[gate_up[0][0]].shape[0] + huff[gate_up[0][0]].shape[1])
        ach = b_gg / (us_gg * 1e-6) / 1e9
        # config 3's batches on the 9B stacked gate+up (both matrices under
        # one table, 2 x 12288 rows): one fused launch per step, every weight
        # decoded once for all T tokens
        from gpu_huffman_functions import split_fewtok
        glus = [splits[("glu", e[0])] for e in gate_up if ("glu", e[0]) in splits]
        hbatch = {}
        if glus:
            Mg = 2 * huff[gate_up[0][0]].shape[0]
            Kg = huff[gate_up[0][0]].shape[1]
            gbytes = split_bytes(glus[0][0])
            for T in (2, 4, 8, 16):
                xg = torch.randn(T, Kg, device=dev)
                with mark(f"huffman:gate_up_stacked:T{T}"):
                    ms_T, _ = timed_graph(
                        torch, lambda xg=xg: [split_fewtok([g], xg, [Mg], Kg) for g in glus],
                        args.steps, args.warmup)
                us_T = ms_T * 1e3 / len(glus)
                hbatch[f"T{T}"] = {"us_per_launch": round(us_T, 2),
                                   "GB/s": round(gbytes / (us_T * 1e-6) / 1e9, 1),
                                   "vs_T1": round(us_T / us_gg, 3)}
            log(f"huffman stacked gate+up at T=2/4/8/16: {hbatch}")
        result["huffman"] = {
            "value": round(sbytes / (ms_h * 1e-3) / 1e9, 1), "unit": "GB/s",
            "ms_per_step": round(ms_h, 4), "bytes_per_step": sbytes,
            "format": "split (raw low byte of bf16, <=7-bit Huffman code of the high byte), "
                      "built on the GPU from each matrix's canonical-Huffman index stream, "
                      "which is then freed: the only resident format; each layer's gate/up "
                      "pair stacked under one shared table",
            "stream_format_kernel": stream_k,
            "batch_stacked_gate_up": {
                "kernel": "cbq_split_linear_fewtok_f32 (split_fewtok_kernel: decode into LDS, "
                          "bf16 MFMA, x split into three exact bf16 parts), stacked gate+up "
                          "4096->24576 under one table",
                "vs_T1_is": "against the one-token GLU launch of the same stacked matrix",
                **hbatch},
            "stream_bytes_per_step": hbytes,
            "stream_equivalent_GB/s": round(hbytes / (ms_h * 1e-3) / 1e9, 1),
            "launches_per_step": len(plan),
            "bits_per_weight_resident": round(8.0 * res_b / n_w, 3),
            "bits_per_weight_stream_incl_index": round(8.0 * hbytes / n_w, 3),
            "weight_stream_tok_per_s": round(1000.0 / ms_h, 1),
            "roofline": {
                "bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                "frac": round(ach / HBM_PEAK_GBPS, 4),
                "stream_equivalent_achieved": round(s_gg / (us_gg * 1e-6) / 1e9, 1),
                "stream_equivalent_frac": round(s_gg / (us_gg * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4),
                "traffic": read_traffic("split_gemv_kernel_gate_up_qwen3-8b_pmc.md"),
                "kernel": "split_gemv_kernel<16,glu> stacked gate+up under one table, "
                          "4096->2x12288, silu(gate)*up in the epilogue",
                "bytes_per_launch": b_gg, "us_per_launch": round(us_gg, 2)}}
        log(f"huffman sweep (split format): {ms_h:.3f} ms/step, {sbytes / 1e9:.2f} GB/step; "
            f"stacked gate+up {us_gg:.2f} us; {8.0 * res_b / n_w:.3f} bits/weight resident")
        del huff, splits
        torch.cuda.empty_cache()

    if not args.no_1p7b and args.config == "qwen3-8b" and args.layers is None:
        with mark("1p7b"):
            result["qwen3_1_7b"] = sweep_1p7b(torch, nat, lib, dev, synthetic, args)
        log(f"1.7B sweeps: {result['qwen3_1_7b']['fixed']['sweep']}")

    if not args.no_e2e:
        with mark("e2e"):
            result["e2e"] = e2e_section(torch, dec, args)

    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
