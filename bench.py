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

value = algorithmic compressed bytes per step / step time (GB/s).  The same
sweep is also run with canonical-Huffman streams (24-bit codes, 4096-symbol
chunks; q/k/v and gate/up as grouped launches, one code per matrix) and
reported under "huffman".  "roofline" is the dominant kernel (the stacked
gate+up GEMV): algorithmic bytes per launch / its mean launch time from HIP
events around back-to-back launches over all 36 layers' distinct weights (so
the 256 MB MALL cannot serve repeats).  "breakdown" times every unstacked
shape the same way.  "prefill" is the bf16 MFMA GEMM (T = 512, 2048) and
"e2e" the greedy decode of the whole model.  "cpu_baseline" times the
reference's own C kernel (oracle/_ref, compiled from src/compressed_matmul.c)
on one gate_proj matrix on the host cores.
"""
import argparse
import json
import os
import re
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "codebook-quantization_amd"))

METRIC = "compressed GEMV HBM GB/s (% of peak) + decode tok/s, batch 1, 9B-scale shapes"
HBM_PEAK_GBPS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0      # MI355X dense bf16


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def fixed_bytes(M, K, bits, C, T=1):
    return (M * K * bits + 7) // 8 + 4 * C + T * K * 4 + T * M * 4


def huff_bytes(t, T=1):
    M, K = t.shape
    tabs = t.tables
    aux = 4 * tabs["lut1"].numel() + 4 * tabs["lut2"].numel() + 4 * tabs["codebook"].numel()
    return t.nbytes + aux + T * K * 4 + T * M * 4


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


def read_traffic(name):
    """HBM bytes per launch from a committed rocprofv3 PMC summary, if any."""
    p = os.path.join(ROOT, "profiles", name)
    if not os.path.exists(p):
        return None
    m = re.search(r"traffic_bytes_per_launch:\s*([0-9.eE+]+)", open(p).read())
    return float(m.group(1)) if m else None


def cpu_baseline(np, packed, cb, x, M, K, bits, seconds):
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import cbq_oracle as O
    kind = "reference" if O.ref_available() else "port"
    lib_kind = "ref" if kind == "reference" else "oracle"
    threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or min(16, os.cpu_count() or 1)
    threads = min(threads, os.cpu_count() or threads)
    nbytes = fixed_bytes(M, K, bits, len(cb))
    O.fixed_gemv(x, packed, cb, M, K, bits, kind=lib_kind, chunk_rows=None, threads=threads)
    times = []
    t_end = time.time() + seconds
    while time.time() < t_end or len(times) < 3:
        t0 = time.perf_counter()
        O.fixed_gemv(x, packed, cb, M, K, bits, kind=lib_kind, chunk_rows=None, threads=threads)
        times.append(time.perf_counter() - t0)
    med = float(np.median(times))
    t0 = time.perf_counter()
    O.fixed_gemv(x, packed, cb, M, K, bits, kind=lib_kind, chunk_rows=256, threads=threads)
    as_called = time.perf_counter() - t0
    return {"value": round(nbytes / med / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": kind,
            "sample": (f"gate_proj {K}->{M} 13-bit fixed-width GEMV, T=1, one call over all rows "
                       f"(src/compressed_matmul.c compressed_matmul_f32_chunk, gcc -O3 -fopenmp), "
                       f"median of {len(times)} runs = {med * 1e3:.2f} ms; as called by the "
                       f"reference wrapper (256-row chunks) {as_called * 1e3:.2f} ms = "
                       f"{nbytes / as_called / 1e9:.3f} GB/s")}


def prefill_section(torch, nat, lib, dev, fixed, kinds, args):
    """bf16 MFMA prefill over the same fixed-width weights,
    T = 512 and 2048 tokens of bf16 N(0, 1) activations; per shape the mean
    launch time over all layers' distinct weights (graph-replayed)."""
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
                                             "k_splits": max(1, nws // (4 * T * M)),
                                             "TFLOP/s": round(tf, 1),
                                             "frac": round(tf / MFMA_BF16_PEAK_TFLOPS, 4)}
    g = out["shapes"]["T2048_gate_proj"]
    out["roofline"] = {"bound": "mfma", "achieved": g["TFLOP/s"], "peak": MFMA_BF16_PEAK_TFLOPS,
                       "unit": "TFLOP/s", "frac": g["frac"],
                       "kernel": "fixed_prefill_kernel<13> gate/up 4096->12288, T=2048"}
    return out


def e2e_section(torch, dec, args):
    """always-compressed greedy decode of the random-init
    36-layer Qwen3-8B-shape decoder at batch 1: all linears, the lm_head and
    the embedding Huffman-coded (24-bit canonical codes, 4096-symbol chunks);
    128-token uniform random prompt, then args.e2e_tokens greedy tokens (EOS
    ignored).  tok/s over the decode steps, which are captured once as a HIP
    graph and replayed.  The same model with fixed-width 13-bit indices (the
    same weights) runs too; its tokens must agree."""
    import numpy as np
    import decoder as D
    import synthetic
    c = dec.cfg
    cfg = D.DecoderConfig(layers=c["layers"], hidden=c["hidden"], inter=c["inter"], n_q=c["n_q"],
                          n_kv=c["n_kv"], head_dim=c["head_dim"], vocab=c["vocab"])
    names = dec.all_linears() + [dec.embed]
    prompt = [int(t) for t in np.random.default_rng(2).integers(0, cfg.vocab, 128)]
    n_new = args.e2e_tokens
    out = {"prompt_tokens": len(prompt), "new_tokens": n_new, "batch": 1}
    toks = {}
    for enc in ("huffman", "fixed"):
        t0 = time.time()
        tensors = dec.build_huffman(names) if enc == "huffman" else dec.build_fixed(names)
        torch.cuda.synchronize()
        build_s = time.time() - t0
        model = D.from_synthetic(cfg, tensors, max_len=len(prompt) + n_new)
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
        step_bytes = sum((t.nbytes if enc == "huffman" else t.nbytes) for n, t in tensors.items()
                         if n != dec.embed[0])
        tps = timing["decode_steps"] / timing["decode_s"]
        out[enc] = {"decode_tok_per_s": round(tps, 2),
                    "ms_per_token": round(1e3 / tps, 3),
                    "weight_GB_per_token": round(step_bytes / 1e9, 3),
                    "weight_GB/s": round(step_bytes * tps / 1e9, 1),
                    "prefill_ms_128_tokens": round(prefill_s * 1e3, 1),
                    "prefill_ms_first_call": round(prefill[0] * 1e3, 1),
                    "build_s": round(build_s, 1), "first_tokens": toks[enc][:8]}
        log(f"e2e {enc}: {tps:.1f} tok/s")
        del tensors, model
        torch.cuda.empty_cache()
    out["tokens_equal_huffman_vs_fixed"] = toks["huffman"] == toks["fixed"]
    out["token_agreement"] = round(sum(a == b for a, b in zip(toks["huffman"], toks["fixed"])) /
                                   max(1, n_new), 4)
    return out


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
    ap.add_argument("--e2e-tokens", type=int, default=256)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--copy-probe", type=int, default=0,
                    help="only run a plain device copy of this many MiB (PMC calibration)")
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

    dec = synthetic.SyntheticDecoder(args.config, layers=args.layers, log=log)
    tensors = dec.all_linears()
    t0 = time.time()
    fixed = dec.build_fixed(tensors)
    torch.cuda.synchronize()
    log(f"built {len(fixed)} fixed-width tensors in {time.time() - t0:.1f}s")

    xs, outs = {}, {}
    for name, M, K in tensors:
        if K not in xs:
            xs[K] = torch.randn(1, K, device=dev)
        outs[name] = torch.empty(1, M, device=dev)

    def launch_fixed(names):
        st = nat.stream_ptr(dev)
        for n in names:
            t = fixed[n]
            M, K = t.shape
            rc = lib.ck_linear_f32(xs[K].data_ptr(), t.packed.data_ptr(), t.codebook.data_ptr(),
                                   outs[n].data_ptr(), 1, M, K, t.codebook.numel(), t.bits, st)
            if rc:
                raise RuntimeError(f"ck_linear_f32 rc={rc} on {n}")

    # The decode step's launches, as the decoder makes them: per layer the
    # q/k/v rows stacked into one matrix and gate/up into one (same codebook
    # and index width, so the packed bytes concatenate exactly), o, down; and
    # the lm_head.
    import synthetic
    stacked = {}
    step_names = []
    for i in range(dec.cfg["layers"]):
        p = f"model.layers.{i}."
        for fused, parts in (("self_attn.qkv_proj", ("self_attn.q_proj", "self_attn.k_proj",
                                                     "self_attn.v_proj")),
                             ("mlp.gate_up_proj", ("mlp.gate_proj", "mlp.up_proj"))):
            st = synthetic.stack_fixed([fixed[p + n] for n in parts], p + fused)
            if st is None:
                step_names += [p + n for n in parts]
                continue
            stacked[p + fused] = st
            outs[p + fused] = torch.empty(1, st.shape[0], device=dev)
            step_names.append(p + fused)
        step_names += [p + "self_attn.o_proj", p + "mlp.down_proj"]
    step_names += [n for n, _, _ in tensors if "layers" not in n]
    fixed.update(stacked)
    names = [n for n, _, _ in tensors]
    step_bytes = sum(fixed_bytes(fixed[n].shape[0], fixed[n].shape[1], fixed[n].bits,
                                 fixed[n].codebook.numel()) for n in step_names)
    ms_step, _ = timed_graph(torch, lambda: launch_fixed(step_names), args.steps, args.warmup)
    log(f"fixed sweep: {ms_step:.3f} ms/step, {step_bytes / 1e9:.2f} GB/step, "
        f"{len(step_names)} launches")

    # per-shape mean launch time (each shape over all layers' distinct weights)
    kinds = {}
    for n in names + list(stacked):
        kinds.setdefault(n.split(".")[-1] if "layers" in n else n, []).append(n)
    breakdown = {}
    for kind, ns in kinds.items():
        ms, _ = timed_graph(torch, lambda ns=ns: launch_fixed(ns), max(3, args.steps // 2), 1)
        t = fixed[ns[0]]
        per = ms / len(ns)
        b = fixed_bytes(t.shape[0], t.shape[1], t.bits, t.codebook.numel())
        breakdown[kind] = {"shape": f"{t.shape[1]}->{t.shape[0]}", "bits": t.bits,
                           "us_per_launch": round(per * 1e3, 2),
                           "GB/s": round(b / (per * 1e-3) / 1e9, 1)}
    gu = kinds.get("gate_proj", []) + kinds.get("up_proj", [])
    gus = kinds.get("gate_up_proj", []) or gu          # the decoder's stacked launch
    ms_gu, _ = timed_graph(torch, lambda: launch_fixed(gus), args.steps, args.warmup)
    t = fixed[gus[0]]
    b_gu = fixed_bytes(t.shape[0], t.shape[1], t.bits, t.codebook.numel())
    us_gu = ms_gu * 1e3 / len(gus)
    achieved = b_gu / (us_gu * 1e-6) / 1e9
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS,
                "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4),
                "traffic": read_traffic("fixed_stream_kernel_gate_up_stacked_qwen3-8b_pmc.md"),
                "kernel": (f"fixed_stream_kernel<13,1,f32> stacked gate+up "
                           f"{t.shape[1]}->{t.shape[0]}"),
                "bytes_per_launch": b_gu, "us_per_launch": round(us_gu, 2)}

    # config 2's batch 4 / 16 (and 2, 8): the same stacked gate+up launches with
    # T tokens (every weight is read once for all T rows of x)
    batch = {}
    for T in (2, 4, 8, 16):
        xT = torch.randn(T, t.shape[1], device=dev)
        oT = torch.empty(T, t.shape[0], device=dev)

        def launch_T(T=T, xT=xT, oT=oT):
            st = nat.stream_ptr(dev)
            for n in gus:
                f = fixed[n]
                rc = lib.ck_linear_f32(xT.data_ptr(), f.packed.data_ptr(), f.codebook.data_ptr(),
                                       oT.data_ptr(), T, f.shape[0], f.shape[1],
                                       f.codebook.numel(), f.bits, st)
                if rc:
                    raise RuntimeError(f"ck_linear_f32 T={T} rc={rc}")
        ms_T, _ = timed_graph(torch, launch_T, args.steps, args.warmup)
        us_T = ms_T * 1e3 / len(gus)
        bT = fixed_bytes(t.shape[0], t.shape[1], t.bits, t.codebook.numel(), T)
        batch[f"T{T}"] = {"us_per_launch": round(us_T, 2),
                          "GB/s": round(bT / (us_T * 1e-6) / 1e9, 1),
                          "GFLOP/s": round(2.0 * T * t.shape[0] * t.shape[1] / (us_T * 1e-6) / 1e9, 1)}
    log(f"stacked gate+up at T=2/4/8/16: {batch}")

    result = {
        "metric": METRIC, "value": round(step_bytes / (ms_step * 1e-3) / 1e9, 1), "unit": "GB/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_step, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic: random-init N(0,0.02) bf16 weights, lossless per-category codebooks",
        "config": {"workload": f"{args.config} decode-step GEMV sweep, batch 1, fixed-width",
                   "layers": dec.cfg["layers"], "linears_per_step": len(names),
                   "launches_per_step": len(step_names),
                   "stacking": "per layer q/k/v rows in one matrix, gate/up in one",
                   "bytes_per_step": step_bytes, "pct_of_hbm_peak":
                       round(100 * step_bytes / (ms_step * 1e-3) / 1e9 / HBM_PEAK_GBPS, 1),
                   "weight_stream_tok_per_s": round(1000.0 / ms_step, 1)},
        "roofline": roofline,
        "breakdown": breakdown,
        "batch_stacked_gate_up": batch,
    }

    if not args.no_prefill:
        result["prefill"] = prefill_section(torch, nat, lib, dev, fixed, kinds, args)

    if not args.no_cpu_baseline:
        n0 = gu[0]
        t = fixed[n0]
        M, K = t.shape
        packed = t.packed.cpu().numpy()[:(M * K * t.bits + 7) // 8]
        result["cpu_baseline"] = cpu_baseline(np, packed, t.codebook.cpu().numpy(),
                                              xs[K].cpu().numpy(), M, K, t.bits, args.cpu_seconds)

    if not args.no_huffman:
        del fixed
        torch.cuda.empty_cache()
        t0 = time.time()
        huff = dec.build_huffman(tensors)
        torch.cuda.synchronize()
        log(f"built {len(huff)} Huffman tensors in {time.time() - t0:.1f}s")
        descs = {}
        for n, t in huff.items():
            tb = t.tables
            descs[n] = nat.HuffStream(
                words=t.words.data_ptr(), n_words=t.words.numel(),
                chunk_off=t.chunk_off.data_ptr(), sub_len=t.sub_len.data_ptr(),
                lut1=tb["lut1"].data_ptr(), lut2=tb["lut2"].data_ptr(), n_lut2=tb["lut2"].numel(),
                canon=tb["canon"].data_ptr(), canon_pay=tb["pay"].data_ptr(), value_cb=None,
                C=tb["codebook"].numel(), stage_words=tb["stage_words"])
        import ctypes
        from gpu_huffman_functions import (build_columns, build_split, columns_eligible,
                                           decode_symbols, split_bytes)
        # split format (the single-token GEMV's format), decoded from
        # each matrix's own stream; column layout for the gate/up comparison
        splits = {}
        for n, t in huff.items():
            M, K = t.shape
            if K % 4096 == 0:
                idx = decode_symbols(t.words, t.chunk_off, t.sub_len, t.lengths, M * K, dev)
                sp = build_split(idx, t.tables["codebook"].cpu().numpy(), dev)
                del idx
                if sp is not None:
                    splits[n] = sp
        cols = {}
        for n in gu:
            t = huff[n]
            if columns_eligible(descs[n], t.shape[1]):
                cols[n] = build_columns(descs[n], t.shape[0] * t.shape[1], dev, t.lengths,
                                        t.tables["codebook"].cpu().numpy())
        torch.cuda.synchronize()
        log(f"split format for {len(splits)} of {len(huff)} Huffman tensors")

        def split_args(ns):
            k = len(ns)
            return (k, (ctypes.POINTER(nat.SplitMatrix) * k)(*[ctypes.pointer(splits[n][1])
                                                               for n in ns]),
                    (ctypes.c_void_p * k)(*[outs[n].data_ptr() for n in ns]),
                    (ctypes.c_int * k)(*[huff[n].shape[0] for n in ns]), huff[ns[0]].shape[1])

        def launch_split(a):
            k, mats, out_a, m_a, K = a
            rc = lib.cbq_split_linear_f32(xs[K].data_ptr(), None, None, 0, 0.0, k, mats, out_a,
                                          m_a, K, nat.stream_ptr(dev))
            if rc:
                raise RuntimeError(f"split GEMV rc={rc}")

        def launch_huff(ns):
            st = nat.stream_ptr(dev)
            for n in ns:
                M, K = huff[n].shape
                if n in splits:
                    launch_split(single[n])
                    continue
                rc = lib.cbq_huff_linear_f32(xs[K].data_ptr(), ctypes.byref(descs[n]),
                                             outs[n].data_ptr(), 1, M, K, st)
                if rc:
                    raise RuntimeError(f"Huffman GEMV rc={rc} on {n}")

        def launch_cols(ns):
            st = nat.stream_ptr(dev)
            for n in ns:
                M, K = huff[n].shape
                rc = lib.cbq_huff_linear_col_f32(xs[K].data_ptr(), ctypes.byref(descs[n]),
                                                 ctypes.byref(cols[n][1]), outs[n].data_ptr(),
                                                 M, K, st)
                if rc:
                    raise RuntimeError(f"column GEMV rc={rc} on {n}")

        single = {n: split_args([n]) for n in splits}
        # the decoder's launches: per layer q/k/v and gate/up grouped (one code
        # each, one launch), o, down; then the lm_head
        n_arr = {}
        groups = []
        for i in range(dec.cfg["layers"]):
            p = f"model.layers.{i}."
            for parts in (("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj"),
                          ("mlp.gate_proj", "mlp.up_proj")):
                ns = [p + n for n in parts]
                if all(n in splits for n in ns):
                    n_arr[ns[0]] = split_args(ns)
                    groups.append(ns[0])
                else:
                    groups += ns
            groups += [p + "self_attn.o_proj", p + "mlp.down_proj"]
        groups += [n for n in names if "layers" not in n]

        def launch_huff_step():
            for n in groups:
                if n in n_arr:
                    launch_split(n_arr[n])
                else:
                    launch_huff([n])

        hbytes = sum(huff_bytes(t) for t in huff.values())
        sbytes = sum(split_bytes(splits[n][0]) + 4 * (huff[n].shape[0] + huff[n].shape[1])
                     if n in splits else huff_bytes(huff[n]) for n in huff)
        ms_h, _ = timed_graph(torch, launch_huff_step, args.steps, args.warmup)
        ms_hgu, _ = timed_graph(torch, lambda: launch_huff(gu), args.steps, args.warmup)
        us_hgu = ms_hgu * 1e3 / len(gu)
        g0 = huff[gu[0]]
        sb_gu = split_bytes(splits[gu[0]][0]) + 4 * (g0.shape[0] + g0.shape[1])
        us_cgu = None
        if all(n in cols for n in gu):
            ms_cgu, _ = timed_graph(torch, lambda: launch_cols(gu), args.steps, args.warmup)
            us_cgu = ms_cgu * 1e3 / len(gu)
        # the decoder's gate/up launch: both matrices in one grouped launch
        # (timed last, after the column-layout comparison)
        gug = [n for n in n_arr if n.endswith("mlp.gate_proj")]
        us_gg = b_gg = None
        if gug:
            ms_gg, _ = timed_graph(torch, lambda: [launch_split(n_arr[n]) for n in gug],
                                   args.steps, args.warmup)
            us_gg = ms_gg * 1e3 / len(gug)
            up0 = gug[0].replace("gate_proj", "up_proj")
            b_gg = (split_bytes(splits[gug[0]][0]) + split_bytes(splits[up0][0])
                    + 4 * (g0.shape[0] + huff[up0].shape[0] + g0.shape[1]))
        n_w = sum(h.shape[0] * h.shape[1] for h in huff.values())
        result["huffman"] = {
            "value": round(sbytes / (ms_h * 1e-3) / 1e9, 1), "unit": "GB/s",
            "ms_per_step": round(ms_h, 4), "bytes_per_step": sbytes,
            "format": "split (raw low byte of bf16, <=7-bit Huffman code of the high byte), "
                      "built on the GPU from each matrix's canonical-Huffman index stream",
            "stream_bytes_per_step": hbytes,
            "stream_equivalent_GB/s": round(hbytes / (ms_h * 1e-3) / 1e9, 1),
            "launches_per_step": len(groups),
            "bits_per_weight_split": round(8.0 * sbytes / n_w, 3),
            "bits_per_weight_stream_incl_index": round(
                8.0 * sum(h.nbytes for h in huff.values()) / n_w, 3),
            "weight_stream_tok_per_s": round(1000.0 / ms_h, 1),
            "column_kernel_gate_up_us_per_launch": None if us_cgu is None else round(us_cgu, 2),
            "single_matrix_gate_up": {"us_per_launch": round(us_hgu, 2), "bytes_per_launch": sb_gu,
                                      "GB/s": round(sb_gu / (us_hgu * 1e-6) / 1e9, 1)}}
        if us_gg is not None:
            ach = b_gg / (us_gg * 1e-6) / 1e9
            result["huffman"]["roofline"] = {
                "bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                "frac": round(ach / HBM_PEAK_GBPS, 4),
                "traffic": read_traffic("split_gemv_kernel_gate_up_qwen3-8b_pmc.md"),
                "kernel": "split_gemv_kernel<16> grouped gate+up, 2 x 4096->12288 in one launch",
                "bytes_per_launch": b_gg, "us_per_launch": round(us_gg, 2)}
        log(f"huffman sweep (split format): {ms_h:.3f} ms/step, {sbytes / 1e9:.2f} GB/step, "
            f"{len(groups)} launches; gate/up {us_hgu:.2f} us (column kernel {us_cgu} us), "
            f"grouped gate+up {us_gg} us")

    if not args.no_e2e:
        result["e2e"] = e2e_section(torch, dec, args)

    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
