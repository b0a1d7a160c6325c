#!/usr/bin/env python3
"""Per-wave timeline of the one-token fixed-width streaming GEMV on the
9B-scale decode shapes, from the diagnostic library build.

    python codebook-quantization_amd/build_native.py --timeline   # once, on the build host
    python codebook-quantization_amd/timeline.py [--lib PATH]      # on the GPU
    python codebook-quantization_amd/timeline.py --prefill          # the bf16 prefill GEMM
    python codebook-quantization_amd/timeline.py --split            # the split-format row walk

Each shape: N(0, 0.02) bf16 weights (synthetic.make_bf16), the tensor's own
frequency-sorted codebook, 13-bit packed indices, four copies; one second of
back-to-back launches to bring the clocks up, then one launch timed with HIP
events whose per-wave timestamps (cbq_timeline_read) are summarised: the
dispatch skew, the staging of codebook and x, the first ring of items, the
per-item time after it, when the waves finish their loops (and how that
differs between the first and the second wave of each SIMD), and the whole
in-kernel span.  Prints a markdown report.
"""
import argparse
import os
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
if HERE not in sys.path:
    sys.path.insert(0, HERE)

import numpy as np  # noqa: E402
import torch  # noqa: E402

SHAPES = (("stacked gate+up", 24576, 4096), ("gate_proj", 12288, 4096),
          ("down_proj", 4096, 12288), ("stacked q/k/v", 6144, 4096), ("o_proj", 4096, 4096))


def pct(a, ps=(0, 10, 50, 90, 100)):
    return " / ".join(f"{np.percentile(a, p):.2f}" for p in ps)


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--lib", default=os.path.join(HERE, "libcbq_hip_timeline.so"))
    ap.add_argument("--warm", type=float, default=1.0)
    ap.add_argument("--graph", action="store_true",
                    help="also time the four copies graph-replayed")
    args = ap.parse_args(argv)
    import cbq_native as nat
    import codebook_builder as cbb
    import synthetic
    lib = nat.load(args.lib)
    probe = np.zeros(4096 * 6, np.uint64)
    if lib.cbq_timeline_read(probe.ctypes.data, probe.nbytes) == nat.CK_ERR_ARG:
        raise SystemExit(f"{args.lib} is not a timeline build (build_native.py --timeline)")
    dev = torch.device("cuda:0")
    st = torch.cuda.current_stream().cuda_stream
    print("| shape | event µs | in-kernel span µs | staged after entry µs | first ring µs | "
          "µs per item after it (p0/p10/p50/p90/p100) | loop end µs (p0/p10/p50/p90/p100) | "
          "waves 0-3 / 4-7 loop end µs | MB | span GB/s |")
    print("|---|---|---|---|---|---|---|---|---|---|")
    xcd_rows = []
    for name, M, K in SHAPES:
        w = synthetic.make_bf16((M, K), f"timeline.{name}", device=dev)
        cb, lut = cbb.codebook_from_counts_torch(cbb.counts_torch(w))
        idx = lut[cbb.patterns_torch(w).reshape(-1).to(torch.int64)]
        del w
        C, bits = cb.numel(), cbb.bits_for(cb.numel())
        pk = cbb.pack_torch(idx, bits)
        nb = pk.numel()
        mats = []
        for _ in range(4):
            p = torch.zeros(nb + 32, dtype=torch.uint8, device=dev)
            p[:nb] = pk
            mats.append(p)
        del idx, pk
        x = torch.randn(1, K, device=dev)
        out = torch.empty(1, M, device=dev)
        t0 = time.time()
        while time.time() - t0 < args.warm:
            for p in mats:
                nat.check(lib.ck_linear_f32(x.data_ptr(), p.data_ptr(), cb.data_ptr(),
                                            out.data_ptr(), 1, M, K, C, bits, st), "warm-up")
            torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        nat.check(lib.ck_linear_f32(x.data_ptr(), mats[1].data_ptr(), cb.data_ptr(),
                                    out.data_ptr(), 1, M, K, C, bits, st), "timed launch")
        e1.record()
        torch.cuda.synchronize()
        ev_us = e0.elapsed_time(e1) * 1e3
        tl = np.zeros(4096 * 6, np.uint64)
        nat.check(lib.cbq_timeline_read(tl.ctypes.data, tl.nbytes), "cbq_timeline_read")
        if args.graph:
            # the four copies graph-replayed: time per launch, and the span of
            # the last launch (its waves overwrite the record)
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                for p in mats:
                    nat.check(lib.ck_linear_f32(x.data_ptr(), p.data_ptr(), cb.data_ptr(),
                                                out.data_ptr(), 1, M, K, C, bits,
                                                torch.cuda.current_stream().cuda_stream), "graph")
            g.replay()
            torch.cuda.synchronize()
            e0.record()
            for _ in range(20):
                g.replay()
            e1.record()
            torch.cuda.synchronize()
            tg = np.zeros(4096 * 6, np.uint64)
            nat.check(lib.cbq_timeline_read(tg.ctypes.data, tg.nbytes), "cbq_timeline_read")
            tg = tg.reshape(4096, 6).astype(np.int64)
            tg = tg[(tg[:, 0] > 0) & (tg[:, 0] >= tg[:, 0].max() - 100_000)]
            print(f"graph {name}: {e0.elapsed_time(e1) * 1e3 / (20 * len(mats)):.1f} us per launch, "
                  f"last launch span {(tg[:, 4].max() - tg[:, 0].min()) * 0.01:.1f} us", flush=True)
            del g
        cus = torch.cuda.get_device_properties(dev).multi_processor_count
        W = min(4096, 8 * min(cus, (M + 7) // 8))                # waves of the launch
        tl = tl.reshape(4096, 6)[:W].astype(np.int64)
        r = (tl[:, :5] - tl[:, 0].min()) * 0.01                 # µs from the first entry
        items = tl[:, 5]
        per_item = (r[:, 3] - r[:, 2]) / np.maximum(items - 2, 1)
        half = (np.arange(W) % 8) < 4
        span = float(r[:, 4].max())
        mb = (M * K * bits + 7) // 8 / 1e6
        print(f"| {name} {K}->{M} | {ev_us:.1f} | {span:.1f} | {np.median(r[:, 1] - r[:, 0]):.2f} | "
              f"{np.median(r[:, 2] - r[:, 1]):.2f} | {pct(per_item)} | {pct(r[:, 3])} | "
              f"{r[half, 3].mean():.2f} / {r[~half, 3].mean():.2f} | {mb:.1f} | "
              f"{mb / span * 1e3:.0f} |", flush=True)
        # per XCD (block b runs on XCD b % 8): when its blocks start and end
        blk = np.arange(W) // 8
        nbk = W // 8
        b_entry = np.array([r[blk == b, 0].min() for b in range(nbk)])
        b_end = np.array([r[blk == b, 3].max() for b in range(nbk)])
        xe = [b_entry[np.arange(nbk) % 8 == k].mean() for k in range(8)]
        xd = [b_end[np.arange(nbk) % 8 == k].mean() for k in range(8)]
        corr = float(np.corrcoef(b_entry, b_end)[0, 1]) if nbk > 2 else float("nan")
        xcd_rows.append(f"| {name} | {' / '.join(f'{v:.2f}' for v in xe)} | "
                        f"{' / '.join(f'{v:.2f}' for v in xd)} | "
                        f"{b_end.min():.2f} - {b_end.max():.2f} | {corr:.2f} |")
        del mats
        torch.cuda.empty_cache()
    print()
    print("| shape | XCD 0..7 block entry mean µs | XCD 0..7 block loop end mean µs | "
          "block loop end min - max µs | corr(block entry, block end) |")
    print("|---|---|---|---|---|")
    for row in xcd_rows:
        print(row)


PREFILL_SHAPES = (("gate/up, one round of 192 tiles", 1024, 12288, 4096),
                  ("gate/up, one round, K = 1024", 1024, 12288, 1024),
                  ("q, 128 tiles, K split 2", 2048, 4096, 4096),
                  ("q, 32 tiles, K split 8", 512, 4096, 4096),
                  ("k, 8 tiles, K split 16", 512, 1024, 4096))


def prefill(args):
    """Per-wave timeline of the bf16 prefill GEMM (cbq_linear_bf16_ws) on
    9B shapes: one timed call per shape after a second of warm-up; the last
    prefill launch of the call is the one recorded."""
    import cbq_native as nat
    import codebook_builder as cbb
    import synthetic
    lib = nat.load(args.lib)
    probe = np.zeros(4096 * 6, np.uint64)
    if lib.cbq_prefill_timeline_read(probe.ctypes.data, probe.nbytes) == nat.CK_ERR_ARG:
        raise SystemExit(f"{args.lib} is not a timeline build (build_native.py --timeline)")
    dev = torch.device("cuda:0")
    st = torch.cuda.current_stream().cuda_stream
    print("| shape | T, K->M | call µs (events) | prefill launch span µs | waves | entry skew µs "
          "(p50/p100) | codebook staged µs | prologue µs | K loop µs (p10/p50/p90) | µs per K "
          "step | epilogue µs (p50/p90) | loop end -> launch end µs |")
    print("|---|---|---|---|---|---|---|---|---|---|---|---|")
    for name, T, M, K in PREFILL_SHAPES:
        w = synthetic.make_bf16((M, K), f"timeline.prefill.{M}.{K}", device=dev)
        cb, lut = cbb.codebook_from_counts_torch(cbb.counts_torch(w))
        idx = lut[cbb.patterns_torch(w).reshape(-1).to(torch.int64)]
        del w
        C, bits = cb.numel(), cbb.bits_for(cb.numel())
        pk = cbb.pack_torch(idx, bits)
        p = torch.zeros(pk.numel() + 32, dtype=torch.uint8, device=dev)
        p[:pk.numel()] = pk
        del idx, pk
        x = torch.randn(T, K, device=dev).bfloat16()
        out = torch.empty(T, M, device=dev, dtype=torch.bfloat16)
        nws = int(lib.cbq_linear_bf16_workspace(T, M, K))
        ws = torch.empty(max(1, nws // 4), dtype=torch.float32, device=dev)

        def call():
            nat.check(lib.cbq_linear_bf16_ws(x.data_ptr(), p.data_ptr(), cb.data_ptr(),
                                             out.data_ptr(), T, M, K, C, bits, ws.data_ptr(), nws,
                                             st), "cbq_linear_bf16_ws")
        t0 = time.time()
        while time.time() - t0 < args.warm:
            for _ in range(8):
                call()
            torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        call()
        e1.record()
        torch.cuda.synchronize()
        ev_us = e0.elapsed_time(e1) * 1e3
        tl = np.zeros(4096 * 6, np.uint64)
        nat.check(lib.cbq_prefill_timeline_read(tl.ctypes.data, tl.nbytes),
                  "cbq_prefill_timeline_read")
        tl = tl.reshape(4096, 6).astype(np.int64)
        last = tl[:, 0].max()
        tl = tl[(tl[:, 0] > 0) & (tl[:, 0] >= last - 100_000)]  # this launch (1 ms window)
        r = (tl[:, :5] - tl[:, 0].min()) * 0.01                  # µs from the first entry
        G = tl[:, 5]
        loop = r[:, 3] - r[:, 2]
        print(f"| {name} | {T}, {K}->{M} | {ev_us:.1f} | {r[:, 4].max():.1f} | {len(tl)} | "
              f"{np.median(r[:, 0]):.2f} / {r[:, 0].max():.2f} | {np.median(r[:, 1] - r[:, 0]):.2f} | "
              f"{np.median(r[:, 2] - r[:, 1]):.2f} | "
              f"{' / '.join(f'{np.percentile(loop, q):.1f}' for q in (10, 50, 90))} | "
              f"{np.median(loop / np.maximum(G, 1)):.3f} | "
              f"{np.median(r[:, 4] - r[:, 3]):.2f} / {np.percentile(r[:, 4] - r[:, 3], 90):.2f} | "
              f"{r[:, 4].max() - np.median(r[:, 3]):.2f} |", flush=True)
        del p, x, out, ws
        torch.cuda.empty_cache()


SPLIT_SHAPES = (("stacked gate+up, SiLU product in the epilogue", True, 12288, 4096),
                ("stacked q/k/v rows as one matrix", False, 6144, 4096),
                ("o_proj", False, 4096, 4096))


def split(args):
    """Per-wave timeline of the one-token split-format row walk
    (split_gemv_kernel) on 9B shapes: the split format built from each
    matrix's indices, one second of warm-up launches, then one launch timed
    with HIP events."""
    import ctypes
    import cbq_native as nat
    import codebook_builder as cbb
    import synthetic
    from gpu_huffman_functions import build_split
    lib = nat.load(args.lib)
    probe = np.zeros(4096 * 6, np.uint64)
    if lib.cbq_split_timeline_read(probe.ctypes.data, probe.nbytes) == nat.CK_ERR_ARG:
        raise SystemExit(f"{args.lib} is not a timeline build (build_native.py --timeline)")
    dev = torch.device("cuda:0")
    st = torch.cuda.current_stream().cuda_stream
    print("| shape | event µs (one launch) | graph-replayed µs per launch / in-kernel span µs "
          "of the last | in-kernel span µs | waves | staged after entry µs (p50/p90) | "
          "first chunk decoded µs after that (p50/p90) | µs per further chunk (p50) | "
          "loop end µs (p10/p50/p90/p100) | loop end -> exit µs (p50) |")
    print("|---|---|---|---|---|---|---|---|---|---|")
    for name, glu, M, K in SPLIT_SHAPES:
        rows = 2 * M if glu else M
        w = synthetic.make_bf16((rows, K), f"timeline.split.{rows}.{K}", device=dev)
        cb, lut = cbb.codebook_from_counts_torch(cbb.counts_torch(w))
        idx = lut[cbb.patterns_torch(w).reshape(-1).to(torch.int64)].to(torch.int32)
        del w
        keep, desc = build_split(idx, cb.cpu().numpy(), dev)
        del idx
        x = torch.randn(1, K, device=dev)
        out = torch.empty(1, M, device=dev)
        mp = (ctypes.POINTER(nat.SplitMatrix) * 1)(ctypes.pointer(desc))
        op = (ctypes.c_void_p * 1)(out.data_ptr())
        mr = (ctypes.c_int * 1)(M)

        def launch():
            st = torch.cuda.current_stream().cuda_stream     # the capture stream in a graph
            if glu:
                nat.check(lib.cbq_split_linear_glu_f32(x.data_ptr(), None, None, 0, 0.0,
                                                       ctypes.pointer(desc), out.data_ptr(), M, K,
                                                       st), "cbq_split_linear_glu_f32")
            else:
                nat.check(lib.cbq_split_linear_f32(x.data_ptr(), None, None, 0, 0.0, 1, mp, op,
                                                   mr, K, st), "cbq_split_linear_f32")
        t0 = time.time()
        while time.time() - t0 < args.warm:
            for _ in range(8):
                launch()
            torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        launch()
        e1.record()
        torch.cuda.synchronize()
        ev_us = e0.elapsed_time(e1) * 1e3
        tl = np.zeros(4096 * 6, np.uint64)
        nat.check(lib.cbq_split_timeline_read(tl.ctypes.data, tl.nbytes), "cbq_split_timeline_read")
        # the same launch graph-replayed: time per launch, and the span of
        # the last replay's last launch (its waves overwrite the record)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for _ in range(8):
                launch()
        g.replay()
        torch.cuda.synchronize()
        e0.record()
        for _ in range(10):
            g.replay()
        e1.record()
        torch.cuda.synchronize()
        graph_us = e0.elapsed_time(e1) * 1e3 / 80
        tg = np.zeros(4096 * 6, np.uint64)
        nat.check(lib.cbq_split_timeline_read(tg.ctypes.data, tg.nbytes), "cbq_split_timeline_read")
        tg = tg.reshape(4096, 6).astype(np.int64)
        tg = tg[(tg[:, 0] > 0) & (tg[:, 0] >= tg[:, 0].max() - 100_000) & (tg[:, 5] > 0)]
        graph_span = float((tg[:, 4].max() - tg[:, 0].min()) * 0.01)
        del g
        tl = tl.reshape(4096, 6).astype(np.int64)
        last = tl[:, 0].max()
        tl = tl[(tl[:, 0] > 0) & (tl[:, 0] >= last - 100_000) & (tl[:, 5] > 0)]
        r = (tl[:, :5] - tl[:, 0].min()) * 0.01
        items = tl[:, 5] * (2 if glu else 1)
        per = (r[:, 3] - r[:, 2]) / np.maximum(items - 1, 1)
        p = lambda a, qs: " / ".join(f"{np.percentile(a, q):.2f}" for q in qs)  # noqa: E731
        print(f"| {name} {K}->{M} | {ev_us:.1f} | {graph_us:.1f} / {graph_span:.1f} | "
              f"{r[:, 4].max():.1f} | {len(tl)} | "
              f"{p(r[:, 1] - r[:, 0], (50, 90))} | {p(r[:, 2] - r[:, 1], (50, 90))} | "
              f"{np.median(per):.2f} | {p(r[:, 3], (10, 50, 90, 100))} | "
              f"{np.median(r[:, 4] - r[:, 3]):.2f} |", flush=True)
        del keep, x, out
        torch.cuda.empty_cache()


if __name__ == "__main__":
    if "--split" in sys.argv:
        sys.argv.remove("--split")
        ap = argparse.ArgumentParser()
        ap.add_argument("--lib", default=os.path.join(HERE, "libcbq_hip_timeline.so"))
        ap.add_argument("--warm", type=float, default=1.0)
        split(ap.parse_args())
    elif "--prefill" in sys.argv:
        sys.argv.remove("--prefill")
        ap = argparse.ArgumentParser()
        ap.add_argument("--lib", default=os.path.join(HERE, "libcbq_hip_timeline.so"))
        ap.add_argument("--warm", type=float, default=1.0)
        prefill(ap.parse_args())
    else:
        main()
