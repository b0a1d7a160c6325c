#!/usr/bin/env python3
"""Text summaries of rocprofv3 CSV output, as kept in the profile notes.

    python codebook-quantization_amd/trace_report.py sections DIR
        kernel trace (+ marker trace of bench.py's "bench:<section>" ranges)
        -> per section and kernel: dispatches, mean / median / min / max us
    python codebook-quantization_amd/trace_report.py steps DIR
        kernel trace of bench.py's e2e decode -> one decode step (the span
        between two consecutive embedding dispatches less than 20 ms apart),
        the last 20 steps of each encoding aggregated per kernel
    python codebook-quantization_amd/trace_report.py pmc DIR COUNTER
        counter collection -> per kernel and grid: dispatches, mean / min /
        max of the counter

DIR is the folder given to `rocprofv3 -d`; the CSV files are searched below
it.  Every report is printed and also written to DIR (sections.txt,
step_summary.txt, pmc_<COUNTER>.txt).  Reads nothing but the CSV files, runs
on any host.
"""
import argparse
import collections
import csv
import glob
import os
import statistics
import sys


def _one(folder, suffix):
    hits = sorted(glob.glob(os.path.join(folder, "**", "*" + suffix), recursive=True))
    if not hits:
        raise SystemExit(f"no *{suffix} under {folder}")
    return hits[0]


def _short(name, width=100):
    return name.replace("(anonymous namespace)::", "").split("(")[0][:width]


def _dur_us(row):
    return (int(row["End_Timestamp"]) - int(row["Start_Timestamp"])) / 1e3


def _grid(row):
    return row.get("Grid_Size_X") or row.get("Grid_Size") or "?"


def _emit(folder, fname, text):
    with open(os.path.join(folder, fname), "w") as f:
        f.write(text)
    print(text, end="")
    return text


def sections(folder):
    """Attribute each dispatch to the innermost "bench:" marker range holding
    its start."""
    rows = list(csv.DictReader(open(_one(folder, "kernel_trace.csv"))))
    ranges = []
    marker = glob.glob(os.path.join(folder, "**", "*marker_api_trace.csv"), recursive=True)
    if marker:
        for r in csv.DictReader(open(marker[0])):
            name = next((v[6:] for v in r.values()
                         if isinstance(v, str) and v.startswith("bench:")), None)
            if name is not None:
                ranges.append((int(r["Start_Timestamp"]), int(r["End_Timestamp"]), name))

    def section_of(t):
        inner = None
        for a, b, n in ranges:
            if a <= t <= b and (inner is None or b - a < inner[1] - inner[0]):
                inner = (a, b, n)
        return inner[2] if inner else "-"

    agg = collections.defaultdict(list)
    for r in rows:
        agg[(section_of(int(r["Start_Timestamp"])), _short(r["Kernel_Name"]), _grid(r))].append(_dur_us(r))
    lines = [f"{len(rows)} dispatches, {len(ranges)} marker ranges\n"]
    for (sec, kern, grid), v in sorted(agg.items()):
        lines.append(f"{sec:34s} n={len(v):5d} mean {statistics.mean(v):9.2f} "
                     f"med {statistics.median(v):9.2f} min {min(v):9.2f} max {max(v):9.2f}"
                     f"  {kern} grid {grid}\n")
    return _emit(folder, "sections.txt", "".join(lines))


def steps(folder, last=20, max_gap_ns=20e6):
    rows = list(csv.DictReader(open(_one(folder, "kernel_trace.csv"))))
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))
    start = [int(r["Start_Timestamp"]) for r in rows]
    lines = []
    for enc, tag in (("huff", "huff_embedding"), ("fixed", "fixed_embedding")):
        idx = [i for i, r in enumerate(rows) if tag in r["Kernel_Name"]]
        pairs = [(a, b) for a, b in zip(idx, idx[1:]) if start[b] - start[a] < max_gap_ns][-last:]
        if not pairs:
            continue
        agg = collections.defaultdict(list)
        span, busy, count = [], [], []
        for a, b in pairs:
            span.append((start[b] - start[a]) / 1e3)
            d = [_dur_us(r) for r in rows[a:b]]
            busy.append(sum(d))
            count.append(b - a)
            for r, t in zip(rows[a:b], d):
                agg[(_short(r["Kernel_Name"], 90), _grid(r))].append(t)
        n = len(pairs)
        lines.append(f"== {enc}: {n} steps, {statistics.mean(span):.1f} us per step "
                     f"(busy {statistics.mean(busy):.1f} us), {statistics.mean(count):.0f} dispatches\n")
        for (kern, grid), v in sorted(agg.items(), key=lambda kv: -sum(kv[1])):
            lines.append(f"  {sum(v) / n:9.1f} us/step  {len(v) / n:5.1f}/step  "
                         f"mean {statistics.mean(v):7.2f}  {kern} grid {grid}\n")
    return _emit(folder, "step_summary.txt", "".join(lines))


def pmc(folder, counter):
    agg = collections.defaultdict(list)
    for r in csv.DictReader(open(_one(folder, "counter_collection.csv"))):
        if r.get("Counter_Name") == counter:
            agg[(_short(r["Kernel_Name"], 90), _grid(r))].append(float(r["Counter_Value"]))
    lines = [f"== {folder} {counter}\n"]
    for (kern, grid), v in agg.items():
        lines.append(f"  n={len(v):4d} mean {statistics.mean(v):14.1f} min {min(v):14.1f} "
                     f"max {max(v):14.1f}  ({kern!r}, {grid!r})\n")
    return _emit(folder, f"pmc_{counter}.txt", "".join(lines))


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    sub = ap.add_subparsers(dest="cmd", required=True)
    sub.add_parser("sections").add_argument("dir")
    sub.add_parser("steps").add_argument("dir")
    p = sub.add_parser("pmc")
    p.add_argument("dir")
    p.add_argument("counter")
    a = ap.parse_args(argv)
    if a.cmd == "sections":
        sections(a.dir)
    elif a.cmd == "steps":
        steps(a.dir)
    else:
        pmc(a.dir, a.counter)
    return 0


if __name__ == "__main__":
    sys.exit(main())
