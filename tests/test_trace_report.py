"""The rocprofv3 CSV summariser used for the profile notes, on a hand-made
trace (no GPU)."""
import csv
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", "codebook-quantization_amd"))

import trace_report  # noqa: E402


def _write(path, fields, rows):
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=fields)
        w.writeheader()
        w.writerows(rows)


KT = ["Kernel_Name", "Grid_Size_X", "Start_Timestamp", "End_Timestamp"]


def test_sections_innermost_marker(tmp_path):
    d = tmp_path / "kt"
    d.mkdir()
    _write(d / "run_kernel_trace.csv", KT, [
        {"Kernel_Name": "void a<1>(int)", "Grid_Size_X": 64, "Start_Timestamp": 100, "End_Timestamp": 1100},
        {"Kernel_Name": "void a<1>(int)", "Grid_Size_X": 64, "Start_Timestamp": 2000, "End_Timestamp": 5000},
        {"Kernel_Name": "b(float)", "Grid_Size_X": 32, "Start_Timestamp": 9000, "End_Timestamp": 9500},
        {"Kernel_Name": "b(float)", "Grid_Size_X": 32, "Start_Timestamp": 20000, "End_Timestamp": 20100},
    ])
    _write(d / "run_marker_api_trace.csv", ["Function", "Start_Timestamp", "End_Timestamp"], [
        {"Function": "bench:outer", "Start_Timestamp": 0, "End_Timestamp": 10000},
        {"Function": "bench:inner", "Start_Timestamp": 1500, "End_Timestamp": 6000},
    ])
    text = trace_report.sections(str(d))
    lines = {ln.split()[0] + "|" + ln.split("  ")[-1].strip(): ln for ln in text.splitlines()[1:]}
    assert "n=    1 mean      1.00" in lines["outer|void a<1> grid 64"]
    assert "n=    1 mean      3.00" in lines["inner|void a<1> grid 64"]
    assert "mean      0.50" in lines["outer|b grid 32"]
    assert "mean      0.10" in lines["-|b grid 32"]
    assert (d / "sections.txt").read_text() == text


def test_steps_span_and_gap(tmp_path):
    d = tmp_path / "e2e"
    d.mkdir()
    rows = []
    t = 0
    for step in range(4):
        rows.append({"Kernel_Name": "fixed_embedding_kernel<13>(x)", "Grid_Size_X": 1024,
                     "Start_Timestamp": t, "End_Timestamp": t + 2000})
        rows.append({"Kernel_Name": "gemv(x)", "Grid_Size_X": 8, "Start_Timestamp": t + 3000,
                     "End_Timestamp": t + 7000})
        t += 10000 if step != 1 else 50_000_000     # a gap of 50 ms ends a generate call
    _write(d / "run_kernel_trace.csv", KT, rows)
    text = trace_report.steps(str(d))
    head = text.splitlines()[0]
    # pairs (0,1) and (2,3) are steps; (1,2) spans the 50 ms gap and is dropped
    assert head.startswith("== fixed: 2 steps, 10.0 us per step (busy 6.0 us), 2 dispatches")
    assert "4.0 us/step    1.0/step  mean    4.00  gemv grid 8" in text


def test_pmc_mean_per_kernel(tmp_path):
    d = tmp_path / "p"
    d.mkdir()
    _write(d / "run_counter_collection.csv", ["Kernel_Name", "Grid_Size", "Counter_Name", "Counter_Value"], [
        {"Kernel_Name": "k(int)", "Grid_Size": 16, "Counter_Name": "FETCH_SIZE", "Counter_Value": 10},
        {"Kernel_Name": "k(int)", "Grid_Size": 16, "Counter_Name": "FETCH_SIZE", "Counter_Value": 30},
        {"Kernel_Name": "k(int)", "Grid_Size": 16, "Counter_Name": "WRITE_SIZE", "Counter_Value": 99},
    ])
    text = trace_report.pmc(str(d), "FETCH_SIZE")
    assert "n=   2 mean           20.0 min           10.0 max           30.0" in text
    assert "99" not in text
