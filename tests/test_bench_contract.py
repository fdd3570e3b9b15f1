"""bench.py's host-side contract, on the CPU: it refuses more than one GPU with a message and
a non-zero status, summarises a kernel trace over the last dispatches of each kernel (the
profiles' tables), and reads the HBM traffic per launch from the committed counter summary."""

from __future__ import annotations

import csv
import importlib
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
bench = importlib.import_module("bench")


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120, cwd=ROOT)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


def test_trace_summary_averages_the_last_dispatches(tmp_path):
    path = tmp_path / "run_kernel_trace.csv"
    with open(path, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(["Kernel_Name", "Start_Timestamp", "End_Timestamp"])
        # kernel A: 5 dispatches of 10, 20, 30, 40, 50 us (out of order); kernel B: 2 of 1 us
        for i, d in [(3, 40), (0, 10), (4, 50), (1, 20), (2, 30)]:
            w.writerow(["A", 1_000_000 * i, 1_000_000 * i + d * 1000])
        for i in range(2):
            w.writerow(["B", 500_000 * i, 500_000 * i + 1000])
    table = bench.summarize_kernel_trace(str(path), 3).splitlines()
    assert table[0].startswith("| kernel |")
    rows = {line.split("`")[1]: line for line in table[2:]}
    # the last 3 dispatches of A by start time: 30, 40, 50 us
    assert [c.strip() for c in rows["A"].split("|")[2:7]] == ["5", "3", "40.00", "30.00", "50.00"]
    assert [c.strip() for c in rows["B"].split("|")[2:7]] == ["2", "2", "1.00", "1.00", "1.00"]
    assert table[2].startswith("| `A`")  # sorted by total time


def test_traffic_comes_from_the_counter_summary():
    text = (ROOT / "profiles" / "attn_prefill_ring_share_pmc.md").read_text()
    line = next(l for l in text.splitlines() if l.startswith("traffic_bytes_per_launch:"))
    assert bench._measured_traffic("attn_prefill_ring_share") == int(line.split(":")[1].split()[0])
    assert bench._measured_traffic("no_such_kernel") is None
