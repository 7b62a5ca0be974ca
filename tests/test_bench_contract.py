"""CPU checks of bench.py's contract: one GPU only, the algorithmic byte
count of a decode step, and the CPU-baseline leg on a tiny sample."""
import os
import subprocess
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
import bench  # noqa: E402


def test_more_than_one_gpu_exits_with_a_message():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


def test_decode_step_bytes():
    # K and V read once per context token and KV head, q read and the
    # output written once per query head, and the appended token's K and V
    # read from the step's input and written into the cache
    ctx = np.array([17, 64, 200, 511], np.int32)
    x = dict(ctx=ctx, B=4, hq=16, hkv=8, d=128)
    attend, step = bench.decode_bytes(x)
    assert attend == int(ctx.sum()) * 8 * 128 * 2 * 2 + 2 * 4 * 16 * 128 * 2
    assert step == attend + 2 * 4 * 8 * 128 * 2 * 2


def test_cpu_baseline_reports_a_port_on_one_core():
    ctx = np.array([5, 300, 1], np.int32)
    r = bench.cpu_baseline(dict(ctx=ctx, hq=4, hkv=2, d=128, bs=256), reps=1)
    assert r["kind"] == "port" and r["cores"] == 1 and r["unit"] == "GB/s"
    assert r["value"] > 0 and r["seconds_per_step"] >= 0
    assert "3 sequences (306 context tokens)" in r["sample"]


def test_cpu_e2e_baseline_runs_the_layer_on_the_host():
    import torch
    ctx = np.array([3, 40, 17], np.int32)
    r = bench.cpu_e2e_baseline(torch, ctx, threads=2, reps=1, hidden=64, inter=96, hq=4, hkv=2,
                               d=16, layers=2, vocab=50)
    assert r["unit"] == "output tok/s" and r["kind"] == "port" and r["cores"] == 2
    assert r["value"] > 0 and "3 sequences (context 3-40" in r["sample"]
