"""CPU checks of bench.py's contract: one GPU only, the algorithmic byte
count of a decode step, and the CPU-baseline leg on a tiny sample."""
import os
import subprocess
import sys
import time

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


def test_oracle_1core_reports_a_port_on_one_core():
    ctx = np.array([5, 300, 1], np.int32)
    r = bench.oracle_1core(dict(ctx=ctx, hq=4, hkv=2, d=128, bs=256), reps=1)
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


def test_cpu_path_baselines_run_on_the_host_threads():
    """The fp32 torch store+attend legs (decode, prefill) and the complete
    small engine run report a rate, the threads used and what was timed."""
    import torch
    ctx = np.array([5, 300, 1, 77], np.int32)
    r = bench.cpu_decode_baseline(torch, ctx, 4, 2, "tiny", threads=2, budget_s=0.2)
    assert r["unit"] == "GB/s" and r["cores"] == 2 and r["kind"] == "port" and r["value"] > 0
    assert r["bytes_per_step"] == int(ctx.sum()) * 2 * 128 * 2 * 2 + 2 * 4 * 4 * 128 * 2 + \
        4 * 4 * 2 * 128 * 2
    p = bench.cpu_prefill_baseline(torch, 2, 300, 4, 2, threads=2, budget_s=0.2)
    assert p["unit"] == "TFLOP/s" and p["value"] > 0 and "2 x 300" in p["sample"]


def test_cpu_timing_repeats_until_its_budget():
    calls = []
    med, ts = bench._median_time(lambda: calls.append(time.sleep(0.01)), warmup=1, reps=2,
                                 budget_s=0.1)
    assert len(calls) == 1 + len(ts) and len(ts) >= 5 and sum(ts) >= 0.1
    med, ts = bench._median_time(lambda: None, warmup=0, reps=3, budget_s=10.0, max_reps=7)
    assert len(ts) == 7


def test_traffic_summaries_are_read_from_profiles():
    # the decode summary is committed; a missing file reads as None
    assert bench.measured_traffic() and bench.measured_traffic() > 1.6e9
    assert bench.measured_traffic("profiles/no_such_file.md") is None
