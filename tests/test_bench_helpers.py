"""CPU tests of bench.py's measurement helpers: the correctness gate that runs
before any timing, the roofline arithmetic, the traffic lookup in the
committed counter summaries, the repetition statistics, and the one-GPU
guard of the command line. No GPU is touched."""

import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402


def _bf16_values(n, seed=0):
    from oracle.packed_q6 import bf16_round

    return bf16_round(np.random.default_rng(seed).normal(size=n).astype(np.float32))


def test_check_close_accepts_identical_and_reports_the_gate():
    want = _bf16_values(1000)
    r = bench.check_close("same", want.copy(), want)
    assert r == {"passed": True, "max_rel_error": 0.0, "bit_identical_frac": 1.0}


@pytest.mark.parametrize("plant", ["nan", "inf", "one_large_error", "many_one_ulp_flips"])
def test_check_close_rejects_planted_mistakes(plant):
    want = _bf16_values(1000, seed=1)
    got = want.copy()
    if plant == "nan":
        got[17] = np.nan
    elif plant == "inf":
        got[3] = np.inf
    elif plant == "one_large_error":
        got[5] += 0.05 * np.abs(want).max()  # 5 % of the largest output: beyond the 1e-2 gate
    else:
        # every output moved by a relative 2^-8 (about one BF16 step): within
        # 1e-2, but far below the 90 % bit-identical floor
        got = (got * np.float32(1 + 2.0 ** -8)).astype(np.float32)
    with pytest.raises(bench.CheckFailed):
        bench.check_close(plant, got, want)


def test_roofline_arithmetic_and_units():
    r = bench.roofline("no_such_kernel", "hbm", 4e9, 1000.0, work_unit="bytes_per_launch")
    assert r["unit"] == "GB/s" and r["peak"] == bench.HBM_PEAK_GBS
    assert r["achieved"] == pytest.approx(4000.0)  # 4 GB in 1 ms
    assert r["frac"] == pytest.approx(0.5)
    assert r["traffic"] is None and r["traffic_source"] is None
    assert r["bytes_per_launch"] == 4_000_000_000
    m = bench.roofline("no_such_kernel", "mfma", 2.5e12, 2000.0, work_unit="flops_per_launch")
    assert m["unit"] == "TFLOP/s" and m["achieved"] == pytest.approx(1250.0)
    assert m["frac"] == pytest.approx(0.5)


def test_traffic_comes_from_the_committed_counter_summary():
    t, src = bench.traffic_of("q6moe::moe_dec_gate_up_kernel<0, true>")
    assert src == "profiles/bench_workloads__hbm_bytes.txt"
    # the headline gate/up launch moves ~129 MB of algorithmic bytes; the
    # counters read within a few percent of that
    assert 120e6 < t < 140e6
    # per-workload rows of one kernel are told apart by their note
    t1, _ = bench.traffic_of("q6moe::moe_dec_gate_up_kernel<1, true>", tag="1 token")
    t64, _ = bench.traffic_of("q6moe::moe_dec_gate_up_kernel<1, true>", tag="64 token")
    assert t1 is not None and t64 is not None and t64 > 4 * t1


def test_stats_of_repetitions():
    s = bench.stats([3.0, 1.0, 2.0, 10.0, 2.0])
    assert s == {"median": 2.0, "min": 1.0, "max": 10.0, "mean": 3.6, "n": 5}


def test_more_than_one_gpu_is_refused_without_touching_a_gpu():
    p = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=300)
    assert p.returncode == 2
    assert "one GPU" in p.stderr
    assert p.stdout == ""
