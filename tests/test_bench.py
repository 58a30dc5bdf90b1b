"""bench.py's contract where no GPU is needed: the one-GPU refusal, the no-GPU exit, and the CPU
baseline leg (the reference's fp64 path, or the C oracle, on a bounded sample)."""
import importlib.util
import os
import subprocess
import sys

import pytest

from conftest import ROOT

BENCH = os.path.join(ROOT, "bench.py")


def load_bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", BENCH)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, BENCH, "--gpus", "2"], capture_output=True, text=True, timeout=300)
    assert r.returncode == 2
    assert "one GPU" in r.stdout + r.stderr
    assert not r.stdout.strip().startswith("{")  # no JSON line


def test_no_gpu_exits_without_a_line(kvb):
    if kvb.gpu_available():
        pytest.skip("a GPU is present")
    r = subprocess.run([sys.executable, BENCH, "--steps", "1", "--warmup", "0"], capture_output=True, text=True,
                       timeout=300)
    assert r.returncode != 0
    assert "{" not in r.stdout


def test_cpu_baseline_leg(kvb, oracle):
    """On a small workload: the fields the JSON line carries, a positive rate, and the sample named."""
    bench = load_bench()
    w = kvb.Workload(kvb.Shape(2, 8, 2, 128), "f16", [0, 300], seed=5)
    c = kvb.PagedCache(w, 16, 7)
    cpu = bench.cpu_baseline(kvb, oracle, w, c, seconds_budget=5.0)
    assert set(cpu) >= {"value", "unit", "cores", "kind", "sample", "cpu", "ms_per_step"}
    assert cpu["value"] > 0 and cpu["unit"] == "GB/s" and cpu["cores"] >= 1
    assert cpu["kind"] == ("reference" if oracle.ref is not None else "port")
    assert cpu["sample"].startswith("the whole step (2 sequences, 300 tokens)")
    # Past max_bytes: the longest prefix that fits, never fewer than one non-empty sequence.
    w3 = kvb.Workload(kvb.Shape(3, 8, 2, 128), "f16", [0, 300, 200], seed=5)
    c3 = kvb.PagedCache(w3, 16, 7)
    part = bench.cpu_baseline(kvb, oracle, w3, c3, seconds_budget=5.0, max_bytes=300 * 2 * 128 * 2 * 2)
    assert part["sample"].startswith("sequences 0-1 of 3 (300 of 500 tokens)")
    assert "ms_per_step" not in part and part["ms_per_step_extrapolated"] > 0
    tiny = bench.cpu_baseline(kvb, oracle, w3, c3, seconds_budget=5.0, max_bytes=1)
    assert tiny["sample"].startswith("sequences 0-1 of 3")
    wi = kvb.Workload(kvb.Shape(2, 8, 2, 128), "i8", [40, 0], seed=6)
    ci = kvb.PagedCache(wi, 16, 8)
    assert "dequantised int8" in bench.cpu_baseline(kvb, oracle, wi, ci, seconds_budget=5.0)["sample"]
