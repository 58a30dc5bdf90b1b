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


@pytest.mark.gpu
def test_bench_line_contract(kvb):
    """On a GPU: one JSON line with the driver's keys, the roofline object and a CPU baseline, and
    numbers that agree with each other (c1 keeps it short)."""
    import json
    from conftest import progress
    progress("[bench] c1 contract run")
    r = subprocess.run([sys.executable, BENCH, "--config", "c1", "--steps", "5", "--warmup", "1", "--no-extras"],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    lines = [l for l in r.stdout.splitlines() if l.strip()]
    assert len(lines) == 1, r.stdout
    d = json.loads(lines[0])
    for key in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better",
                "scaling", "vs_baseline", "dtype", "data", "config", "roofline", "cpu_baseline"):
        assert key in d, key
    assert (d["n_gpus"], d["steps"], d["warmup"]) == (1, 5, 1)
    assert d["unit"] == "GB/s" and d["higher_is_better"] is True and d["vs_baseline"] is None
    rf = d["roofline"]
    assert rf["bound"] == "hbm" and rf["peak"] == 8000.0 and rf["unit"] == "GB/s"
    assert abs(rf["frac"] - rf["achieved"] / rf["peak"]) < 1e-3
    assert rf["bytes_per_launch"] == d["config"]["bytes_per_step"]
    assert abs(d["value"] - d["config"]["bytes_per_step"] / (d["ms_per_step"] * 1e-3) / 1e9) < 0.01 * d["value"]
    cpu = d["cpu_baseline"]
    assert cpu["value"] > 0 and cpu["cores"] >= 1 and cpu["kind"] in ("reference", "port")
    assert cpu["sample"].startswith("the whole step")
    env = d["env"]
    assert env["hip_runtime_version"] > 0 and env["compute_units"] > 0 and len(env["loadavg_before"]) == 3
    assert env["commit"] and env["sources_sha256"] and env["cpu_threads"] >= 1
    assert rf["kernel"].startswith("void kvbk::paged_decode_kernel<")
    if rf["traffic"] is not None:  # a record measured on this very kernel
        assert rf["traffic_source"] == "profiles/traffic_c1.json"


def test_traffic_record_needs_the_same_kernel(tmp_path, monkeypatch):
    """bench.py attaches profiles/traffic_<config>.json only when it was measured on the kernel the run
    launches; a record for another instantiation, or none at all, gives null with the reason."""
    import json
    bench = load_bench()
    k = "void kvbk::paged_decode_kernel<1, 128, 4, true, false, true, false, false, false>(kvbk::DecodeParams)"
    os.makedirs(tmp_path / "profiles")
    with open(tmp_path / "profiles" / "traffic_c2.json", "w") as f:
        json.dump({"config": "c2", "kernel_name": k, "bytes_per_launch": 135000000, "tcc_hit_rate": 0.34}, f)
    monkeypatch.setattr(bench, "ROOT", str(tmp_path))
    rec, why = bench.traffic_record("c2", k)
    assert why is None and rec["bytes_per_launch"] == 135000000 and rec["tcc_hit_rate"] == 0.34
    rec, why = bench.traffic_record("c2", k.replace("true, false, true", "true, false, false"))
    assert rec is None and "was measured on" in why
    rec, why = bench.traffic_record("c3", k)
    assert rec is None and why.startswith("no profiles/traffic_c3.json")


def test_env_record_names_the_build():
    """The build's source identity (build/build_info.json, written by the package Makefile) matches
    the sources as they are, and names a commit; a GPU run adds the device and HIP versions."""
    import json
    bench = load_bench()
    bi = bench.build_info
    with open(bi.BUILD_INFO) as f:
        built = json.load(f)
    assert set(built) >= {"commit", "dirty", "sources_sha256", "built_at", "hipcc"}
    assert built["sources_sha256"] == bi.sources_sha256()
    assert bi.cpu_threads() >= 1 and bi.cpu_model()
    assert bench.cpu_threads() == bi.cpu_threads()
