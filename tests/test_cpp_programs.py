"""The C++ test programs that mirror the reference's (tests/cpp/*.cpp): exit 0 = all checks pass,
77 = skipped for want of a GPU (the reference's CTest convention)."""
import os
import subprocess

import pytest

from conftest import ROOT, progress

# KVB_BUILD_DIR: programs built from a mutated copy of the sources (tests/mutation/mutate.py)
BUILD = os.environ.get("KVB_BUILD_DIR") or os.path.join(ROOT, "kv-cache-bench_amd", "build")
BIN = os.path.join(BUILD, "tests")


def run(name, timeout):
    progress(f"[cpp] {name} starts")
    log_dir = os.environ.get("KVB_LOG_DIR")  # optional: keep each program's full output there
    log = open(os.path.join(log_dir, f"{name}.log"), "w") if log_dir and os.path.isdir(log_dir) else None
    p = subprocess.Popen([os.path.join(BIN, name)], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    lines = []
    for line in p.stdout:  # streamed, so a long run keeps showing progress
        lines.append(line)
        if log:
            log.write(line)
            log.flush()
    rc = p.wait(timeout=timeout)
    if log:
        log.close()
    out = "".join(lines)
    progress(f"[cpp] {name} rc={rc}: {lines[-1].strip() if lines else ''}")
    return rc, out


def test_cpu_tests():
    rc, out = run("cpu_tests", 120)
    assert rc == 0, out
    assert " 0 failed" in out


def test_boundary_tests_cpu_part(kvb):
    if kvb.gpu_available():
        pytest.skip("the GPU run covers it")
    rc, out = run("boundary_tests", 120)
    assert rc == 77, out
    assert " 0 failed" in out


@pytest.mark.gpu
def test_gpu_tests_grid(gpu):
    rc, out = run("gpu_tests", 900)
    assert rc == 0, out[-4000:]


@pytest.mark.gpu
def test_boundary_tests(gpu):
    rc, out = run("boundary_tests", 900)
    assert rc == 0, out[-4000:]


KVBENCH = os.path.join(BUILD, "kvbench")


@pytest.mark.gpu
def test_kvbench_accuracy(gpu):
    """--accuracy (the reference's bench/bench.cpp:186-215): one CSV row per (data, type, page); the
    fp32 cache's error is the kernel's own (<= 2e-5 against fp64 on the same values), fp16 and int8
    add their storage error."""
    out = subprocess.run([KVBENCH, "--accuracy", "--batch=2", "--lens=300,1000", "--pages=16,64"],
                         capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stderr
    rows = [r.split(",") for r in out.stdout.splitlines() if r and not r.startswith("#")]
    assert rows[0] == ["data", "dtype", "seq_len", "page", "max_abs_err", "rms_err"]
    body = rows[1:]
    assert len(body) == 2 * 2 * 3 * 2  # data x lens x types x pages
    for data, dtype, L, page, mx, rms in body:
        mx, rms = float(mx), float(rms)
        assert 0 <= rms <= mx
        assert mx <= {"f32": 2e-5, "f16": 2e-3, "i8": 5e-2}[dtype], (data, dtype, L, page, mx)
    progress("[kvbench] accuracy: " + "; ".join(f"{d} {t} L{L} p{p}: {m}" for d, t, L, p, m, _ in body[:6]))


@pytest.mark.gpu
def test_kvbench_dump(gpu, oracle, tmp_path):
    """--dump: raw fp32 inputs and fp64 outputs; the f32 output recomputed by the oracle from the
    dumped inputs must agree (both are fp64 attention on the same values)."""
    import numpy as np
    B, H, Hkv, D, L = 2, 32, 8, 128, 200
    out = subprocess.run([KVBENCH, f"--dump={tmp_path}", f"--batch={B}", f"--lens={L}"],
                         capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stderr
    q = np.fromfile(tmp_path / f"L{L}_q.f32", np.float32).reshape(B, H, D)
    k = np.fromfile(tmp_path / f"L{L}_k.f32", np.float32).reshape(B, Hkv, L, D)
    v = np.fromfile(tmp_path / f"L{L}_v.f32", np.float32).reshape(B, Hkv, L, D)
    ref32 = np.fromfile(tmp_path / f"L{L}_ref_f32.f32", np.float32).reshape(B, H, D)
    ref16 = np.fromfile(tmp_path / f"L{L}_ref_f16.f32", np.float32).reshape(B, H, D)
    want = oracle.attention(gpu.Shape(B, H, Hkv, D), np.array([L] * B, np.int32), L, q, k, v)
    assert oracle.max_abs_diff(ref32, want) <= 1e-6
    # the f16 dump is of the fp16-rounded values: close to, not equal to, the fp32 one
    assert 0 < oracle.max_abs_diff(ref16, ref32) < 1e-2


@pytest.mark.gpu
def test_kvbench_csv_and_loads(gpu):
    """The default CSV (the reference's bench/bench.cpp:121-259 schema, plus decode/reduce split and
    kv_bytes): gpu_naive and gpu_paged rows per (type, length, page, partition), the paged output
    against the naive one, and --loads rows timed below the full step; --bw one read_bw row."""
    out = subprocess.run([KVBENCH, "--batch=2", "--lens=2048", "--pages=16,64", "--parts=256", "--reps=3",
                          "--warmup=1", "--loads", "--types=f32,f16,i8"],
                         capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stderr
    lines = [r for r in out.stdout.splitlines() if r and not r.startswith("#")]
    head = lines[0].split(",")
    assert head[:11] == ["impl", "dtype", "batch", "seq_len", "page", "part", "reps", "median_us", "min_us",
                         "max_us", "gbps"]
    rows = [dict(zip(head, r.split(","))) for r in lines[1:]]
    by = {}
    for r in rows:
        by.setdefault(r["impl"], []).append(r)
    assert len(by["gpu_naive"]) == 2  # f32 and f16 (the naive kernels take no int8)
    assert len(by["gpu_paged"]) == 3 * 2 and len(by["gpu_paged_loads"]) == 3 * 2
    for r in by["gpu_paged"]:
        if r["dtype"] != "i8":
            assert float(r["max_diff_vs_naive"]) <= 2e-5, r
    step = {(r["dtype"], r["page"]): float(r["median_us"]) for r in by["gpu_paged"]}
    for r in by["gpu_paged_loads"]:
        assert 0 < float(r["median_us"]) <= 1.5 * step[(r["dtype"], r["page"])], r
    bw = subprocess.run([KVBENCH, "--bw", "--bw-bytes=268435456", "--reps=3"], capture_output=True, text=True,
                        timeout=300)
    assert bw.returncode == 0, bw.stderr
    b = [r.split(",") for r in bw.stdout.splitlines() if r.startswith("read_bw,")]
    assert len(b) == 1 and 500 < float(b[0][6]) < 12000
    progress(f"[kvbench] paged f16 page 64: {step[('f16', '64')]} us; read_bw 256 MiB: {b[0][6]} GB/s")
