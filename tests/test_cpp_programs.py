"""The C++ test programs that mirror the reference's (tests/cpp/*.cpp): exit 0 = all checks pass,
77 = skipped for want of a GPU (the reference's CTest convention)."""
import os
import subprocess

import pytest

from conftest import ROOT, progress

BIN = os.path.join(ROOT, "kv-cache-bench_amd", "build", "tests")


def run(name, timeout):
    progress(f"[cpp] {name} starts")
    log_dir = os.path.join(ROOT, "gpurun_out")
    log = open(os.path.join(log_dir, f"{name}.log"), "w") if os.path.isdir(log_dir) else None
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
