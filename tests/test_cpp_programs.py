"""The reference's own C++ test programs, compiled unmodified against this build's drop-in headers.

`make -C oracle ref-tests` compiles /root/reference/tests/{cpu,gpu,boundary}_tests.cpp as they are,
with `-I include/kvb` standing in for the reference's src/ (its "workload.hpp" and "reference.hpp"
are this build's headers of those names), and links them with libkvb_host, libkvb_hip and libkvref
(the reference's own src/reference.cpp, exporting only attention_reference). The binaries land in
oracle/_ref/ and travel to the GPU box prebuilt. Exit status as in the reference's CTest setup
(CMakeLists.txt:58-61): 0 = every check passed, 77 = no GPU (the CPU checks have run by then).

What each program checks (the reference's tests):
  cpu_tests       the fp64 reference's exact properties and the host layout/quantiser round trips
                  (tests/cpu_tests.cpp:30-152), run on this build's make_paged_layout, scatter and
                  int8 quantiser;
  gpu_tests       the paged kernel (shared and per-head), the naive kernels and the fp16/int8
                  storage-error bounds over shapes x lengths x pages x types x seeds
                  (tests/gpu_tests.cpp:66-166);
  boundary_tests  lengths next to pages, partitions and capacity; refusals that leave the output
                  untouched; empty sequences that give exactly 0 (tests/boundary_tests.cpp:78-210).
"""
import os
import subprocess

import pytest

from conftest import ROOT, progress

# KVB_REF_BIN: programs built from a mutated copy of the sources (tests/mutation/mutate.py), whose
# libraries are found through KVB_BUILD_DIR.
BIN = os.environ.get("KVB_REF_BIN") or os.path.join(ROOT, "oracle", "_ref")
# KVB_BUILD_DIR: libraries built from a mutated copy (the programs' RUNPATH yields to LD_LIBRARY_PATH)
LIBS = os.environ.get("KVB_BUILD_DIR")


def program(name):
    path = os.path.join(BIN, name)
    if not os.path.exists(path):
        pytest.skip(f"{path} is not built: the reference's sources were not mounted at build time")
    return path


def run(name, timeout):
    path = program(name)
    progress(f"[cpp] {name} starts")
    env = dict(os.environ)
    if LIBS:
        env["LD_LIBRARY_PATH"] = LIBS + os.pathsep + env.get("LD_LIBRARY_PATH", "")
    log_dir = os.environ.get("KVB_LOG_DIR")  # optional: keep each program's full output there
    log = open(os.path.join(log_dir, f"{name}.log"), "w") if log_dir and os.path.isdir(log_dir) else None
    p = subprocess.Popen([path], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, env=env)
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
    assert "9 passed, 0 failed" in out


def test_boundary_tests_cpu_part(kvb):
    if kvb.gpu_available():
        pytest.skip("the GPU run covers it")
    rc, out = run("boundary_tests", 120)
    # the reference's program returns 1 if a check that needs no GPU failed, else 77 (no GPU)
    assert rc == 77, out
    assert "FAIL" not in out


@pytest.mark.gpu
def test_gpu_tests_grid(gpu):
    rc, out = run("gpu_tests", 900)
    assert rc == 0, out[-4000:]
    assert " 0 failed" in out


@pytest.mark.gpu
def test_boundary_tests(gpu):
    rc, out = run("boundary_tests", 900)
    assert rc == 0, out[-4000:]
    assert " 0 failed" in out


def test_programs_link_the_drop_in(kvb):
    """The programs resolve the kernels' entry points in libkvb_hip, the host layer in libkvb_host, and
    only attention_reference in libkvref (the reference's own CPU code)."""
    path = program("gpu_tests")
    ldd = subprocess.run(["ldd", path], capture_output=True, text=True, check=True).stdout
    for lib in ("libkvb_hip.so", "libkvb_host.so", "libkvref.so"):
        assert lib in ldd, ldd
    kvref = os.path.join(BIN, "libkvref.so")
    syms = subprocess.run(["nm", "-D", "--defined-only", kvref], capture_output=True, text=True, check=True).stdout
    exported = [ln.split()[-1] for ln in syms.splitlines() if ln.split()[1:2] in (["T"], ["W"])]
    assert exported and all(s.startswith("_ZN3kvb19attention_reference") for s in exported), exported
