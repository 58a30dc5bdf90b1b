"""The kernels' own HIP source on the CPU: tests/kernel_emu compiles kv-cache-bench_amd/csrc for a CPU
emulation of the gfx950 execution model (wave64 lanes as fibers, MFMA, DPP, transposing LDS reads,
range-checked buffer loads) into a libkvb_hip.so with the same C ABI, and the GPU test files run on
it unchanged (tests/kernel_emu/run_gpu_tests.py). The mutation harness plants kernel mistakes in
that source and checks them the same way (tests/mutation/mutate.py, group hip).

Under AddressSanitizer (make -C tests/kernel_emu asan) every plain load and store of the kernels is
checked as well; that build runs the cases only the emulation may run: device lengths that disagree
with the host's (tests/kernel_emu/cases_emu_only.py).

The emulation itself is pinned two ways: its cross-lane operations against their documented
definitions (lane_ops_kat, which tests/test_lane_ops_gpu.py also runs on the MI355X), and the faults
it must stop a launch for (emu_faults)."""
import os
import subprocess
import sys

import pytest

from conftest import ROOT, progress

EMU = os.path.join(ROOT, "tests", "kernel_emu")
BUILD = os.path.join(EMU, "build")


ASAN_BUILD = os.path.join(EMU, "build-asan")


@pytest.fixture(scope="module")
def emu_build():
    need = ("libkvb_hip.so", "libkvb_host.so", "emu_faults", "lane_ops_kat")
    if not all(os.path.exists(os.path.join(BUILD, f)) for f in need):
        subprocess.run(["make", "-j", str(min(8, os.cpu_count() or 1)), "-C", EMU, "all"], check=True)
    return BUILD


def _run(cmd, timeout):
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=timeout, cwd=ROOT)
    return r.returncode, r.stdout + r.stderr


def test_cross_lane_operations_known_answers(emu_build):
    rc, out = _run([os.path.join(emu_build, "lane_ops_kat")], 120)
    assert rc == 0 and "PASSED" in out, out


def test_emulation_reports_faults(emu_build):
    rc, out = _run([os.path.join(emu_build, "emu_faults")], 120)
    assert rc == 0 and "PASSED" in out, out


def test_gpu_tests_pass_on_the_emulated_kernels(emu_build):
    progress("[emu] the GPU test files on the CPU emulation of the kernels (about 2.5 minutes)")
    rc, out = _run([sys.executable, os.path.join(EMU, "run_gpu_tests.py"), "--build-dir", emu_build], 1800)
    tail = "\n".join(out.strip().splitlines()[-30:])
    progress(f"[emu] {tail.splitlines()[-1] if tail else ''}")
    assert rc == 0, tail


def test_lengths_the_host_did_not_check_under_address_sanitizer(emu_build):
    """The kernels given device lengths that disagree with the host's (cases_emu_only.py), in the
    AddressSanitizer build: every plain load and store is checked as well as every buffer access."""
    if not all(os.path.exists(os.path.join(ASAN_BUILD, f)) for f in ("libkvb_hip.so", "libkvb_host.so")):
        subprocess.run(["make", "-j", str(min(8, os.cpu_count() or 1)), "-C", EMU, "asan"], check=True)
    rc, out = _run([sys.executable, os.path.join(EMU, "run_gpu_tests.py"), "--asan", "-k", "disagree"], 1800)
    tail = "\n".join(out.strip().splitlines()[-30:])
    assert rc == 0, tail
