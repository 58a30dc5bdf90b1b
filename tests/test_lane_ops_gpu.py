"""The known answers of the cross-lane operations (tests/kernel_emu/lane_ops_kat.hip: MFMA operand
layouts, transposing LDS reads, DPP, shuffles, readlane, ballot) on the MI355X. The same checks pass
on the CPU emulation (tests/test_kernel_emu.py), which pins the emulation's semantics of these
operations, and so its runs of the kernels, to the hardware's."""
import os
import subprocess

import pytest

from conftest import ROOT

pytestmark = pytest.mark.gpu
BIN = os.path.join(ROOT, "tests", "kernel_emu", "build", "lane_ops_kat_gfx950")


def test_cross_lane_operations_known_answers_on_the_gpu(gpu):
    assert os.path.exists(BIN), f"{BIN} is not built: make -C tests/kernel_emu"
    r = subprocess.run([BIN], capture_output=True, text=True, timeout=120)
    out = r.stdout + r.stderr
    assert r.returncode == 0 and "PASSED" in out, out
    assert out.count("ok: ") == 15, out
