#!/usr/bin/env python3
"""Runs the GPU test files on the CPU emulation of the kernels (tests/kernel_emu).

The package's HIP sources, compiled for the CPU emulation (make -C tests/kernel_emu), form a
libkvb_hip.so with the same C ABI. With KVB_BUILD_DIR pointing at that build the package loads it,
and the GPU tests run as they are: the same cases, the same oracle, the same tolerances and
bit-identity checks, on the kernels' own source code. Left out are the tests that measure the
hardware or need the HIP runtime itself: full-size configurations (hours on the emulation), the
4 GiB read probe, stream switching through libamdhip64, and the C++ programs and benchmarks that
load the GPU build. Graph capture is emulated: a captured stream records its work, and a launch of
the graph replays it in order.

With --asan the libraries are the AddressSanitizer build (make -C tests/kernel_emu asan), so every
plain load and store the kernels make is checked against its allocation, in addition to the
emulation's own checks of buffer accesses.

Usage:
  python tests/kernel_emu/run_gpu_tests.py [--build-dir DIR] [--asan] [--all] [-x] [-n WORKERS] [pytest args...]
--all adds the slow cases (about 25 minutes of CPU time); the default set takes about 6 minutes of
CPU time, spread over the workers.
"""
from __future__ import annotations

import argparse
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
BUILD = os.path.join(HERE, "build")
ASAN_BUILD = os.path.join(HERE, "build-asan")
CXX = "/opt/rocm/lib/llvm/bin/clang++"

FILES = ["tests/test_gpu_parity.py", "tests/test_gpu_groups.py", "tests/test_gpu_pair.py", "tests/test_gpu_merge.py",
         "tests/test_gpu_writer.py", "tests/test_gpu_graph.py", "tests/test_zz_no_alloc.py",
         "tests/kernel_emu/cases_emu_only.py"]  # (the last: lengths the host did not check)
# hardware measurements, or calls into the HIP runtime itself
HARDWARE = "not full_size and not stream_switch and not read_bandwidth"
# slow on the emulation (a minute or more each); --all runs them
SLOW = [
    "tests/test_gpu_writer.py::test_writer_c5_shape",
    "tests/test_gpu_parity.py::test_random_layouts[11]",
    "tests/test_gpu_parity.py::test_random_layouts[23]",
    "tests/test_gpu_parity.py::test_fused_merge_reads_fresh_partitions",
    "tests/test_gpu_graph.py::test_graph_replays_match_eager",
]


def command(build_dir: str, all_cases: bool, stop_first: bool, workers: int, extra: list[str]) -> list[str]:
    cmd = [sys.executable, "-m", "pytest", *FILES, "-m", "gpu", "-q", "-p", "no:cacheprovider", "-k", HARDWARE]
    if not all_cases:
        for node in SLOW:
            cmd += ["--deselect", node]
    if stop_first:
        cmd.append("-x")
    if workers > 1:
        cmd += ["-n", str(workers)]
    return cmd + extra


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--build-dir", help="the emulated build (default: tests/kernel_emu/build, or build-asan)")
    ap.add_argument("--asan", action="store_true", help="the AddressSanitizer build, with its runtime preloaded")
    ap.add_argument("--all", action="store_true", help="include the slow cases")
    ap.add_argument("-x", action="store_true", help="stop at the first failure")
    ap.add_argument("-n", type=int, default=min(8, os.cpu_count() or 1), help="pytest-xdist workers")
    args, extra = ap.parse_known_args(argv)
    args.build_dir = args.build_dir or (ASAN_BUILD if args.asan else BUILD)
    for lib in ("libkvb_hip.so", "libkvb_host.so"):
        if not os.path.exists(os.path.join(args.build_dir, lib)):
            print(f"{args.build_dir}/{lib} is not built: make -C tests/kernel_emu", file=sys.stderr)
            return 2
    env = dict(os.environ, KVB_BUILD_DIR=os.path.abspath(args.build_dir))
    if args.asan:
        runtime = subprocess.run([CXX, "-print-file-name=libclang_rt.asan-x86_64.so"], capture_output=True,
                                 text=True, check=True).stdout.strip()
        env["LD_PRELOAD"] = runtime
        # (Python and numpy are not instrumented: only the emulated libraries' accesses are checked)
        env["ASAN_OPTIONS"] = "detect_leaks=0:abort_on_error=1:allocator_may_return_null=1"
    return subprocess.run(command(args.build_dir, args.all, args.x, args.n, extra), cwd=ROOT, env=env).returncode


if __name__ == "__main__":
    sys.exit(main())
