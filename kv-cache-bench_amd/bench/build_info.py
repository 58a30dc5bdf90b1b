"""Source identity of a build and the environment record of a result (the counterpart of the
reference's scripts/env.sh, which saves machine, toolchain, commit and load beside every result set).

`python3 build_info.py OUT` (run by the package Makefile) writes OUT, a JSON record of the build: the
git commit and whether tracked files differed from it, the sha256 of the sources the libraries are
built from, the time and the hipcc version. The GPU box receives the tree without .git, so a result
measured there names its build through this file; `sources_sha256` recomputed at run time shows
whether the sources on the box are the ones built.

`env_record(kvb)` is the environment object of a bench line: that source identity, the HIP runtime
and driver versions and the device (kvb_device_info), the ROCm release, the CPU and the load average
before the run. `python3 build_info.py --env` prints it as JSON (sweep.sh saves it as env.json).
"""
from __future__ import annotations

import hashlib
import json
import os
import platform
import subprocess
import sys
import time

PKG = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ROOT = os.path.dirname(PKG)
BUILD_INFO = os.path.join(PKG, "build", "build_info.json")


def source_files():
    """The files the libraries and kvbench are built from, in a fixed order."""
    out = []
    for d, exts in ((os.path.join(PKG, "csrc"), (".hip", ".hpp")), (os.path.join(PKG, "host"), (".cpp",)),
                    (os.path.join(ROOT, "include"), (".h",)), (os.path.join(ROOT, "include", "kvb"), (".hpp",))):
        out += sorted(os.path.join(d, f) for f in os.listdir(d) if f.endswith(exts))
    out += [os.path.join(PKG, "bench", "kvbench.cpp"), os.path.join(PKG, "Makefile")]
    return out


def sources_sha256() -> str:
    h = hashlib.sha256()
    for p in source_files():
        h.update(os.path.relpath(p, ROOT).encode() + b"\0")
        with open(p, "rb") as f:
            h.update(f.read())
    return h.hexdigest()


def git_state():
    """(commit, dirty) from git, or (None, None) where there is no repository (the GPU box)."""
    try:
        commit = subprocess.run(["git", "-C", ROOT, "rev-parse", "HEAD"], capture_output=True, text=True,
                                timeout=10).stdout.strip()
        if not commit:
            return None, None
        st = subprocess.run(["git", "-C", ROOT, "status", "--porcelain", "--untracked-files=no"],
                            capture_output=True, text=True, timeout=10)
        return commit, bool(st.stdout.strip()) if st.returncode == 0 else None
    except (OSError, subprocess.SubprocessError):
        return None, None


def hipcc_version() -> str:
    try:
        out = subprocess.run(["/opt/rocm/bin/hipcc", "--version"], capture_output=True, text=True, timeout=30).stdout
        return next((l.split(":", 1)[1].strip() for l in out.splitlines() if l.startswith("HIP version")), "unknown")
    except (OSError, subprocess.SubprocessError):
        return "unknown"


def build_record() -> dict:
    commit, dirty = git_state()
    return {"commit": commit, "dirty": dirty, "sources_sha256": sources_sha256(),
            "built_at": time.strftime("%Y-%m-%dT%H:%M:%SZ", time.gmtime()), "hipcc": hipcc_version()}


def read_text(path, default="unknown"):
    try:
        with open(path) as f:
            return f.read().strip()
    except OSError:
        return default


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            return next((l.split(":", 1)[1].strip() for l in f if l.startswith("model name")), "unknown")
    except OSError:
        return "unknown"


def cpu_threads() -> int:
    """The CPUs this process may run on (the counterpart of std::thread::hardware_concurrency)."""
    try:
        return len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        return os.cpu_count() or 1


def env_record(kvb, loadavg=None) -> dict:
    """The environment of a result. `loadavg`: os.getloadavg() taken before the run (now if None)."""
    built = {}
    try:
        with open(BUILD_INFO) as f:
            built = json.load(f)
    except (OSError, ValueError):
        pass
    commit, dirty = git_state()
    src = sources_sha256()
    dev = kvb.device_info()
    la = loadavg if loadavg is not None else os.getloadavg()
    return {
        "commit": commit or built.get("commit"),
        "dirty": dirty if commit else built.get("dirty"),
        "commit_from": "git" if commit else ("build_info" if built else None),
        "sources_sha256": src,
        "sources_match_build": (built.get("sources_sha256") == src) if built else None,
        "built_at": built.get("built_at"),
        "hipcc": built.get("hipcc"),
        "hip_runtime_version": dev["runtime_version"],
        "hip_driver_version": dev["driver_version"],
        "rocm": read_text("/opt/rocm/.info/version"),
        "device": dev["name"],
        "arch": dev["arch"],
        "pci_bus_id": dev["pci_bus_id"],
        "compute_units": dev["compute_units"],
        "sclk_mhz": dev["clock_khz"] // 1000,
        "mclk_mhz": dev["memory_clock_khz"] // 1000,
        "memory_bus_bits": dev["memory_bus_bits"],
        "hbm_gib": round(dev["total_memory"] / 2 ** 30, 1),
        "hbm_free_gib": round(dev["free_memory"] / 2 ** 30, 1),
        "cpu": cpu_model(),
        "cpu_logical": os.cpu_count(),
        "cpu_threads": cpu_threads(),
        "loadavg_before": [round(x, 2) for x in la],
        "kernel": platform.release(),
        "python": platform.python_version(),
    }


if __name__ == "__main__":
    if sys.argv[1:] == ["--env"]:  # the environment record of a result set, now (needs the GPU library)
        sys.path.insert(0, ROOT)
        import __graft_entry__ as graft

        sys.stdout.write(json.dumps(env_record(graft.load_package()), indent=1) + "\n")
        sys.exit(0)
    rec = build_record()
    text = json.dumps(rec, indent=1) + "\n"
    if len(sys.argv) > 1:
        os.makedirs(os.path.dirname(os.path.abspath(sys.argv[1])), exist_ok=True)
        with open(sys.argv[1], "w") as f:
            f.write(text)
    else:
        sys.stdout.write(text)
