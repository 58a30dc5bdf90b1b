"""What a short decode step is made of on one MI355X: the dispatch floor of an empty kernel at several
grid sizes, c1's launch with every sequence empty, and c1's step, each timed cold (after the 1 GiB
read flush, as bench.py times a step) and warm (back to back, no flush), with the same hipEvent pairs
stamped by the dispatches. Run it under `rocprofv3 --kernel-trace --stats` to see the same launches
as the profiler times them.

usage: python3 kv-cache-bench_amd/bench/launch_floor.py [--reps N]
"""
from __future__ import annotations

import argparse
import os
import statistics
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
import __graft_entry__ as graft  # noqa: E402


def timed(kvb, fn, reps, cold):
    fn()
    out = []
    for _ in range(reps):
        if cold:
            kvb.flush_gpu_caches()
        out.append(fn() * 1e3)
    return statistics.median(out), min(out)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--reps", type=int, default=30)
    args = ap.parse_args()
    kvb = graft.load_package()
    if not kvb.gpu_available():
        sys.exit("no GPU")
    print(f"# {kvb.device_name()}", flush=True)
    w, c, cfg = kvb.make_config("c1")
    part = kvb.config_part(cfg, w)
    dev = kvb.DeviceCase(w, c)
    we = kvb.Workload(w.shape, w.kv_type, [0] * w.shape.batch, seed=1)
    de = kvb.DeviceCase(we, kvb.PagedCache(we, 16, 1, poison=False))
    cases = [
        ("empty kernel, 1 workgroup of 64 threads", lambda: kvb.run_empty_grid(1, 64)),
        ("empty kernel, 1 workgroup of 256 threads", lambda: kvb.run_empty_grid(1, 256)),
        ("empty kernel, 32 workgroups of 256 (c1's grid)", lambda: kvb.run_empty_grid(32, 256)),
        ("empty kernel, 256 workgroups of 256 (one per CU)", lambda: kvb.run_empty_grid(256, 256)),
        ("empty kernel, 2048 workgroups of 256", lambda: kvb.run_empty_grid(2048, 256)),
        ("c1's launch, every sequence empty", lambda: de.run(part)),
        ("c1's step (fused paged_decode)", lambda: dev.run(part)),
        ("c1's decode alone, two-kernel form", lambda: dev.run_split(part)[0]),
        ("c1's paged_reduce, two-kernel form", lambda: dev.run_split(part)[1]),
        ("c1's loads alone", lambda: dev.run_loads(part)),
    ]
    print("| launch | cold median us | cold min us | warm median us | warm min us |")
    print("|---|---|---|---|---|")
    for name, fn in cases:
        cm, cn = timed(kvb, fn, args.reps, True)
        wm, wn = timed(kvb, fn, args.reps, False)
        print(f"| {name} | {cm:.2f} | {cn:.2f} | {wm:.2f} | {wn:.2f} |", flush=True)
    print(f"\nc1 kernel: `{dev.kernel_name(part)}`")
    de.free()
    dev.free()


if __name__ == "__main__":
    main()
