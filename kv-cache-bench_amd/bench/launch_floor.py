"""What a short decode step is made of on one MI355X: the dispatch floor of an empty kernel at several
grid sizes, c1's launch with every sequence empty, and c1's step, each timed cold (after the 1 GiB
read flush, as bench.py times a step) and warm (back to back, no flush), with the same hipEvent pairs
stamped by the dispatches. Run it under `rocprofv3 --kernel-trace --stats` to see the same launches
as the profiler times them.

usage: python3 kv-cache-bench_amd/bench/launch_floor.py [--reps N]
       python3 kv-cache-bench_amd/bench/launch_floor.py --trace DIR   (summarise DIR/run_kernel_trace.csv,
           a rocprofv3 --kernel-trace of the first form: each kernel and grid, dispatched right after the
           flush (cold) or not (warm), with the profiler's durations)
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


def summarise_trace(out):
    """Median profiler duration per (kernel, workgroups, cold/warm), in dispatch order of first use."""
    import csv
    rows = sorted(csv.DictReader(open(os.path.join(out, "run_kernel_trace.csv"))), key=lambda r: int(r["Dispatch_Id"]))
    groups, order, prev = {}, [], None
    for i, r in enumerate(rows):
        name = r["Kernel_Name"]
        if "paged_decode_kernel" in name and i + 1 < len(rows) and "paged_reduce" in rows[i + 1]["Kernel_Name"]:
            name += " [two-kernel form]"
        wgs = int(r["Grid_Size_X"]) * int(r["Grid_Size_Y"]) * int(r["Grid_Size_Z"]) // (
            int(r["Workgroup_Size_X"]) * int(r["Workgroup_Size_Y"]) * int(r["Workgroup_Size_Z"]))
        dur = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
        flush = "read_bw_kernel<false>" in name
        if not flush and "fill_kernel" not in name and "copyBuffer" not in name:
            key = (name, wgs, int(r["Workgroup_Size_X"]), "cold" if prev == "flush" else "warm")
            if key not in groups:
                groups[key] = []
                order.append(key)
            groups[key].append(dur)
        prev = "flush" if flush or (prev == "flush" and "[two-kernel form]" in name) else "other"
    print("| kernel | workgroups x threads | in a cold step (after the flush) | dispatches | median us | min us |")
    print("|---|---|---|---|---|---|")
    for key in order:
        v = groups[key]
        print(f"| `{key[0]}` | {key[1]} x {key[2]} | {'yes' if key[3] == 'cold' else 'no'} | "
              f"{len(v)} | {statistics.median(v):.2f} | {min(v):.2f} |")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--reps", type=int, default=30)
    ap.add_argument("--trace", default=None)
    args = ap.parse_args()
    if args.trace:
        return summarise_trace(args.trace)
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
