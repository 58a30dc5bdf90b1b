"""Per-workgroup timelines of one decode step, from the measurement build with workgroup timestamps
(make -C kv-cache-bench_amd timestamps -> kv-cache-bench_amd/build-ts).

For each BASELINE configuration named on the command line, runs cold steps (1 GiB read flush before
each) of three launches of paged_decode on the same cache, and summarises their stamps:
  fused    the step as kvb_run_paged runs it (the partition merge fused in);
  decode   the same kernel with the merge left to paged_reduce (the two-kernel form's first kernel);
  loads    the loads-only variant (kvb_run_paged_loads): every K/V load, no arithmetic.
Stamps (s_memrealtime, 100 MHz, relative to the launch's first workgroup start), per workgroup:
start, wave 0's loop end, the slowest wave's loop end, partition stores issued, stores acknowledged,
arrival count returned, merge done. Reported: the event time, the span of the stamps, percentiles of
starts, loop durations (wave 0) and loop ends, then the medians of each step of the epilogue: the
other waves' lag behind wave 0, the wave merge up to the stores issued, the stores' acknowledgement,
the arrival count, and (merging workgroups) the merge; and the time from the last loop end to the end.
A second table follows the workgroup that ended last through the same steps (the step's critical
path). Median over 5 launches after 1 discarded. Prints markdown tables per configuration.

With --heads=H, each configuration runs with H query heads (its KV heads, batch and lengths
unchanged), for the wide GQA groups. With --warm, no flush before the launches (caches and the previous launch as a decode loop leaves
them). With --where, also where the workgroups ran (wave 0's HW_ID and XCC_ID, stamped by the same build),
for the last launch of each form: loop durations and loop ends per XCD, and per rank of a workgroup
among those that ran on the same CU (by start time), which separates a CU's first workgroup from the
ones that shared or followed it.

usage: python3 kv-cache-bench_amd/bench/wg_timeline.py [--where] [--warm] [--heads=H] c2 [c3 c4 c5i8 ...]
"""
from __future__ import annotations

import ctypes
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
os.environ["KVB_BUILD_DIR"] = os.path.join(ROOT, "kv-cache-bench_amd", "build-ts")
sys.path.insert(0, ROOT)
import __graft_entry__ as graft  # noqa: E402

GROUPS, WORDS = 65536, 8  # kWgStampGroups, kWgStampWords in paged_decode_impl.hpp
COLUMNS = [("event_us", "event"), ("span_us", "stamp span"), ("wgs", "workgroups"), ("start_p50", "start p50"),
           ("start_max", "start max"), ("loop_p10", "loop p10"), ("loop_p50", "loop p50"), ("loop_p90", "loop p90"),
           ("loopend_p50", "loop end p50"), ("loopend_max", "loop end max"), ("lag_p50", "other waves' lag p50"),
           ("merge_w_p50", "wave merge + stores issued p50"), ("ack_p50", "stores acked p50"),
           ("count_p50", "arrival count p50"), ("mergers", "mergers"), ("merge_p50", "merge p50"),
           ("tail_us", "last loop end to end")]
LAST = [("l_loopend", "wave 0 loop end"), ("l_lag", "other waves' lag"), ("l_merge_w", "wave merge + stores issued"),
        ("l_ack", "stores acked"), ("l_count", "arrival count"), ("l_merge", "merge"), ("l_end", "end")]


def where_tables(t, start, loop_end):
    """Loop durations and ends by XCD and by a workgroup's rank on its CU, as markdown rows."""
    hw = (t[:, 7] & 0xFFFFFFFF).astype(np.int64)  # word 7: where wave 0 ran
    xcc = (t[:, 7] >> 32).astype(np.int64) & 0xF
    cu = (xcc << 16) | (((hw >> 13) & 7) << 8) | (((hw >> 12) & 1) << 4) | ((hw >> 8) & 15)
    loop = loop_end - start
    order = np.lexsort((start, cu))
    rank = np.zeros(len(cu), np.int64)
    prev, r = -1, 0
    for i in order:
        r = r + 1 if cu[i] == prev else 0
        rank[i], prev = r, cu[i]
    lines = [f"{len(np.unique(cu))} CUs used; per XCD:", "",
             "| XCD | workgroups | start p50 | loop p10 | loop p50 | loop p90 | loop end p50 | loop end max |",
             "|---|---|---|---|---|---|---|---|"]
    pct = lambda a, q: float(np.percentile(a, q))
    for x in np.unique(xcc):
        m = xcc == x
        lines.append(f"| {x} | {int(m.sum())} | {pct(start[m], 50):.2f} | {pct(loop[m], 10):.2f} | "
                     f"{pct(loop[m], 50):.2f} | {pct(loop[m], 90):.2f} | {pct(loop_end[m], 50):.2f} | "
                     f"{float(loop_end[m].max()):.2f} |")
    lines += ["", "per rank on the CU (0 = the CU's first workgroup):", "",
              "| rank | workgroups | start p50 | loop p10 | loop p50 | loop p90 | loop end p50 | loop end max |",
              "|---|---|---|---|---|---|---|---|"]
    for k in np.unique(rank):
        m = rank == k
        lines.append(f"| {k} | {int(m.sum())} | {pct(start[m], 50):.2f} | {pct(loop[m], 10):.2f} | "
                     f"{pct(loop[m], 50):.2f} | {pct(loop[m], 90):.2f} | {pct(loop_end[m], 50):.2f} | "
                     f"{float(loop_end[m].max()):.2f} |")
    return lines


def summarise(kvb, dev, part, mode, read, reps=6, where=None, warm=False):
    buf = np.zeros(GROUPS * WORDS, np.uint64)
    prev = 0
    rows = []
    for rep in range(reps):
        if not warm:
            kvb.flush_gpu_caches()
        if mode == "fused":
            ms = dev.run(part)
        elif mode == "decode":
            ms = dev.run_split(part)[0]
        else:
            ms = dev.run_loads(part)
        kvb.synchronize()
        if read(buf.ctypes.data, buf.size) != 0:
            raise RuntimeError("reading the workgroup stamps failed")
        ts = buf.reshape(-1, WORDS).astype(np.int64)
        valid = ts[:, 0] > prev  # written by this launch (workgroups with no tokens write none)
        prev = int(ts[:, :5].max())
        t = ts[valid]
        base = t[:, 0].min()
        start, loop_end, slowest, issued, acked = ((t[:, i] - base) / 100.0 for i in range(5))
        counted = t[:, 5] > 0
        count = np.where(counted, (t[:, 5] - base) / 100.0, acked)
        merged = t[:, 6] > 0
        done = np.where(merged, (t[:, 6] - base) / 100.0, count)
        end = float(done.max())
        if rep == 0:
            continue
        if where is not None and rep == reps - 1:
            where[:] = where_tables(t, start, loop_end)
        pct = lambda a, q: float(np.percentile(a, q)) if len(a) else 0.0
        loop = loop_end - start
        i = int(np.argmax(done))  # the workgroup that ended last
        rows.append({
            "event_us": ms * 1e3, "span_us": end, "wgs": int(valid.sum()),
            "start_p50": pct(start, 50), "start_max": float(start.max()),
            "loop_p10": pct(loop, 10), "loop_p50": pct(loop, 50), "loop_p90": pct(loop, 90),
            "loopend_p50": pct(loop_end, 50), "loopend_max": float(loop_end.max()),
            "lag_p50": pct(slowest - loop_end, 50), "merge_w_p50": pct(issued - slowest, 50),
            "ack_p50": pct(acked - issued, 50), "count_p50": pct(count[counted] - acked[counted], 50),
            "mergers": int(merged.sum()), "merge_p50": pct(done[merged] - count[merged], 50),
            "tail_us": end - float(loop_end.max()),
            "l_loopend": float(loop_end[i]), "l_lag": float(slowest[i] - loop_end[i]),
            "l_merge_w": float(issued[i] - slowest[i]), "l_ack": float(acked[i] - issued[i]),
            "l_count": float(count[i] - acked[i]), "l_merge": float(done[i] - count[i]), "l_end": float(done[i]),
        })
    return {k: float(np.median([r[k] for r in rows])) for k in rows[0]}


def main(args):
    show_where = "--where" in args
    heads = next((int(a.split("=", 1)[1]) for a in args if a.startswith("--heads=")), 0)
    args = [a for a in args if not a.startswith("--heads=")]
    warm = "--warm" in args
    configs = [a for a in args if a not in ("--where", "--warm")] or ["c2"]
    kvb = graft.load_package()
    if not kvb.gpu_available():
        sys.exit("wg_timeline: no GPU")
    print(f"device: {kvb.device_name()}; us, relative to the launch's first workgroup start\n")
    for cfg in configs:
        if heads:
            s = kvb.CONFIGS[cfg]["shape"]
            kvb.CONFIGS[cfg] = dict(kvb.CONFIGS[cfg], shape=kvb.Shape(s.batch, heads, s.num_kv_heads, s.head_dim))
        w, c, cfgd = kvb.make_config(cfg, threads=16)
        part = kvb.config_part(cfgd, w)
        read = getattr(kvb.hip, "kvb_wg_stamps_" + kvb.KV_NAMES[w.kv_type])
        read.argtypes, read.restype = [ctypes.c_void_p, ctypes.c_size_t], ctypes.c_int
        dev = kvb.DeviceCase(w, c)
        with_heads = f" with {heads} query heads" if heads else ""
        print(f"### {cfg}{with_heads}: partition {part}, {int(w.lens.sum())} tokens\n")
        print("| launch | " + " | ".join(h for _, h in COLUMNS) + " |")
        print("|---" * (len(COLUMNS) + 1) + "|")
        wheres, last = {}, {}
        for mode in ("fused", "decode", "loads"):
            wheres[mode] = []
            r = summarise(kvb, dev, part, mode, read, where=wheres[mode] if show_where else None, warm=warm)
            cells = [f"{r[k]:.0f}" if k in ("wgs", "mergers") else f"{r[k]:.2f}" for k, _ in COLUMNS]
            print(f"| {mode} | " + " | ".join(cells) + " |", flush=True)
            last[mode] = r
        print(f"\nThe workgroup that ended last, step by step (medians over the launches):\n")
        print("| launch | " + " | ".join(h for _, h in LAST) + " |")
        print("|---" * (len(LAST) + 1) + "|")
        for mode in ("fused", "decode"):
            print(f"| {mode} | " + " | ".join(f"{last[mode][k]:.2f}" for k, _ in LAST) + " |")
        print()
        for mode, lines in wheres.items():
            if lines:
                print(f"#### {cfg}, {mode}: where the workgroups ran (last launch)\n")
                print("\n".join(lines) + "\n", flush=True)
        dev.free()


if __name__ == "__main__":
    main(sys.argv[1:])
