"""Summarise the measurements of profile_groups.sh OUT into markdown (stdout), as kept in
profiles/paged_decode_groups.md: per storage type and GQA group at c4's size, the decode kernel's
name, its kernel-trace durations (the 30 timed dispatches) with the effective KV-read rate, kvbench's
own median, and the SQ counters per wave.

usage: python3 kv-cache-bench_amd/bench/prof_groups.py OUT
"""
from __future__ import annotations

import csv
import os
import statistics
import sys
from collections import defaultdict

B, HKV, D, LEN = 4, 8, 128, 32768
ESZ = {"f16": 2, "i8": 1}
SQ = ("SQ_INSTS_VALU", "SQ_INSTS_LDS", "SQ_INSTS_VMEM_RD", "SQ_WAVE_CYCLES", "SQ_BUSY_CYCLES", "SQ_WAIT_INST_ANY")


def min_bytes(t, g):  # Workload::min_bytes: live K and V, then q and out in fp32
    return B * HKV * LEN * D * 2 * ESZ[t] + 2 * B * HKV * g * D * 4


def decode_trace(path):
    rows = sorted(csv.DictReader(open(path)), key=lambda r: int(r["Dispatch_Id"]))
    dec = [r for r in rows if "paged_decode_kernel" in r["Kernel_Name"]]
    return dec[-30:]


def counters(path):
    per, names = defaultdict(dict), {}
    for r in csv.DictReader(open(path)):
        d = int(r["Dispatch_Id"])
        per[d][r["Counter_Name"]] = float(r["Counter_Value"])
        names[d] = r["Kernel_Name"]
    dec = [per[d] for d in sorted(per) if "paged_decode_kernel" in names[d]]
    return dec[-1]


def kvbench_median(path):
    for line in open(path):
        if line.startswith("gpu_paged,"):
            return float(line.split(",")[7])
    return float("nan")


def main(out):
    print("# paged_decode with 8 to 64 query heads per KV head — MI355X\n")
    print("Workload: batch 4, 8 KV heads, head_dim 128, context 32768, page 128, partition 4096, cold (1 GiB read "
          "flush per step); q, K, V ~ U(-1, 1) from kvbench's seeds, K/V stored as fp16 (RNE) or int8 per-(page, KV "
          "head) scales; shuffled block table.\n")
    print("## Commands (from the repository root on the GPU box)\n")
    print("```\nbash kv-cache-bench_amd/bench/profile_groups.sh gpurun_out/prof_groups\n```\n")
    print("For each storage type t and group G (query heads H = 8 G), from /tmp with TMPDIR=/tmp (R = the repository "
          "root, A = `--batch=4 --heads=H --kv-heads=8 --dim=128 --lens=32768 --pages=128 --parts=4096 --types=t "
          "--no-cpu --no-naive`):\n")
    print("```\nrocprofv3 --kernel-trace --stats -d OUT -o run --output-format csv -- $R/kv-cache-bench_amd/build/kvbench A "
          "--reps=30 --warmup=3\nrocprofv3 --pmc SQ_WAVES SQ_INSTS_VALU SQ_INSTS_LDS SQ_INSTS_SALU SQ_INSTS_VMEM_RD "
          "SQ_WAVE_CYCLES SQ_BUSY_CYCLES SQ_WAIT_INST_ANY GRBM_GUI_ACTIVE -d OUT -o run --output-format csv -- "
          "$R/kv-cache-bench_amd/build/kvbench A --reps=10 --warmup=1\n"
          "python3 $R/kv-cache-bench_amd/bench/prof_groups.py OUT\n```\n")
    print("## Kernel trace (the 30 timed dispatches) and kvbench's median\n")
    print("| storage | group | workgroups x waves | avg us | min us | max us | kvbench median us | GB/s (avg) | "
          "% of 8 TB/s |")
    print("|---|---|---|---|---|---|---|---|---|")
    names = []
    for t in ("f16", "i8"):
        for g in (8, 16, 32, 64):
            d = os.path.join(out, f"{t}_g{g}")
            tr = decode_trace(os.path.join(d, "trace", "run_kernel_trace.csv"))
            us = [(int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3 for r in tr]
            avg = statistics.mean(us)
            gbps = min_bytes(t, g) / (avg * 1e-6) / 1e9
            r0 = tr[0]
            wg = 1
            for ax in "XYZ":
                wg *= int(r0[f"Grid_Size_{ax}"]) // int(r0[f"Workgroup_Size_{ax}"])
            waves = int(r0["Workgroup_Size_X"]) * int(r0["Workgroup_Size_Y"]) * int(r0["Workgroup_Size_Z"]) // 64
            names.append((t, g, r0["Kernel_Name"], r0["VGPR_Count"], r0["Accum_VGPR_Count"], r0["LDS_Block_Size"]))
            print(f"| {t} | {g} | {wg} x {waves} | {avg:.2f} | {min(us):.2f} | {max(us):.2f} | "
                  f"{kvbench_median(os.path.join(d, 'kvbench.csv')):.2f} | {gbps:.0f} | {gbps / 80:.1f} |")
    print("\nAlgorithmic bytes per launch: live K+V, q and out (`Workload::min_bytes`); 537 MB fp16, 269 MB int8 "
          "(plus 0.26-2.1 MB of q and out).\n")
    print("## Kernels (as rocprofv3 reports them)\n")
    print("| storage | group | kernel | VGPR_Count | Accum_VGPR_Count | LDS_Block_Size |")
    print("|---|---|---|---|---|---|")
    for t, g, n, v, a, l in names:
        print(f"| {t} | {g} | `{n}` | {v} | {a} | {l} |")
    print("\n## SQ counters per wave (the last timed dispatch)\n")
    print("SQ_WAVE_CYCLES, SQ_BUSY_CYCLES and SQ_WAIT_INST_ANY count in units of 4 cycles.\n")
    print("| storage | group | waves | " + " | ".join(k[3:] for k in SQ) + " |")
    print("|---|---|---|" + "---|" * len(SQ))
    for t in ("f16", "i8"):
        for g in (8, 16, 32, 64):
            c = counters(os.path.join(out, f"{t}_g{g}", "sq", "run_counter_collection.csv"))
            w = c["SQ_WAVES"]
            print(f"| {t} | {g} | {int(w)} | " + " | ".join(f"{c[k] / w:.0f}" for k in SQ) + " |")


if __name__ == "__main__":
    main(sys.argv[1])
