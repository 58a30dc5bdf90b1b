"""Summarise the measurements of profile.sh CONFIG OUT into markdown (stdout), as kept in
profiles/paged_decode_<CONFIG>.md, and write OUT/traffic.json: the kernel's name, its per-launch HBM
traffic and L2 hit rate, which bench.py --config CONFIG reports as roofline.traffic and
roofline.tcc_hit_rate (kept as profiles/traffic_<CONFIG>.json) when the kernel it launches has that
name.

Dispatches of one `bench.py --no-extras` run, in order: the library's set-up fill, the flush
buffer's 1 GiB fill, then (1 GiB flush read, paged_decode) per step, warm-up steps first. The
calibration kernels are the 1 GiB flush read (FETCH_SIZE) and the 1 GiB fill (WRITE_SIZE), whose
byte counts are known.

usage: python3 kv-cache-bench_amd/bench/prof_summary.py CONFIG OUT
"""
from __future__ import annotations

import csv
import json
import os
import statistics
import sys
from collections import defaultdict

GiB = 1 << 30


def load_json_line(path):
    with open(path) as f:
        return json.loads(f.read().strip().splitlines()[-1])


def kind(name):
    if "paged_decode_kernel" in name:
        return "decode"
    if "read_bw_kernel" in name:
        return "read"
    if "fill_kernel" in name:
        return "fill"
    return name


def trace_rows(out):
    path = os.path.join(out, "trace", "run_kernel_trace.csv")
    rows = sorted(csv.DictReader(open(path)), key=lambda r: int(r["Dispatch_Id"]))
    return [(kind(r["Kernel_Name"]), r["Kernel_Name"], (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3,
             r) for r in rows]


def counter_rows(out, sub):
    path = os.path.join(out, sub, "run_counter_collection.csv")
    per = defaultdict(dict)
    names = {}
    for r in csv.DictReader(open(path)):
        d = int(r["Dispatch_Id"])
        per[d][r["Counter_Name"]] = float(r["Counter_Value"])
        names[d] = r["Kernel_Name"]
    return [(kind(names[d]), per[d]) for d in sorted(per)]


def main(cfg, out):
    line = load_json_line(os.path.join(out, "bench.json"))
    steps = 30
    algo = float(line["config"]["bytes_per_step"])
    tr = trace_rows(out)
    dec = [(t, r) for k, _, t, r in tr if k == "decode"]
    timed = dec[-steps:]
    dur = [t for t, _ in timed]
    kname = timed[0][1]["Kernel_Name"]
    reads = [t for k, _, t, _ in tr if k == "read"]
    avg = statistics.mean(dur)

    # traffic per launch from the counter passes (10 timed steps each), calibrated on the flush
    fetch = counter_rows(out, "fetch")
    write = counter_rows(out, "write")
    f_dec = [c["FETCH_SIZE"] for k, c in fetch if k == "decode"][-10:]
    f_read = [c["FETCH_SIZE"] for k, c in fetch if k == "read"]
    w_dec = [c["WRITE_SIZE"] for k, c in write if k == "decode"][-10:]
    w_fill = max(c["WRITE_SIZE"] for k, c in write if k == "fill")
    f_factor = (GiB / 1024) / statistics.median(f_read)
    w_factor = (GiB / 1024) / w_fill
    fetch_kib, write_kib = statistics.mean(f_dec), statistics.mean(w_dec)
    traffic = fetch_kib * 1024 * f_factor + write_kib * 1024 * w_factor

    tcc = counter_rows(out, "tcc")
    t_dec = [c for k, c in tcc if k == "decode"][-10:]
    t_read = [c for k, c in tcc if k == "read"]

    def hit_rate(rows):
        hit = sum(c["TCC_HIT_sum"] for c in rows)
        return hit / (hit + sum(c["TCC_MISS_sum"] for c in rows))

    dec_hit, read_hit = hit_rate(t_dec), hit_rate(t_read)

    sq = [c for k, c in counter_rows(out, "sq") if k == "decode"][-10:]
    sq_names = sorted(sq[0])
    waves = statistics.mean(c["SQ_WAVES"] for c in sq)

    print(f"# paged_decode on {cfg} — MI355X\n")
    print(f"Workload: {line['config']['workload']}; K/V stored as {line['config']['kv_storage']}; "
          f"{line['data']}.\n")
    print(f"Kernel: `{kname}` (grid {timed[0][1]['Grid_Size_X']} threads, {timed[0][1]['VGPR_Count']} arch VGPR + "
          f"{timed[0][1]['Accum_VGPR_Count']} AGPR, LDS {timed[0][1]['LDS_Block_Size']} B).\n")
    print("## Commands (from the repository root on the GPU box)\n")
    print("```")
    root = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
    print(f"bash kv-cache-bench_amd/bench/profile.sh {cfg} {os.path.relpath(out, root)}")
    print("```\n")
    print("That script runs, from /tmp with TMPDIR=/tmp (R = the repository root):\n")
    print("```")
    print(f"python3 $R/bench.py --no-cpu --config {cfg}")
    for what in ("--kernel-trace --stats", "--pmc FETCH_SIZE", "--pmc WRITE_SIZE", "--pmc TCC_HIT_sum TCC_MISS_sum",
                 "--pmc SQ_WAVES SQ_INSTS_VALU SQ_INSTS_LDS SQ_INSTS_SALU SQ_INSTS_VMEM_RD SQ_WAVE_CYCLES "
                 "SQ_BUSY_CYCLES SQ_WAIT_INST_ANY GRBM_GUI_ACTIVE"):
        n = 30 if "trace" in what else 10
        print(f"rocprofv3 {what} -d OUT -o run --output-format csv -- "
              f"python3 $R/bench.py --no-cpu --no-extras --config {cfg} --steps {n}")
    print(f"python3 $R/kv-cache-bench_amd/bench/wg_timeline.py {cfg}")
    print(f"python3 $R/kv-cache-bench_amd/bench/prof_summary.py {cfg} OUT")
    print("```\n")

    print("## bench.py (plain run, hipEvent pairs stamped by the dispatches; cold = after a 1 GiB flush read)\n")
    keys = [("us_per_step", "step, cold (median of 30)"), ("unfused_decode_us", "paged_decode alone, two-kernel form"),
            ("unfused_reduce_us", "paged_reduce, two-kernel form"), ("loads_only_us", "the decode's loads alone"),
            ("warm_step_us", "step, warm (no flush, one launch each)"), ("warm_chain_us", "step, warm chain of 20"),
            ("graph_chain_us", "step, warm, 20 replayed from one HIP graph"),
            ("empty_step_us", "the same launch with every sequence empty"),
            ("int8_us_per_step", "c4's shape with an int8 cache"), ("int8_loads_only_us", "its loads alone")]
    print("| measurement | us |")
    print("|---|---|")
    for k, what in keys:
        if k in line:
            print(f"| {what} | {line[k]} |")
    print(f"\nvalue {line['value']} GB/s ({line['pct_hbm_peak']}% of 8 TB/s"
          + (f", {line['pct_of_probe']}% of the {line['probe_gbps']} GB/s read probe" if "probe_gbps" in line else "")
          + f"); roofline.achieved {line['roofline']['achieved']} GB/s from the event mean "
            f"{line['roofline']['kernel_avg_us']} us.\n")

    print("## Kernel trace (the 30 timed dispatches)\n")
    print("| kernel | dispatches | avg us | min us | max us | GB/s (avg) | % of 8 TB/s |")
    print("|---|---|---|---|---|---|---|")
    print(f"| paged_decode (fused step) | {len(dur)} | {avg:.2f} | {min(dur):.2f} | {max(dur):.2f} | "
          f"{algo / (avg * 1e-6) / 1e9:.0f} | {100 * algo / (avg * 1e-6) / 8e12:.1f} |")
    print(f"| read_bw, 1 GiB flush (ordinary loads) | {len(reads)} | {statistics.mean(reads):.2f} | "
          f"{min(reads):.2f} | {max(reads):.2f} | {GiB / (statistics.mean(reads) * 1e-6) / 1e9:.0f} | |")
    print(f"\nAlgorithmic bytes per launch: {algo:.0f} (live K+V, q and out: `Workload::min_bytes`).\n")

    print("## HBM traffic per launch (FETCH_SIZE, WRITE_SIZE; KiB per dispatch, mean of the 10 timed)\n")
    print(f"Calibration in the same runs: the 1 GiB flush read reports FETCH_SIZE {statistics.median(f_read):.0f} KiB "
          f"(factor {f_factor:.4f} to bytes / 1024); the 1 GiB fill reports WRITE_SIZE {w_fill:.0f} KiB "
          f"(factor {w_factor:.4f}).\n")
    print("| FETCH_SIZE KiB | WRITE_SIZE KiB | traffic, calibrated (B) | algorithmic (B) | ratio |")
    print("|---|---|---|---|---|")
    print(f"| {fetch_kib:.0f} | {write_kib:.0f} | {traffic:.0f} | {algo:.0f} | {traffic / algo:.4f} |\n")

    print("## L2 (TCC) hit rate (TCC_HIT_sum / (TCC_HIT_sum + TCC_MISS_sum), the 10 timed dispatches)\n")
    print("Every K/V byte is read once per step, so the decode's hits are requests for a line that an earlier "
          "request already brought in. One K load instruction reads 16 bytes per lane for 16 tokens (the MFMA "
          "operand layout): 64 bytes of each of 16 rows at fp16 and int8, so each 128-byte K line is two "
          "requests and the second hits. One V load instruction reads whole rows, a request per line. K and V "
          "are half the lines each, which gives one hit per two misses: a rate of 1/3. Misses equal the lines "
          "read (algorithmic bytes / 128). The 1 GiB flush read in the same run is a plain streaming read for "
          "comparison.\n")
    print("| kernel | TCC_HIT_sum | TCC_MISS_sum | hit rate |")
    print("|---|---|---|---|")
    for what, rows, rate in (("paged_decode", t_dec, dec_hit), ("read_bw, 1 GiB flush", t_read, read_hit)):
        print(f"| {what} | {statistics.mean(c['TCC_HIT_sum'] for c in rows):.0f} | "
              f"{statistics.mean(c['TCC_MISS_sum'] for c in rows):.0f} | {rate:.4f} |")
    print()

    print("## SQ counters, paged_decode (mean per timed dispatch, and per wave)\n")
    print("SQ_WAVE_CYCLES, SQ_BUSY_CYCLES and SQ_WAIT_INST_ANY count in units of 4 cycles; GRBM_GUI_ACTIVE is "
          "the value rocprofv3 reports for the dispatch.\n")
    print("| counter | per dispatch | per wave |")
    print("|---|---|---|")
    for n in sq_names:
        m = statistics.mean(c[n] for c in sq)
        print(f"| {n} | {m:.0f} | {m / waves:.1f} |")
    print()
    print("## Per-workgroup timeline (measurement build with workgroup timestamps, build-ts/)\n")
    with open(os.path.join(out, "timeline.md")) as f:
        print(f.read().strip())
    with open(os.path.join(out, "traffic.json"), "w") as f:
        json.dump({"config": cfg, "kernel_name": kname, "bytes_per_launch": round(traffic),
                   "algorithmic_bytes": round(algo), "fetch_kib": fetch_kib, "write_kib": write_kib,
                   "fetch_factor": f_factor, "write_factor": w_factor, "tcc_hit_rate": round(dec_hit, 4),
                   "trace_avg_us": round(avg, 2), "bench_us_per_step": line["us_per_step"],
                   "env": line.get("env"), "source": f"paged_decode_{cfg}.md"}, f, indent=1)


if __name__ == "__main__":
    main(sys.argv[1], sys.argv[2])
