"""Headline benchmark: effective KV-read GB/s and us per decode step of paged_decode -> paged_reduce
on one MI355X, for BASELINE config c4 (fp16 cache, batch 4, 64 query / 8 KV heads, head_dim 128,
32768-token contexts, page 128, partition 2048, 1.25x shuffled pool, N(0,1) data).

A step is one decode step over inputs already resident in HBM: one launch of paged_decode with
the partition merge fused in (the reference's paged_decode + paged_reduce), preceded by a 1 GiB
read-only cache flush outside its hipEvent pair (cold HBM, as the reference measures,
src/metal_attn.mm:266-276). value = algorithmic bytes (live K+V, q, out: src/workload.hpp:68-74) /
median step time. The same event pairs time the kernel for the roofline (one launch per pair). The reference's fp64 CPU path (oracle/_ref, else the C oracle) is timed on a
bounded sample of the same workload. Prints one JSON line.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
import __graft_entry__ as graft  # noqa: E402

HBM_PEAK_GBPS = 8000.0
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic_c4_decode.json")


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def timed_steps(kvb, dev, part, steps, warmup):
    """warmup + steps cold decode steps (one fused paged_decode launch each, its hipEvent pair on the
    library's stream); returns the per-step GPU ms and the wall time of the timed steps."""
    for _ in range(warmup):
        kvb.flush_gpu_caches()
        dev.run(part)
    kvb.synchronize()
    t0 = time.perf_counter()
    times = []
    for _ in range(steps):
        kvb.flush_gpu_caches()
        times.append(dev.run(part))
    kvb.synchronize()
    return times, time.perf_counter() - t0


def split_steps(kvb, dev, part, steps):
    """The reference's two-kernel form (paged_decode, then paged_reduce), timed per kernel."""
    out = []
    for _ in range(steps):
        kvb.flush_gpu_caches()
        out.append(dev.run_split(part))
    return statistics.median(d for d, _ in out), statistics.median(r for _, r in out)


def warm_chain(kvb, dev, part, steps=20):
    """Back-to-back steps with warm caches (one event pair around the chain)."""
    dev.run(part)
    return dev.run(part, steps=steps) / steps


def cpu_baseline(oracle, w, seconds_budget=20.0):
    """The reference's fp64 attention (oracle/_ref when built, else this build's C oracle) on a bounded
    sample of the workload: the first sequence (all its heads, full context)."""
    import numpy as np

    threads = max(1, min(16, os.cpu_count() or 1))
    s1 = type(w.shape)(1, w.shape.num_heads, w.shape.num_kv_heads, w.shape.head_dim)
    lens = w.lens[:1]
    q, k, v = w.q[:1], w.k[:1], w.v[:1]
    use_ref = oracle.ref is not None
    fn = oracle.ref_attention if use_ref else oracle.attention
    fn(s1, lens, w.max_len, q, k, v, threads=threads)  # warm-up
    times = []
    t_start = time.perf_counter()
    while len(times) < 3 and (time.perf_counter() - t_start) < seconds_budget:
        t0 = time.perf_counter()
        fn(s1, lens, w.max_len, q, k, v, threads=threads)
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    sample_bytes = float(lens.sum()) * w.shape.num_kv_heads * w.shape.head_dim * 2 * 2 + \
        w.shape.num_heads * w.shape.head_dim * 2 * 4
    return {
        "value": round(sample_bytes / med / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "reference" if use_ref else "port",
        "sample": f"sequence 0 of {w.shape.batch} ({w.shape.num_heads} heads x {int(lens[0])} tokens, fp16 K/V), "
                  f"median of {len(times)} runs after 1 warm-up: {med * 1e3:.1f} ms "
                  f"(~{med * w.shape.batch * 1e3:.0f} ms per full step)",
        "ms_per_step_extrapolated": round(med * w.shape.batch * 1e3, 2),
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--part", type=int, default=2048, help="partition tokens for c4 (BASELINE: >= 2048)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extras", action="store_true", help="skip the int8, warm and probe measurements")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (each GPU would run the same kernel "
              "on its own shard of sequences / KV heads); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    kvb = graft.load_package()
    if not kvb.gpu_available():
        print("bench.py: no GPU", file=sys.stderr)
        sys.exit(1)
    log(f"device: {kvb.device_name()}")
    t_setup = time.perf_counter()
    w, c, cfg = kvb.make_config("c4", threads=16)
    dev = kvb.DeviceCase(w, c)
    log(f"c4 ready in {time.perf_counter() - t_setup:.1f}s: {int(w.lens.sum())} tokens, pool {c.num_blocks} blocks")

    times, wall = timed_steps(kvb, dev, args.part, args.steps, args.warmup)
    med = statistics.median(times)
    decode_avg = statistics.mean(times)  # the step is one launch of the fused paged_decode kernel
    bytes_step = w.min_bytes()
    value = bytes_step / (med * 1e-3) / 1e9
    s = w.shape
    kv_bytes = float(w.lens.sum()) * s.num_kv_heads * s.head_dim * 2 * 2
    decode_bytes = kv_bytes + s.batch * s.num_heads * s.head_dim * 4  # live K+V rows and q
    achieved = decode_bytes / (decode_avg * 1e-3) / 1e9
    log(f"c4: step median {med * 1e3:.1f} us (mean {decode_avg * 1e3:.1f} us), {value:.0f} GB/s; "
        f"wall {wall:.3f}s for {args.steps} steps")

    traffic = None
    if os.path.exists(TRAFFIC_FILE):
        with open(TRAFFIC_FILE) as f:
            traffic = json.load(f).get("bytes_per_launch")

    extras = {}
    if not args.no_extras:
        ud, ur = split_steps(kvb, dev, args.part, 10)
        extras["unfused_decode_us"] = round(ud * 1e3, 2)
        extras["unfused_reduce_us"] = round(ur * 1e3, 2)
        extras["warm_chain_us"] = round(warm_chain(kvb, dev, args.part) * 1e3, 2)
        extras["warm_gbps"] = round(bytes_step / (extras["warm_chain_us"] * 1e-6) / 1e9, 1)
        probe = kvb.Buffer(4 << 30)
        probe.fill(1)
        kvb.run_read_bandwidth(probe)
        pt = [kvb.run_read_bandwidth(probe) for _ in range(5)]
        extras["probe_gbps"] = round((4 << 30) / (statistics.median(pt) * 1e-3) / 1e9, 1)
        extras["pct_of_probe"] = round(100 * value / extras["probe_gbps"], 1)
        probe.free()
        # the same shape with an int8 cache (per-(page, KV head) scales): the int8 / fp16 speed ratio
        dev.free()
        wi = kvb.Workload(s, "i8", list(w.lens), seed=32768, q_amp=1.0, dist="normal", threads=16)
        ci = kvb.PagedCache(wi, 128, 32768 * 131 + 128, pool_factor=1.25, poison=False)
        devi = kvb.DeviceCase(wi, ci)
        ti, _ = timed_steps(kvb, devi, args.part, args.steps, args.warmup)
        medi = statistics.median(ti)
        extras["int8_us_per_step"] = round(medi * 1e3, 2)
        extras["int8_gbps"] = round(wi.min_bytes() / (medi * 1e-3) / 1e9, 1)
        extras["int8_speedup_vs_fp16"] = round(med / medi, 3)
        devi.free()
        log(f"int8 c4-shape: {medi * 1e3:.1f} us ({extras['int8_speedup_vs_fp16']}x fp16)")
    else:
        dev.free()

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(graft.load_oracle(), w)
        log(f"cpu baseline: {cpu['sample']}, {cpu['value']} GB/s on {cpu['cores']} threads ({cpu['kind']})")

    line = {
        "metric": "effective KV-read GB/s (% of HBM peak) + us per decode step, 1 MI355X",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(med, 5),
        "us_per_step": round(med * 1e3, 2),
        "pct_hbm_peak": round(100 * value / HBM_PEAK_GBPS, 1),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16 storage, f32 math",
        "data": "synthetic: q, K, V ~ N(0,1), K/V rounded to fp16, shuffled block table over a 1.25x pool",
        "config": {"workload": "c4: fp16 paged decode, batch 4, 64 q / 8 KV heads (GQA 8), head_dim 128, "
                               "context 32768, page 128, partition %d, cold HBM (1 GiB flush per step)" % args.part,
                   "bytes_per_step": bytes_step, "timed_wall_s": round(wall, 4)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": traffic,
                     "kernel": "paged_decode", "kernel_avg_us": round(decode_avg * 1e3, 2),
                     "bytes_per_launch": decode_bytes},
        "cpu_baseline": cpu,
    }
    line.update(extras)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
