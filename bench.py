"""Headline benchmark: effective KV-read GB/s and us per decode step of the paged decode path
(the reference's paged_decode -> paged_reduce) on one MI355X. Default: BASELINE config c4 (fp16
cache, batch 4, 64 query / 8 KV heads, head_dim 128, 32768-token contexts, page 128, partition
chosen from the length by the MI355X policy (4096), 1.25x shuffled pool, N(0,1) data);
--config c1|c2|c3|c5f16|c5i8 measures another BASELINE config with the same contract.

A step is one decode step over inputs already resident in HBM: one launch of paged_decode with the
partition merge fused in, preceded by a 1 GiB read-only cache flush outside its hipEvent pair (cold
HBM, as the reference measures, src/metal_attn.mm:266-276). value = algorithmic bytes (live K+V, q,
out: src/workload.hpp:68-74) / median step time. The same event pairs time the kernel for the
roofline (one launch per pair). The reference's fp64 CPU path (oracle/_ref, else the C oracle) is
timed on a bounded sample of the same workload. Prints one JSON line.
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
sys.path.insert(0, os.path.join(ROOT, "kv-cache-bench_amd", "bench"))
import build_info  # noqa: E402  (the environment record)


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


def loads_only(kvb, dev, part, steps=10):
    """The decode's loads alone (kvb_run_paged_loads), cold: the memory-traffic floor of the kernel."""
    out = []
    for _ in range(steps):
        kvb.flush_gpu_caches()
        out.append(dev.run_loads(part))
    return statistics.median(out)


def warm_chain(kvb, dev, part, steps=20):
    """Back-to-back steps with warm caches (one event pair around the chain)."""
    dev.run(part)
    return dev.run(part, steps=steps) / steps


def graph_chain(kvb, dev, part, steps=20, launches=5):
    """Warm back-to-back steps replayed from a captured HIP graph (kvb_graph_capture_paged): the
    steps of a serving loop with one launch per `steps`; per-step time, median over launches."""
    graph = dev.capture_graph(part, steps)
    try:
        graph.launch()
        return statistics.median(graph.launch() for _ in range(launches)) / steps
    finally:
        graph.free()


def warm_steps(kvb, dev, part, steps=30):
    """Single steps with no flush between them (one launch and event pair each, waited for): beside
    the cold steps, what the flush changes."""
    dev.run(part)
    return statistics.median(dev.run(part) for _ in range(steps))


def empty_steps(kvb, w, part, steps=30):
    """The same launch (shape, partition, grid of one partition per head group) with every sequence
    empty: each workgroup writes its zero output and exits. The floor that dispatch and the event pair
    put under any step of this shape."""
    we = kvb.Workload(w.shape, w.kv_type, [0] * w.shape.batch, seed=1)
    de = kvb.DeviceCase(we, kvb.PagedCache(we, 16, 1, poison=False))
    de.run(part)
    t = statistics.median(de.run(part) for _ in range(steps))
    de.free()
    return t


def cpu_threads():
    """Threads for the CPU baseline: every CPU this process may run on, the counterpart of the
    reference's std::thread::hardware_concurrency (bench/bench.cpp:94)."""
    return max(1, build_info.cpu_threads())


def cpu_model():
    """The host CPU's model name (/proc/cpuinfo), and the core count the OS reports."""
    return f"{build_info.cpu_model()}, {os.cpu_count()} logical CPUs"


def traffic_record(config, kernel):
    """profiles/traffic_<config>.json, the per-launch HBM traffic and L2 hit rate that rocprofv3
    counters gave for this configuration (prof_summary.py), and None in its place (with the reason)
    unless it was measured on the kernel this run launches: a record whose kernel name differs
    describes other code."""
    path = os.path.join(ROOT, "profiles", f"traffic_{config}.json")
    if not os.path.exists(path):
        return None, f"no {os.path.relpath(path, ROOT)}"
    with open(path) as f:
        rec = json.load(f)
    if rec.get("kernel_name") != kernel:
        return None, f"{os.path.relpath(path, ROOT)} was measured on {rec.get('kernel_name')!r}, this run launches {kernel!r}"
    return rec, None


def cpu_baseline(kvb, oracle, w, c, seconds_budget=20.0, max_bytes=1 << 30):
    """The reference's fp64 attention (oracle/_ref when built, else this build's C oracle), timed on
    the whole step when its stored K/V fit in max_bytes (every configuration but the ragged c5), else
    on the longest prefix of sequences that fits (at least one non-empty one): all heads, full
    context. int8 caches are dequantised first (outside the timing), as the reference's
    PagedCache::reference does."""
    threads = cpu_threads()
    esz = {kvb.KV_F32: 4, kvb.KV_F16: 2, kvb.KV_I8: 1}[w.kv_type]
    row = w.shape.num_kv_heads * w.shape.head_dim * esz * 2  # stored K + V bytes per token
    n, tokens = 0, 0
    for L in w.lens:
        if tokens > 0 and (tokens + int(L)) * row > max_bytes:
            break
        n, tokens = n + 1, tokens + int(L)
    full = n == w.shape.batch
    sn = type(w.shape)(n, w.shape.num_heads, w.shape.num_kv_heads, w.shape.head_dim)
    lens = w.lens[:n]
    if w.kv_type == kvb.KV_I8:
        kd, vd = c.dequantized(w)
        k, v = kd[:n], vd[:n]
    else:
        k, v = w.k[:n], w.v[:n]
    q = w.q[:n]
    use_ref = oracle.ref is not None
    fn = oracle.ref_attention if use_ref else oracle.attention
    fn(sn, lens, w.max_len, q, k, v, threads=threads)  # warm-up
    times = []
    t_start = time.perf_counter()
    while len(times) < 5 and (time.perf_counter() - t_start) < seconds_budget:
        t0 = time.perf_counter()
        fn(sn, lens, w.max_len, q, k, v, threads=threads)
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    sample_bytes = float(tokens) * row + n * w.shape.num_heads * w.shape.head_dim * 4 * 2
    what = f"the whole step ({n} sequences, {tokens} tokens)" if full else \
        f"sequences 0-{n - 1} of {w.shape.batch} ({tokens} of {int(w.lens.sum())} tokens)"
    out = {
        "value": round(sample_bytes / med / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "cpu": cpu_model(),
        "kind": "reference" if use_ref else "port",
        "sample": f"{what} x {w.shape.num_heads} heads, fp64 attention on the stored "
                  f"{'dequantised int8' if w.kv_type == kvb.KV_I8 else 'K/V'} values, median of {len(times)} "
                  f"runs after 1 warm-up: {med * 1e3:.1f} ms",
    }
    if full:
        out["ms_per_step"] = round(med * 1e3, 2)
    else:
        out["ms_per_step_extrapolated"] = round(med * float(w.lens.sum()) / float(tokens) * 1e3, 2)
    return out


WORKLOAD_TEXT = {
    "c1": "c1: fp32 paged decode, batch 1, 32 q / 8 KV heads (GQA 4), head_dim 128, context 512, page 16",
    "c2": "c2: fp16 paged decode, batch 8, 32 q / 8 KV heads (GQA 4), head_dim 128, context 4096, page 16",
    "c3": "c3: int8 paged decode (per-(page, KV head) scales), batch 16, 32 q / 8 KV heads, head_dim 128, "
          "context 8192, page 64",
    "c4": "c4: fp16 paged decode, batch 4, 64 q / 8 KV heads (GQA 8), head_dim 128, context 32768, page 128",
    "c5f16": "c5: fp16 ragged batch of 72 (64 lengths ~U[1,16384] + 0,1,63,64,65,2047,2048,2049), 32 q / 8 KV "
             "heads, head_dim 128, page 64",
    "c5i8": "c5: int8 ragged batch of 72 (64 lengths ~U[1,16384] + 0,1,63,64,65,2047,2048,2049), 32 q / 8 KV "
            "heads, head_dim 128, page 64",
}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="c4", choices=sorted(WORKLOAD_TEXT))
    ap.add_argument("--part", type=int, default=None,
                    help="partition tokens (default: the config's, else the MI355X policy; 0 = auto_part_tokens)")
    ap.add_argument("--pair", choices=["auto", "off", "always"], default="auto",
                    help="two partitions per decode workgroup (kvb_set_pair_mode); the same bits either way")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extras", action="store_true",
                    help="skip the two-kernel, warm, probe and (c4) int8 measurements")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (each GPU would run the same kernel "
              "on its own shard of sequences / KV heads); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    loadavg = os.getloadavg()  # before this run adds its own load
    kvb = graft.load_package()
    if not kvb.gpu_available():
        print("bench.py: no GPU", file=sys.stderr)
        sys.exit(1)
    env = build_info.env_record(kvb, loadavg)
    log(f"device: {kvb.device_name()}")
    kvb.set_pair_mode(args.pair)
    # The probe runs first, and nothing is freed until every GPU measurement is done: on these boxes
    # kernels run measurably slower for a while after a large hipFree (the same 4 GiB buffer read
    # 7.05 TB/s before and 6.7 TB/s after other buffers were freed).
    keep = []
    if not args.no_extras:
        probe = kvb.Buffer(4 << 30)
        probe.fill(1)
        kvb.run_read_bandwidth(probe)
        pt = [kvb.run_read_bandwidth(probe) for _ in range(5)]
        probe_gbps = round((4 << 30) / (statistics.median(pt) * 1e-3) / 1e9, 1)
        keep.append(probe)
    t_setup = time.perf_counter()
    w, c, cfg = kvb.make_config(args.config, threads=cpu_threads())
    part = kvb.config_part(cfg, w) if args.part is None else args.part
    dev = kvb.DeviceCase(w, c)
    devi = None
    if not args.no_extras and args.config == "c4":
        # c4's shape with an int8 cache (per-(page, KV head) scales), for the int8 / fp16 speed ratio.
        # Its pools are allocated here, with the fp16 ones, as a server allocates its KV pools at start:
        # allocated after the other measurements they have landed where int8 ran up to 9% slower.
        wi = kvb.Workload(w.shape, "i8", list(w.lens), seed=32768, q_amp=1.0, dist="normal", threads=cpu_threads())
        ci = kvb.PagedCache(wi, 128, 32768 * 131 + 128, pool_factor=1.25, poison=False)
        devi = kvb.DeviceCase(wi, ci)
    nparts = dev.max_parts(part)
    part_res = kvb.auto_part_tokens(w.shape.batch, w.shape.num_kv_heads, w.max_len) if part == 0 else part
    log(f"{args.config} ready in {time.perf_counter() - t_setup:.1f}s: {int(w.lens.sum())} tokens, "
        f"pool {c.num_blocks} blocks, partition {part_res} ({nparts} per sequence)")

    times, wall = timed_steps(kvb, dev, part, args.steps, args.warmup)
    med = statistics.median(times)
    kernel_avg = statistics.mean(times)  # the step is one launch of the fused paged_decode kernel
    bytes_step = w.min_bytes()
    value = bytes_step / (med * 1e-3) / 1e9
    achieved = bytes_step / (kernel_avg * 1e-3) / 1e9
    log(f"{args.config}: step median {med * 1e3:.1f} us (mean {kernel_avg * 1e3:.1f} us), {value:.0f} GB/s; "
        f"wall {wall:.3f}s for {args.steps} steps")

    kernel = dev.kernel_name(part)
    rec, why = traffic_record(args.config, kernel)
    traffic = rec["bytes_per_launch"] if rec else None
    tcc_hit = rec["tcc_hit_rate"] if rec else None
    if why:
        log(f"roofline.traffic: null ({why})")

    extras = {}
    if w.kv_type == kvb.KV_I8:
        extras["scale_bytes"] = c.scale_bytes(w)  # read too, reported apart from value (src/workload.hpp:68-74)
    if not args.no_extras:
        ud, ur = split_steps(kvb, dev, part, 10)
        extras["unfused_decode_us"] = round(ud * 1e3, 2)
        extras["unfused_reduce_us"] = round(ur * 1e3, 2)
        if c.page_size % 16 == 0 and part_res % 16 == 0:
            extras["loads_only_us"] = round(loads_only(kvb, dev, part) * 1e3, 2)
        extras["warm_chain_us"] = round(warm_chain(kvb, dev, part) * 1e3, 2)
        extras["graph_chain_us"] = round(graph_chain(kvb, dev, part) * 1e3, 2)
        extras["warm_gbps"] = round(bytes_step / (extras["warm_chain_us"] * 1e-6) / 1e9, 1)
        extras["warm_step_us"] = round(warm_steps(kvb, dev, part) * 1e3, 2)
        extras["empty_step_us"] = round(empty_steps(kvb, w, part) * 1e3, 2)
    keep.append(dev)
    if devi is not None:
        parti = kvb.mi355x_part_tokens(w.shape, wi.max_len,
                                       min_groups=kvb.mi355x_min_groups(kvb.KV_I8, w.shape.head_dim)) \
            if args.part is None else args.part
        extras["int8_part"] = parti
        ti, _ = timed_steps(kvb, devi, parti, args.steps, args.warmup)
        medi = statistics.median(ti)
        extras["int8_us_per_step"] = round(medi * 1e3, 2)
        extras["int8_gbps"] = round(wi.min_bytes() / (medi * 1e-3) / 1e9, 1)
        extras["int8_speedup_vs_fp16"] = round(med / medi, 3)
        if not args.no_extras:
            extras["int8_loads_only_us"] = round(loads_only(kvb, devi, parti) * 1e3, 2)
        keep.append(devi)
        log(f"int8 c4-shape: {medi * 1e3:.1f} us ({extras['int8_speedup_vs_fp16']}x fp16)")
    if not args.no_extras:
        extras["probe_gbps"] = probe_gbps  # the streaming-read ceiling, measured first
        extras["pct_of_probe"] = round(100 * value / probe_gbps, 1)
    for x in keep:
        x.free()

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(kvb, graft.load_oracle(), w, c)
        log(f"cpu baseline: {cpu['sample']}, {cpu['value']} GB/s on {cpu['cores']} threads ({cpu['kind']})")
        if devi is not None:  # the int8 cache too: dequantised (outside the timing), then the fp64 path
            extras["int8_cpu_baseline"] = cpu_baseline(kvb, graft.load_oracle(), wi, ci)

    storage = {kvb.KV_F32: "f32", kvb.KV_F16: "f16", kvb.KV_I8: "i8"}[w.kv_type]
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
        "dtype": "f32",
        "dtype_detail": "fp32 arithmetic and accumulation; q and p enter the fp16 MFMAs as high/low fp16 pairs "
                        "(about 22 bits); int8 scores are exact integer MFMAs of the stored bytes with q split "
                        "into three signed byte digits",
        "data": "synthetic: q, K, V ~ N(0,1) from seeds, K/V stored as %s; shuffled block table over a %gx pool"
                % ({"f32": "fp32", "f16": "fp16 (RNE)", "i8": "int8 per-(page, KV head) scales"}[storage], cfg["pool"]),
        "config": {"workload": WORKLOAD_TEXT[args.config] + ", partition %d, cold (1 GiB read flush per step)" % part_res,
                   "kv_storage": storage, "bytes_per_step": bytes_step, "timed_wall_s": round(wall, 4)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": traffic,
                     "tcc_hit_rate": tcc_hit,
                     "traffic_source": f"profiles/traffic_{args.config}.json" if rec else why,
                     "kernel": kernel, "kernel_avg_us": round(kernel_avg * 1e3, 2),
                     "bytes_per_launch": bytes_step},
        "cpu_baseline": cpu,
        "env": env,
    }
    line.update(extras)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
