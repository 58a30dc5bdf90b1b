#!/bin/bash
# sweep.sh OUT: the reference's full benchmark sweep (its scripts/bench.sh:10-18) on one MI355X, with
# this build's kvbench, into OUT/{env.json,bw.csv,bench.csv,parts.csv,gqa.csv,accuracy.csv}:
#   env.json      the environment record before the run (build_info.py --env), load after appended as
#                 env_after.txt
#   bw.csv        kvbench --bw (the read-bandwidth probe, 512 MiB)
#   bench.csv     kvbench with the reference's defaults (batch 2, 32 q / 8 KV heads, head_dim 128;
#                 lengths 512..32768, pages 16..128, f32/f16/i8, the reference's partition rule), with
#                 cpu_ref_fp64 rows from the reference's own attention_reference (oracle/_ref/libkvref.so)
#   parts.csv     the split-K partition sweep at page 32 (no CPU / naive rows)
#   gqa.csv       one workgroup per KV head against one per query head (--per-head)
#   accuracy.csv  error of each storage type against fp64 on the same fp32 data (no timing)
# Needs the in-tree build (make -C kv-cache-bench_amd all, make -C oracle ref). Each step has its own
# time limit; the first failure ends the script.
set -eo pipefail
O=$(realpath -m "$1")
R=$(cd "$(dirname "$0")/../.." && pwd)
K="$R/kv-cache-bench_amd/build/kvbench"
mkdir -p "$O"
echo "[sweep] env"
timeout -k 10 120 python3 "$R/kv-cache-bench_amd/bench/build_info.py" --env > "$O/env.json"
echo "[sweep] bw"
timeout -k 10 120 "$K" --bw > "$O/bw.csv"
echo "[sweep] bench (defaults)"
timeout -k 10 600 "$K" --cpu-ref="$R/oracle/_ref/libkvref.so" > "$O/bench.csv"
echo "[sweep] parts"
timeout -k 10 300 "$K" --lens=512,2048,8192,32768 --pages=32 --parts=64,128,256,512,1024,2048 --no-cpu --no-naive \
    --types=f32,f16 > "$O/parts.csv"
echo "[sweep] gqa"
timeout -k 10 300 "$K" --lens=512,2048,8192,32768 --pages=32 --per-head --no-cpu --no-naive --types=f32,f16 > "$O/gqa.csv"
echo "[sweep] accuracy"
timeout -k 10 300 "$K" --accuracy --pages=16,128 > "$O/accuracy.csv"
echo "load after: $(cut -d' ' -f1-3 /proc/loadavg)" > "$O/env_after.txt"
echo "[sweep] done: $O"
