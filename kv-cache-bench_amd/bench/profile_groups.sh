#!/bin/bash
# profile_groups.sh OUT: the measurements behind profiles/paged_decode_groups.md, on one MI355X: the
# decode step at c4's size (batch 4, 8 KV heads, head_dim 128, 32768 tokens, page 128, partition
# 4096, cold) with 8, 16, 32 and 64 query heads per KV head, fp16 and int8, from kvbench:
#   1. rocprofv3 kernel trace (3 warm-up + 30 timed steps, each after a flush)
#   2. rocprofv3 --pmc SQ counters (10 timed steps), instruction mix per wave
# then prof_groups.py OUT writes OUT/summary.md. Needs the in-tree build (make -C kv-cache-bench_amd
# all). Each step has its own time limit; the first failure ends the script.
set -eo pipefail
O=$(realpath -m "$1")
R=$(cd "$(dirname "$0")/../.." && pwd)
K="$R/kv-cache-bench_amd/build/kvbench"
mkdir -p "$O"
cd /tmp && export TMPDIR=/tmp
for t in f16 i8; do
  for G in 8 16 32 64; do
    H=$((8 * G))
    A="--batch=4 --heads=$H --kv-heads=8 --dim=128 --lens=32768 --pages=128 --parts=4096 --types=$t --no-cpu --no-naive"
    mkdir -p "$O/${t}_g$G"
    echo "[profile groups] $t group $G: kernel trace"
    timeout -k 10 300 rocprofv3 --kernel-trace --stats -d "$O/${t}_g$G/trace" -o run --output-format csv -- \
        "$K" $A --reps=30 --warmup=3 > "$O/${t}_g$G/kvbench.csv" 2> "$O/${t}_g$G/trace.log"
    echo "[profile groups] $t group $G: SQ counters"
    timeout -s KILL 180 rocprofv3 --pmc SQ_WAVES SQ_INSTS_VALU SQ_INSTS_LDS SQ_INSTS_SALU SQ_INSTS_VMEM_RD \
        SQ_WAVE_CYCLES SQ_BUSY_CYCLES SQ_WAIT_INST_ANY GRBM_GUI_ACTIVE -d "$O/${t}_g$G/sq" -o run --output-format csv -- \
        "$K" $A --reps=10 --warmup=1 > "$O/${t}_g$G/sq.csv" 2> "$O/${t}_g$G/sq.log"
  done
done
python3 "$R/kv-cache-bench_amd/bench/prof_groups.py" "$O" > "$O/summary.md"
echo "[profile groups] done: $O/summary.md"
