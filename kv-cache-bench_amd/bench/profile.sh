#!/bin/bash
# profile.sh CONFIG OUT: the measurements behind profiles/paged_decode_<CONFIG>.md, on one MI355X.
#   1. bench.py (plain run, every extra): the JSON line
#   2. rocprofv3 kernel trace of bench.py --no-extras (3 warm-up + 30 timed steps, each after a flush)
#   3. rocprofv3 --pmc FETCH_SIZE, then WRITE_SIZE (10 timed steps each), for HBM traffic per step
#   4. rocprofv3 --pmc TCC_HIT_sum TCC_MISS_sum (10 timed steps), the L2 hit rate
#   5. rocprofv3 --pmc SQ counters (10 timed steps), instruction mix per wave
#   6. the per-workgroup timeline (wg_timeline.py; needs the build-ts measurement build)
# then prof_summary.py CONFIG OUT writes OUT/summary.md (and, for c4, OUT/traffic.json).
# Needs the in-tree build (make -C kv-cache-bench_amd all timestamps). Each step has its own time
# limit; the first failure ends the script.
set -eo pipefail
C=$1
O=$(realpath -m "$2")
R=$(cd "$(dirname "$0")/../.." && pwd)
mkdir -p "$O"
cd /tmp && export TMPDIR=/tmp
B="python3 $R/bench.py --no-cpu"
echo "[profile $C] bench"
timeout -k 10 300 $B --config "$C" > "$O/bench.json" 2> "$O/bench.err"
echo "[profile $C] kernel trace"
timeout -k 10 300 rocprofv3 --kernel-trace --stats -d "$O/trace" -o run --output-format csv -- \
    python3 "$R/bench.py" --no-cpu --no-extras --config "$C" --steps 30 > "$O/trace.log" 2>&1
echo "[profile $C] FETCH_SIZE"
timeout -s KILL 180 rocprofv3 --pmc FETCH_SIZE -d "$O/fetch" -o run --output-format csv -- \
    python3 "$R/bench.py" --no-cpu --no-extras --config "$C" --steps 10 > "$O/fetch.log" 2>&1
echo "[profile $C] WRITE_SIZE"
timeout -s KILL 180 rocprofv3 --pmc WRITE_SIZE -d "$O/write" -o run --output-format csv -- \
    python3 "$R/bench.py" --no-cpu --no-extras --config "$C" --steps 10 > "$O/write.log" 2>&1
echo "[profile $C] TCC hit rate"
timeout -s KILL 180 rocprofv3 --pmc TCC_HIT_sum TCC_MISS_sum -d "$O/tcc" -o run --output-format csv -- \
    python3 "$R/bench.py" --no-cpu --no-extras --config "$C" --steps 10 > "$O/tcc.log" 2>&1
echo "[profile $C] SQ counters"
timeout -s KILL 180 rocprofv3 --pmc SQ_WAVES SQ_INSTS_VALU SQ_INSTS_LDS SQ_INSTS_SALU SQ_INSTS_VMEM_RD \
    SQ_WAVE_CYCLES SQ_BUSY_CYCLES SQ_WAIT_INST_ANY GRBM_GUI_ACTIVE -d "$O/sq" -o run --output-format csv -- \
    python3 "$R/bench.py" --no-cpu --no-extras --config "$C" --steps 10 > "$O/sq.log" 2>&1
echo "[profile $C] workgroup timeline"
timeout -k 10 300 python3 "$R/kv-cache-bench_amd/bench/wg_timeline.py" "$C" > "$O/timeline.md" 2> "$O/timeline.err"
python3 "$R/kv-cache-bench_amd/bench/prof_summary.py" "$C" "$O" > "$O/summary.md"
echo "[profile $C] done: $O/summary.md"
