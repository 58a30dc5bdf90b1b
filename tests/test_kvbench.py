"""kvbench, this build's benchmark CLI (kv-cache-bench_amd/bench/kvbench.cpp), and the reference's own
bench/bench.cpp compiled unmodified against the drop-in headers (oracle/_ref/kvbench).

kvbench keeps the reference's flags and CSV columns (bench/bench.cpp:48-84, :124, :156, :187, :212),
with this build's columns after them, so the reference's consumer (scripts/tables.py) reads it."""
import os
import subprocess

import numpy as np
import pytest

from conftest import ROOT, progress

BUILD = os.environ.get("KVB_BUILD_DIR") or os.path.join(ROOT, "kv-cache-bench_amd", "build")
KVBENCH = os.path.join(BUILD, "kvbench")
REF_BIN = os.environ.get("KVB_REF_BIN") or os.path.join(ROOT, "oracle", "_ref")
KVREF = os.path.join(REF_BIN, "libkvref.so")  # the reference's src/reference.cpp (attention_reference)

# The reference's CSV headers, by mode (bench/bench.cpp:124, 156, 187, 212), and the columns this
# build appends to each.
REFERENCE_HEADERS = {
    "bw": ("impl,bytes,reps,median_us,min_us,max_us,gbps", ""),
    "chain": ("impl,layout,dtype,batch,seq_len,chain,reps,median_us,min_us,max_us,gbps,max_err,err_vs", "gpu_us"),
    "accuracy": ("data,dtype,seq_len,page,max_abs_err,rms_err", ""),
    "sweep": ("impl,dtype,batch,seq_len,page,part,reps,median_us,min_us,max_us,gbps,max_diff_vs_naive,kv_bytes",
              "decode_us,reduce_us"),
}


def csv_rows(text):
    lines = [ln for ln in text.splitlines() if ln and not ln.startswith("#")]
    head = lines[0].split(",")
    return head, [dict(zip(head, ln.split(","))) for ln in lines[1:]]


def test_kvbench_schema_matches_the_reference():
    """Every mode's header is the reference's, then this build's columns (needs no GPU)."""
    out = subprocess.run([KVBENCH, "--schema"], capture_output=True, text=True, timeout=60, check=True).stdout
    got = dict(line.split(":", 1) for line in out.splitlines())
    assert set(got) == set(REFERENCE_HEADERS)
    for mode, (ref, own) in REFERENCE_HEADERS.items():
        assert got[mode] == ref + ("," + own if own else ""), mode


def test_kvbench_refuses_unknown_flags():
    r = subprocess.run([KVBENCH, "--lens=512", "--no-such-flag"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 2 and "unknown argument --no-such-flag" in r.stderr


@pytest.mark.gpu
def test_kvbench_accuracy(gpu):
    """--accuracy (the reference's bench/bench.cpp:186-210): one CSV row per (data, type, page); the
    fp32 cache's error is the kernel's own (<= 2e-5 against fp64 on the same values), fp16 and int8
    add their storage error."""
    out = subprocess.run([KVBENCH, "--accuracy", "--batch=2", "--lens=300,1000", "--pages=16,64"],
                         capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stderr
    env = [ln for ln in out.stdout.splitlines() if ln.startswith("# env ")]
    assert len(env) == 1 and "hip_runtime=" in env[0] and " hip_runtime=0 " not in env[0], env
    head, body = csv_rows(out.stdout)
    assert ",".join(head) == REFERENCE_HEADERS["accuracy"][0]
    assert len(body) == 2 * 2 * 3 * 2  # data x lens x types x pages
    for r in body:
        mx, rms = float(r["max_abs_err"]), float(r["rms_err"])
        assert 0 <= rms <= mx
        assert mx <= {"f32": 2e-5, "f16": 2e-3, "i8": 5e-2}[r["dtype"]], r
    progress("[kvbench] accuracy: " + "; ".join(f"{r['data']} {r['dtype']} L{r['seq_len']} p{r['page']}: "
                                                f"{r['max_abs_err']}" for r in body[:6]))


@pytest.mark.gpu
def test_kvbench_dump(gpu, oracle, tmp_path):
    """--dump: raw fp32 inputs and fp64 outputs; the f32 output recomputed by the oracle from the
    dumped inputs must agree (both are fp64 attention on the same values)."""
    B, H, Hkv, D, L = 2, 32, 8, 128, 200
    out = subprocess.run([KVBENCH, f"--dump={tmp_path}", f"--batch={B}", f"--lens={L}"],
                         capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stderr
    q = np.fromfile(tmp_path / f"L{L}_q.f32", np.float32).reshape(B, H, D)
    k = np.fromfile(tmp_path / f"L{L}_k.f32", np.float32).reshape(B, Hkv, L, D)
    v = np.fromfile(tmp_path / f"L{L}_v.f32", np.float32).reshape(B, Hkv, L, D)
    ref32 = np.fromfile(tmp_path / f"L{L}_ref_f32.f32", np.float32).reshape(B, H, D)
    ref16 = np.fromfile(tmp_path / f"L{L}_ref_f16.f32", np.float32).reshape(B, H, D)
    want = oracle.attention(gpu.Shape(B, H, Hkv, D), np.array([L] * B, np.int32), L, q, k, v)
    assert oracle.max_abs_diff(ref32, want) <= 1e-6
    # the f16 dump is of the fp16-rounded values: close to, not equal to, the fp32 one
    assert 0 < oracle.max_abs_diff(ref16, ref32) < 1e-2


@pytest.mark.gpu
def test_kvbench_sweep_loads_and_cpu_rows(gpu):
    """The default sweep: gpu_naive, cpu_ref_fp64 (the reference's own attention_reference, loaded
    from its kvref library with --cpu-ref) and gpu_paged rows per (type, length, page, partition),
    the paged and CPU outputs against the naive one, --loads rows timed below the full step, and
    the two-kernel split in the appended columns; --bw one read_bw row."""
    if not os.path.exists(KVREF):
        pytest.skip(f"{KVREF} is not built")
    out = subprocess.run([KVBENCH, "--batch=2", "--lens=2048", "--pages=16,64", "--parts=256", "--reps=3",
                          "--warmup=1", "--cpu-reps=1", "--loads", "--types=f32,f16,i8", f"--cpu-ref={KVREF}"],
                         capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stderr
    head, rows = csv_rows(out.stdout)
    ref, own = REFERENCE_HEADERS["sweep"]
    assert ",".join(head) == ref + "," + own
    by = {}
    for r in rows:
        by.setdefault(r["impl"], []).append(r)
    assert len(by["gpu_naive"]) == 2  # f32 and f16 (the naive kernels take no int8)
    assert len(by["cpu_ref_fp64"]) == 2
    assert len(by["gpu_paged"]) == 3 * 2 and len(by["gpu_paged_loads"]) == 3 * 2
    for r in by["cpu_ref_fp64"]:  # fp64 on the stored values against the naive kernels
        assert float(r["max_diff_vs_naive"]) <= 2e-5 and float(r["median_us"]) > 0, r
    for r in by["gpu_paged"]:
        if r["dtype"] != "i8":
            assert float(r["max_diff_vs_naive"]) <= 2e-5, r
        assert float(r["decode_us"]) > 0 and float(r["reduce_us"]) > 0, r
    step = {(r["dtype"], r["page"]): float(r["median_us"]) for r in by["gpu_paged"]}
    for r in by["gpu_paged_loads"]:
        assert 0 < float(r["median_us"]) <= 1.5 * step[(r["dtype"], r["page"])], r
    bw = subprocess.run([KVBENCH, "--bw", "--bw-bytes=268435456", "--reps=3"], capture_output=True, text=True,
                        timeout=300)
    assert bw.returncode == 0, bw.stderr
    bhead, b = csv_rows(bw.stdout)
    assert ",".join(bhead) == REFERENCE_HEADERS["bw"][0]
    assert len(b) == 1 and b[0]["impl"] == "read_bw" and 500 < float(b[0]["gbps"]) < 12000
    cpu = {r["dtype"]: float(r["median_us"]) for r in by["cpu_ref_fp64"]}
    progress(f"[kvbench] paged f16 page 64: {step[('f16', '64')]} us; cpu_ref_fp64 f16: {cpu['f16']:.0f} us; "
             f"read_bw 256 MiB: {b[0]['gbps']} GB/s")


@pytest.mark.gpu
def test_kvbench_chain(gpu):
    """--chain=N (bench/bench.cpp:155-185): per type, a contiguous and a paged16 row; max_err against
    fp64 on the stored values (f32, f16: within the kernel tolerance 2e-5) or on the unquantised data
    (i8: its storage error), with err_vs saying which."""
    out = subprocess.run([KVBENCH, "--chain=8", "--batch=2", "--lens=1000", "--reps=3", "--warmup=1"],
                         capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stderr
    head, rows = csv_rows(out.stdout)
    ref, own = REFERENCE_HEADERS["chain"]
    assert ",".join(head) == ref + "," + own
    assert {(r["layout"], r["dtype"]) for r in rows} == {(lay, t) for lay in ("contiguous", "paged16")
                                                          for t in ("f32", "f16", "i8")}
    for r in rows:
        assert r["impl"] == "ours" and r["chain"] == "8"
        assert r["err_vs"] == ("fp32_data" if r["dtype"] == "i8" else "stored")
        assert float(r["max_err"]) <= (5e-2 if r["dtype"] == "i8" else 2e-5), r
        assert float(r["median_us"]) > 0 and float(r["gpu_us"]) > 0


@pytest.mark.gpu
def test_kvbench_chain_graph(gpu):
    """--chain=N --graph: each paged16 chain is also captured into a HIP graph and replayed (impl
    ours-graph), with the same schema and the same error as the eager chain's row."""
    out = subprocess.run([KVBENCH, "--chain=8", "--graph", "--batch=2", "--lens=1000", "--reps=3", "--warmup=1",
                          "--types=f16,i8"], capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stderr
    head, rows = csv_rows(out.stdout)
    ref, own = REFERENCE_HEADERS["chain"]
    assert ",".join(head) == ref + "," + own
    eager = {r["dtype"]: r for r in rows if r["impl"] == "ours" and r["layout"] == "paged16"}
    graph = {r["dtype"]: r for r in rows if r["impl"] == "ours-graph"}
    assert set(graph) == set(eager) == {"f16", "i8"}
    for t, r in graph.items():
        assert r["layout"] == "paged16" and r["chain"] == "8"
        assert r["max_err"] == eager[t]["max_err"], (t, r["max_err"], eager[t]["max_err"])
        assert float(r["median_us"]) > 0 and float(r["gpu_us"]) > 0
    progress(f"[kvbench] chain of 8, f16 paged16: eager {eager['f16']['gpu_us']} us, graph {graph['f16']['gpu_us']} us "
             "per step")


@pytest.mark.gpu
def test_reference_bench_runs_on_the_drop_in(gpu):
    """The reference's own bench/bench.cpp, compiled unmodified against this build's headers
    (oracle/_ref/kvbench): its sweep runs on MI355X, with its CPU rows from its own kvref, and the
    paged kernel agrees with the naive one."""
    ref_bench = os.path.join(REF_BIN, "kvbench")
    if not os.path.exists(ref_bench):
        pytest.skip(f"{ref_bench} is not built")
    out = subprocess.run([ref_bench, "--batch=2", "--lens=1024", "--pages=16", "--reps=3", "--warmup=1",
                          "--cpu-reps=1", "--types=f16,i8"], capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stderr
    head, rows = csv_rows(out.stdout)
    assert ",".join(head) == REFERENCE_HEADERS["sweep"][0]
    impls = {(r["impl"], r["dtype"]) for r in rows}
    assert impls == {("gpu_naive", "f16"), ("cpu_ref_fp64", "f16"), ("gpu_paged", "f16"), ("gpu_paged", "i8")}
    for r in rows:
        if r["dtype"] == "f16":
            assert float(r["max_diff_vs_naive"]) <= 2e-5, r
