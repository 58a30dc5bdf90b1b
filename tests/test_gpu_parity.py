"""GPU parity: the HIP kernels through the C ABI against the pinned CPU oracle and the golden
fixtures. Tolerance (the reference's tests/gpu_tests.cpp:13-17, scaled for |v| > 1): kernel vs
oracle on the same stored values <= 2e-5 * max(1, max|v|); fp32 storage also <= 1e-4 relative to
max|out|. Gathers through the block table and partition indexing are checked bit for bit."""
import glob
import os

import numpy as np
import pytest

from conftest import ROOT, progress

pytestmark = pytest.mark.gpu
THREADS = 16
GOLDEN = sorted(glob.glob(os.path.join(ROOT, "tests", "golden", "*.npz")))


def expected(kvb, oracle, w, c):
    """Oracle output on the values the kernel reads, and the tolerance that goes with it."""
    if w.kv_type == kvb.KV_I8:
        kd, vd = c.dequantized(w)
        want = oracle.attention(w.shape, w.lens, w.max_len, w.q, kd, vd, threads=THREADS)
        vmax = float(np.abs(vd).max()) if vd.size else 0.0
    else:
        want = oracle.attention(w.shape, w.lens, w.max_len, w.q, w.k, w.v, threads=THREADS)
        live = [w.v[b, :, :L] for b, L in enumerate(w.lens)]
        vmax = max((float(np.abs(x.astype(np.float32)).max()) for x in live if x.size), default=0.0)
    return want, 2e-5 * max(1.0, vmax)


def run(kvb, w, c, part=0, share_kv=True, workspace=None):
    dev = kvb.DeviceCase(w, c)
    dev.out.fill(0xFF)  # NaN: every output element must be written
    dev.run(part, share_kv, workspace)
    got = dev.output()
    dev.free()
    return got


@pytest.mark.parametrize("name", ["c1", "c2", "c3", "c4", "c5f16", "c5i8"])
def test_baseline_config_full_size(gpu, oracle, name):
    kvb = gpu
    w, c, cfg = kvb.make_config(name, poison=True, threads=THREADS)
    progress(f"[parity] {name}: B={w.shape.batch} max_len={w.max_len} tokens={int(w.lens.sum())} pool={c.num_blocks}")
    part = kvb.config_part(cfg, w)
    got = run(kvb, w, c, part)
    want, tol = expected(kvb, oracle, w, c)
    err = oracle.max_abs_diff(got, want)
    progress(f"[parity] {name}: max err {err:.3g} (tol {tol:.3g})")
    assert err <= tol
    if w.kv_type == kvb.KV_F32:
        assert err <= 1e-4 * float(np.abs(want).max())
    for b in np.flatnonzero(w.lens == 0):
        assert not got[b].any()


def test_storage_bounds_c2_f16(gpu, oracle):
    kvb = gpu
    shape = kvb.Shape(8, 32, 8, 128)
    w = kvb.Workload(shape, "f16", [4096] * 8, seed=4096, q_amp=1.0, keep_f32=True, dist="normal", threads=THREADS)
    c = kvb.PagedCache(w, 16, 4096 * 131 + 16, pool_factor=1.5, poison=True)
    got = run(kvb, w, c, 512)
    exact = oracle.attention(w.shape, w.lens, w.max_len, w.q, w.k32, w.v32, threads=THREADS)
    bound = oracle.fp16_storage_bound(w.shape, w.lens, w.max_len, w.q, w.k32, w.v32)
    assert oracle.max_abs_diff(got, exact) <= bound


def test_storage_bounds_c3_i8(gpu, oracle):
    kvb = gpu
    shape = kvb.Shape(16, 32, 8, 128)
    w = kvb.Workload(shape, "i8", [8192] * 16, seed=8192, q_amp=1.0, dist="normal", threads=THREADS)
    c = kvb.PagedCache(w, 64, 8192 * 131 + 64, poison=True)
    got = run(kvb, w, c, 0)
    exact = oracle.attention(w.shape, w.lens, w.max_len, w.q, w.k, w.v, threads=THREADS)
    bound = oracle.i8_storage_bound(w.shape, w.lens, 64, c.table, w.q, c.k_scale, c.v_scale)
    assert oracle.max_abs_diff(got, exact) <= bound


@pytest.mark.parametrize("path", GOLDEN, ids=[os.path.basename(p) for p in GOLDEN])
def test_golden(gpu, oracle, path):
    kvb = gpu
    g = np.load(path, allow_pickle=False)
    kind = str(g["kind"])
    w = kvb.Workload.from_arrays(kind, g["lens"], g["q"], g["k"], g["v"])
    c = kvb.PagedCache(w, int(g["page"]), table=g["table"], num_blocks=int(g["num_blocks"]), poison=True)
    if kind == "i8":  # the host quantiser reproduces the reference's bytes and scales (unpoisoned pool)
        plain = kvb.PagedCache(w, int(g["page"]), table=g["table"], num_blocks=int(g["num_blocks"]), poison=False)
        assert np.array_equal(plain.k, g["k_paged"]) and np.array_equal(plain.k_scale, g["k_scale"])
        assert np.array_equal(plain.v, g["v_paged"]) and np.array_equal(plain.v_scale, g["v_scale"])
        vmax = float(np.abs(g["v_deq"]).max())
    else:
        vmax = float(np.abs(g["v"].astype(np.float32)).max())
    for part in (0, 16, 7):
        got = run(kvb, w, c, part)
        assert oracle.max_abs_diff(got, g["out"]) <= 2e-5 * max(1.0, vmax), (part,)


@pytest.mark.parametrize("kv", ["f32", "f16", "i8"])
@pytest.mark.parametrize("page,part", [(16, 0), (16, 48), (64, 128), (1, 16), (3, 7), (24, 100)])
def test_dominant_key_gather_is_exact(gpu, kv, page, part):
    """q = 1000 e_0 and a one-hot key make the softmax exactly one-hot: the output must be the hot
    token's V row bit for bit, through the shuffled block table and every partition merge."""
    kvb = gpu
    lens = [300, 77, 16]
    w = kvb.Workload(kvb.Shape(3, 16, 2, 128), kv, lens, seed=11)
    w.q[:] = 0
    w.q[:, :, 0] = 1000.0
    hot = [(37 * b + 5) % L for b, L in enumerate(lens)]
    w.k[:] = 0
    for b, t in enumerate(hot):
        w.k[b, :, t, 0] = 1.0
    if kv == "i8":  # V on the grid k / 128 with a 127/128 in every row: scale 2^-7, every product exact
        w.v[:] = np.round(w.v * 127) / 128
        w.v[:, :, :, 0] = 127 / 128
    c = kvb.PagedCache(w, page, 99, pool_factor=1.5, poison=True)
    got = run(kvb, w, c, part)
    vals = c.dequantized(w)[1] if kv == "i8" else w.v.astype(np.float32)
    for b, t in enumerate(hot):
        for h in range(16):
            assert np.array_equal(got[b, h], vals[b, h // 8, t]), (b, h)


def test_workspace_partition_indexing(gpu, oracle):
    """Every (sequence, head, partition) slot of a caller-owned workspace: written with the oracle's
    (m, l, o) iff the partition holds tokens, untouched (NaN) otherwise."""
    kvb = gpu
    lens, part = [200, 65, 0, 64], 64
    w = kvb.Workload(kvb.Shape(4, 8, 2, 128), "f32", lens, seed=21)
    c = kvb.PagedCache(w, 16, 5, pool_factor=2.0, poison=True)
    dev = kvb.DeviceCase(w, c)
    max_parts = dev.max_parts(part)
    ws = kvb.Buffer(dev.workspace_bytes(part))
    ws.fill(0xFF)
    dev.run(part, workspace=ws)
    B, H, D = 4, 8, 128
    raw = ws.download(np.float32, ws.nbytes // 4)
    part_out = raw[: B * H * max_parts * D].reshape(B, H, max_parts, D)
    part_ml = raw[B * H * max_parts * D: B * H * max_parts * (D + 2)].reshape(B, H, max_parts, 2)
    assert max_parts == 4
    for b in range(B):
        for h in range(H):
            for p in range(max_parts):
                st = oracle.partition_state(w.shape, w.lens, w.max_len, w.q, w.k, w.v, part, b, h, p)
                if st is None:
                    assert np.isnan(part_out[b, h, p]).all() and np.isnan(part_ml[b, h, p]).all(), (b, h, p)
                    continue
                m, l, o = st
                assert abs(part_ml[b, h, p, 0] - m) <= 1e-5 * max(1.0, abs(m)), (b, h, p)
                assert abs(part_ml[b, h, p, 1] - l) <= 1e-5 * l, (b, h, p)
                assert np.abs(part_out[b, h, p] - o).max() <= 2e-5, (b, h, p)
    got = dev.output()
    want = oracle.attention(w.shape, w.lens, w.max_len, w.q, w.k, w.v)
    assert oracle.max_abs_diff(got, want) <= 2e-5
    dev.free()
    ws.free()


@pytest.mark.parametrize("kv", ["f32", "f16", "i8"])
def test_ragged_any_page_and_partition(gpu, oracle, kv):
    kvb = gpu
    lens = [0, 1, 15, 16, 17, 63, 64, 65, 129, 300, 2, 0]
    w = kvb.Workload(kvb.Shape(1, 8, 2, 64), kv, lens, seed=31, varied=(kv == "i8"))
    for page, part in [(1, 0), (3, 5), (8, 100), (16, 16), (32, 0), (48, 96), (64, 1)]:
        c = kvb.PagedCache(w, page, page * 7, pool_factor=3.0, poison=True)
        want, tol = expected(kvb, oracle, w, c)
        for share in (True, False):
            got = run(kvb, w, c, part, share)
            assert oracle.max_abs_diff(got, want) <= tol, (page, part, share)


@pytest.mark.parametrize("shape", [(2, 8, 8, 128), (2, 12, 4, 64), (2, 32, 2, 128), (2, 6, 2, 64)])
def test_gqa_groups(gpu, oracle, shape):
    """Groups 1, 3, 16 and 3: query heads per workgroup chosen from {8,4,2,1} dividing the group."""
    kvb = gpu
    w = kvb.Workload(kvb.Shape(*shape), "f16", [333, 1000], seed=41, dist="normal", q_amp=1.0)
    c = kvb.PagedCache(w, 16, 3, pool_factor=1.25, poison=True)
    want, tol = expected(kvb, oracle, w, c)
    assert oracle.max_abs_diff(run(kvb, w, c, 256), want) <= tol


def test_huge_and_tiny_queries(gpu, oracle):
    """q far from 1 in magnitude: the fp16 high/low split scales q by a power of two first."""
    kvb = gpu
    w = kvb.Workload(kvb.Shape(2, 8, 2, 128), "f16", [500, 20], seed=51)
    c = kvb.PagedCache(w, 16, 3, poison=True)
    for amp in (8000.0, 1e-3, 3e-6):
        w.q[:] = np.random.Generator(np.random.PCG64(7)).uniform(-amp, amp, w.q.shape).astype(np.float32)
        want, tol = expected(kvb, oracle, w, c)
        assert oracle.max_abs_diff(run(kvb, w, c, 64), want) <= tol, amp


def test_naive_matches_oracle(gpu, oracle):
    kvb = gpu
    for kv in ("f32", "f16"):
        w = kvb.Workload(kvb.Shape(3, 8, 2, 128), kv, [257, 1, 0], seed=61)
        bufs = [kvb.Buffer.from_array(x) for x in (w.q, w.k, w.v, w.lens)]
        out = kvb.Buffer(w.out_floats() * 4)
        kvb.run_naive(w, out, *bufs)
        got = out.download(np.float32, w.q.shape)
        want = oracle.attention(w.shape, w.lens, w.max_len, w.q, w.k, w.v)
        assert oracle.max_abs_diff(got, want) <= 2e-5


@pytest.mark.parametrize("kv", ["f32", "f16"])
@pytest.mark.parametrize("shape", [(3, 8, 2, 128), (2, 32, 8, 64), (1, 4, 4, 128)])
def test_attention_fp64_matches_oracle(gpu, oracle, kv, shape):
    """The GPU fp64 reference (kvbench's accuracy reference) and the oracle are both fp64
    two-pass attention on the same stored values: they agree to fp32 rounding."""
    kvb = gpu
    s = kvb.Shape(*shape)
    lens = [0, 1, 300, 77][:s.batch] if s.batch > 1 else [513]
    w = kvb.Workload(s, kv, lens, seed=71, q_amp=3.0)
    bufs = [kvb.Buffer.from_array(x) for x in (w.q, w.k, w.v, w.lens)]
    out = kvb.Buffer(w.out_floats() * 4)
    out.fill(0xFF)
    kvb.run_attention_fp64(w, out, *bufs)
    got = out.download(np.float32, w.q.shape)
    want = oracle.attention(w.shape, w.lens, w.max_len, w.q, w.k, w.v)
    assert oracle.max_abs_diff(got, want) <= 1e-6
    for b in np.flatnonzero(w.lens == 0):
        assert not got[b].any()
    for x in bufs + [out]:
        x.free()


def test_steps_pipelined_and_deterministic(gpu):
    kvb = gpu
    w = kvb.Workload(kvb.Shape(2, 32, 8, 128), "f16", [4096, 1000], seed=71)
    c = kvb.PagedCache(w, 16, 3, pool_factor=1.5)
    dev = kvb.DeviceCase(w, c)
    dev.run(512)
    first = dev.output()
    dev.run(512, steps=4)
    assert np.array_equal(dev.output(), first)
    kvb.begin_pipelined()
    for _ in range(5):
        kvb.flush_gpu_caches()
        assert dev.run(512) == 0.0
    times = kvb.end_pipelined()
    assert len(times) == 5 and all(t > 0 for t in times)
    d, r = dev.run_split(512)
    assert d > 0 and r > 0
    assert np.array_equal(dev.output(), first)
    dev.free()


def test_fused_merge_reads_fresh_partitions(gpu):
    """The fused merge reads partition results that other workgroups (other XCDs) wrote in the same
    launch. Two cases alternate through the library's one workspace and counter array, so a merge
    that saw a stale line would pick up the other case's partitions: every fused output must equal
    the two-kernel (paged_decode, paged_reduce) output bit for bit, on every call."""
    kvb = gpu
    cases = []
    for seed, lens in ((81, [8192, 5000, 3, 8192]), (82, [8192, 7777, 4096, 1])):
        w = kvb.Workload(kvb.Shape(4, 64, 8, 128), "f16", lens, seed=seed)
        c = kvb.PagedCache(w, 16, seed, pool_factor=1.25)
        dev = kvb.DeviceCase(w, c)
        dev.run_split(256)
        cases.append((dev, dev.output()))
    assert not np.array_equal(cases[0][1], cases[1][1])
    for it in range(6):
        for dev, want in cases:
            dev.out.fill(0xFF)
            dev.run(256)
            assert np.array_equal(dev.output(), want), f"call {it}"
    for dev, _ in cases:
        dev.free()


@pytest.mark.parametrize("kv,part", [("f16", 16), ("f16", 32), ("f16", 64), ("f32", 16), ("i8", 16), ("i8", 32)])
def test_many_partitions(gpu, oracle, kv, part):
    """Partition counts at and past what the fused merge stages in LDS: at head_dim 64 and 8 heads
    per group, f16 part 64 (64 partitions) and i8 part 32 (128) fill it exactly; the others exceed
    it and the runtime merges with paged_reduce as a second kernel."""
    kvb = gpu
    w = kvb.Workload(kvb.Shape(2, 16, 2, 64), kv, [4096, 2049], seed=91)
    c = kvb.PagedCache(w, 16, 91, pool_factor=1.25)
    want, tol = expected(kvb, oracle, w, c)
    dev = kvb.DeviceCase(w, c)
    dev.out.fill(0xFF)
    dev.run(part)
    got = dev.output()
    dev.run_split(part)
    assert np.array_equal(got, dev.output())
    dev.free()
    assert oracle.max_abs_diff(got, want) <= tol


def test_read_bandwidth_probe(gpu):
    kvb = gpu
    buf = kvb.Buffer(1 << 30)
    buf.fill(1)
    ms = kvb.run_read_bandwidth(buf)
    gbps = (1 << 30) / (ms * 1e-3) / 1e9
    progress(f"[parity] read probe 1 GiB: {gbps:.0f} GB/s")
    assert 500 < gbps < 12000
    buf.free()
