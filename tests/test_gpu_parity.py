"""GPU parity: the HIP kernels through the C ABI against the pinned CPU oracle and the golden
fixtures. The checks themselves live in parity_battery.py, which the oracle's CPU model of the
kernel runs too (test_split_model.py); the tolerances are stated there. This file adds the checks
only a GPU has: full-size configurations, the fused merge against the two-kernel form, pipelined
timing, the naive and fp64 kernels, and the bandwidth probe."""
import numpy as np
import pytest

import parity_battery as pb
from conftest import progress

pytestmark = pytest.mark.gpu
THREADS = pb.THREADS


def run(kvb, w, c, part=0, share_kv=True, workspace=None):
    dev = kvb.DeviceCase(w, c)
    dev.out.fill(0xFF)  # NaN: every output element must be written
    dev.run(part, share_kv, workspace)
    got = dev.output()
    dev.free()
    return got


def runner(kvb):
    return lambda w, c, part, share_kv: run(kvb, w, c, part, share_kv)


def run_ws(kvb, w, c, part):
    """The decode with a caller-owned workspace, NaN before the run: (out, part_out, part_ml)."""
    dev = kvb.DeviceCase(w, c)
    max_parts = dev.max_parts(part)
    ws = kvb.Buffer(dev.workspace_bytes(part))
    ws.fill(0xFF)
    dev.out.fill(0xFF)
    dev.run(part, workspace=ws)
    B, H, D = w.shape.batch, w.shape.num_heads, w.shape.head_dim
    raw = ws.download(np.float32, ws.nbytes // 4)
    part_out = raw[: B * H * max_parts * D].reshape(B, H, max_parts, D)
    part_ml = raw[B * H * max_parts * D: B * H * max_parts * (D + 2)].reshape(B, H, max_parts, 2)
    got = dev.output()
    dev.free()
    ws.free()
    return got, part_out, part_ml


@pytest.mark.parametrize("name", ["c1", "c2", "c3", "c4", "c5f16", "c5i8"])
def test_baseline_config_full_size(gpu, oracle, name):
    kvb = gpu
    w, c, cfg = kvb.make_config(name, poison=True, threads=THREADS)
    progress(f"[parity] {name}: B={w.shape.batch} max_len={w.max_len} tokens={int(w.lens.sum())} pool={c.num_blocks}")
    err = pb.check_output(kvb, oracle, w, c, run(kvb, w, c, kvb.config_part(cfg, w)))
    progress(f"[parity] {name}: max err {err:.3g}")


def test_storage_bounds_c2_f16(gpu, oracle):
    pb.check_storage_bound_f16(gpu, oracle, runner(gpu))


def test_storage_bounds_c3_i8(gpu, oracle):
    pb.check_storage_bound_i8(gpu, oracle, runner(gpu))


@pytest.mark.parametrize("path", pb.GOLDEN, ids=[p.rsplit("/", 1)[-1] for p in pb.GOLDEN])
def test_golden(gpu, oracle, path):
    pb.check_golden(gpu, oracle, runner(gpu), path)


@pytest.mark.parametrize("kv", ["f32", "f16", "i8"])
@pytest.mark.parametrize("page,part", pb.DOMINANT_LAYOUTS)
def test_dominant_key_gather_is_exact(gpu, kv, page, part):
    pb.check_dominant_key(gpu, runner(gpu), kv, page, part)


def test_workspace_partition_indexing(gpu, oracle):
    pb.check_workspace_partitions(gpu, oracle, lambda w, c, part: run_ws(gpu, w, c, part))


@pytest.mark.parametrize("kv", ["f32", "f16", "i8"])
def test_ragged_any_page_and_partition(gpu, oracle, kv):
    pb.check_ragged(gpu, oracle, runner(gpu), kv)


@pytest.mark.parametrize("shape", pb.GQA_SHAPES)
def test_gqa_groups(gpu, oracle, shape):
    pb.check_gqa(gpu, oracle, runner(gpu), shape)


@pytest.mark.parametrize("kv", ["f32", "f16", "i8"])
def test_huge_and_tiny_queries(gpu, oracle, kv):
    pb.check_huge_and_tiny_queries(gpu, oracle, runner(gpu), kv)


@pytest.mark.parametrize("kv", ["f16", "i8"])
def test_huge_and_tiny_values(gpu, oracle, kv):
    pb.check_huge_and_tiny_values(gpu, oracle, runner(gpu), kv)


@pytest.mark.parametrize("kv", ["f32", "f16", "i8"])
def test_ragged_batch_equals_each_sequence_alone(gpu, kv):
    """A ragged batch runs in the longest-first work order (grid y enumerates partitions, the
    largest first); a batch of one runs in the plain (sequence, partition) grid. Every partition is
    computed by the same code either way, so each sequence's output in the batch must equal its
    output run alone bit for bit, fused and two-kernel: a partition computed twice, skipped, or
    given to the wrong sequence cannot pass."""
    kvb = gpu
    lens = [0, 1, 255, 256, 257, 1000, 4096, 5000, 63, 0, 2049, 700]
    part = 256
    w = kvb.Workload(kvb.Shape(len(lens), 8, 2, 128), kv, lens, seed=101, varied=(kv == "i8"))
    c = kvb.PagedCache(w, 16, 5, pool_factor=1.5, poison=True)
    dev = kvb.DeviceCase(w, c)
    dev.out.fill(0xFF)
    dev.run(part)
    fused = dev.output()
    dev.out.fill(0xFF)
    dev.run_split(part)
    assert np.array_equal(fused, dev.output())
    dev.free()
    for b, L in enumerate(lens):
        n = max(L, 1)
        one = kvb.Workload.from_arrays(kv, [L], w.q[b:b + 1], w.k[b:b + 1, :, :n], w.v[b:b + 1, :, :n])
        d1 = kvb.DeviceCase(one, kvb.PagedCache(one, 16, 7 + b, pool_factor=1.5, poison=True))
        d1.out.fill(0xFF)
        d1.run(part)
        assert np.array_equal(d1.output()[0], fused[b]), (b, L)
        d1.free()


@pytest.mark.parametrize("batch", [2, 65, 300, 512, 513])
def test_ragged_order_at_every_batch_width(gpu, oracle, batch):
    """The longest-first order keeps one lane per sequence and up to 8 sequences per lane (512);
    513 sequences fall back to the plain grid. Random lengths with empty and exact-multiple ones,
    against the oracle; empty sequences exactly 0."""
    kvb = gpu
    g = np.random.Generator(np.random.PCG64(batch))
    lens = g.integers(0, 400, size=batch)
    lens[::7] = 0
    lens[1::11] = 128
    lens[0] = 399
    w = kvb.Workload(kvb.Shape(batch, 4, 2, 64), "f16", lens.tolist(), seed=batch)
    c = kvb.PagedCache(w, 16, batch, pool_factor=1.25, poison=True)
    want, tol = pb.expected(kvb, oracle, w, c)
    for part in (64, 1000):
        got = run(kvb, w, c, part)
        assert oracle.max_abs_diff(got, want) <= tol, part
        for b in np.flatnonzero(w.lens == 0):
            assert not got[b].any(), (part, b)


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


def test_stream_switch_orders_queued_steps(gpu):
    """kvb_set_stream while steps are still queued on the previous stream. Every stream shares the
    library's split-K workspace and fused-merge counters, so the new stream must wait for the old
    one. Two cases queued on alternating streams in pipelined mode (nothing waits in between) give
    the bits each gives alone, three times over."""
    import ctypes
    kvb = gpu
    hiprt = ctypes.CDLL("libamdhip64.so")  # the HIP runtime libkvb_hip already loaded
    streams = [ctypes.c_void_p(), ctypes.c_void_p()]
    for s in streams:
        assert hiprt.hipStreamCreate(ctypes.byref(s)) == 0
    cases = []
    for i, lens in enumerate(([16384, 16384], [9000, 3000, 12000])):
        w = kvb.Workload(kvb.Shape(len(lens), 32, 8, 128), "f16", lens, seed=80 + i)
        dev = kvb.DeviceCase(w, kvb.PagedCache(w, 16, 7 + i, pool_factor=1.5))
        dev.run(1024)
        cases.append((dev, dev.output()))
    try:
        for rep in range(3):
            progress(f"[parity] stream switch, round {rep}")
            for dev, _ in cases:
                dev.out.fill(0xFF)
            kvb.begin_pipelined()
            for i in range(4):
                kvb.set_stream(streams[i % 2])
                cases[i % 2][0].run(1024)
            kvb.set_stream(None)
            assert len(kvb.end_pipelined()) == 4
            for dev, want in cases:
                assert np.array_equal(dev.output(), want)
    finally:
        kvb.set_stream(None)
        kvb.synchronize()
        for s in streams:
            hiprt.hipStreamDestroy(s)
        for dev, _ in cases:
            dev.free()


@pytest.mark.parametrize("kv", ["f32", "f16", "i8"])
def test_loads_only_decode(gpu, kv):
    """kvb_run_paged_loads (the decode's loads, no arithmetic) runs on equal and ragged lengths,
    reports a GPU time, leaves the output untouched, and a decode step afterwards is unchanged."""
    kvb = gpu
    for lens in ([2048, 2048, 2048], [2048, 17, 0]):
        w = kvb.Workload(kvb.Shape(3, 32, 8, 128), kv, lens, seed=91)
        c = kvb.PagedCache(w, 16, 5, pool_factor=1.5)
        dev = kvb.DeviceCase(w, c)
        dev.run(256)
        want = dev.output()
        dev.out.fill(0x7F)
        sentinel = dev.output()
        progress(f"[parity] loads-only {kv} lens {lens}")
        assert dev.run_loads(256) > 0
        assert np.array_equal(dev.output(), sentinel, equal_nan=True)
        dev.run(256)
        assert np.array_equal(dev.output(), want)
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


@pytest.mark.parametrize("kv,part", pb.MANY_PARTITIONS)
def test_many_partitions(gpu, oracle, kv, part):
    """Partition counts below, at and past what the fused merge stages in LDS (1024 (m, l) pairs
    for f16 and i8 at head_dim 64, 4096 for f32): with 8 heads per group, f16 part 64 (64
    partitions) is below it, f16 and i8 part 32 (128) fill it exactly, f16 and i8 part 16 (256)
    exceed it and the runtime merges with paged_reduce as a second kernel. The fused output equals
    the two-kernel output bit for bit."""
    kvb = gpu
    got = pb.check_many_partitions(kvb, oracle, runner(kvb), kv, part)
    w, c = pb.many_partitions_case(kvb, kv)
    dev = kvb.DeviceCase(w, c)
    dev.run_split(part)
    assert np.array_equal(got, dev.output())
    dev.free()


@pytest.mark.parametrize("kv,part", pb.MANY_PARTITIONS_D128)
def test_many_partitions_head_dim_128(gpu, oracle, kv, part):
    """64 and 24 partitions at head_dim 128 (4 query heads per KV head): the fused merge's batches at
    head_dim 128 against the oracle, and bit for bit against the two-kernel form."""
    kvb = gpu
    got = pb.check_many_partitions(kvb, oracle, runner(kvb), kv, part, head_dim=128)
    w, c = pb.many_partitions_case(kvb, kv, head_dim=128)
    dev = kvb.DeviceCase(w, c)
    dev.run_split(part)
    assert np.array_equal(got, dev.output())
    dev.free()


def test_read_bandwidth_probe(gpu):
    kvb = gpu
    buf = kvb.Buffer(1 << 30)
    buf.fill(1)
    ms = kvb.run_read_bandwidth(buf)
    gbps = (1 << 30) / (ms * 1e-3) / 1e9
    progress(f"[parity] read probe 1 GiB: {gbps:.0f} GB/s")
    assert 500 < gbps < 12000
    buf.free()


def random_case(i):
    """Layout i of a fixed pseudo-random sweep: storage type, shape, lengths (with 0, 1 and tile,
    page and partition edges mixed in), page size (tile-aligned or not), partition (automatic,
    tile-aligned or not), pool size and scale variation."""
    r = np.random.RandomState(1000 + i)
    kv = ["f32", "f16", "i8"][i % 3]
    hkv = int(r.choice([1, 2, 4, 8]))
    g = int(r.choice([1, 2, 3, 4, 8]))
    d = int(r.choice([64, 128]))
    b = int(r.randint(1, 7))
    page = int(r.choice([16, 32, 64, 128, 1, 3, 24, 48]))
    part = int(r.choice([0, 16, 64, 256, 1024, 7, 100]))
    edges = [0, 1, 15, 16, 17, 31, 32, 33, page, page + 1, max(part, 1), max(part, 1) + 1]
    lens = [int(r.choice(edges)) if r.rand() < 0.4 else int(r.randint(0, 3000)) for _ in range(b)]
    return kv, (b, hkv * g, hkv, d), lens, page, part, float(r.choice([1.0, 1.5, 3.0])), bool(r.rand() < 0.5)


@pytest.mark.parametrize("i", range(30))
def test_random_layouts(gpu, oracle, i):
    """A fixed sweep of 30 layouts: the fused step against the oracle (tolerance) and against the
    two-kernel step (bit for bit), with and without one workgroup per GQA group; where the
    layout is tile-aligned, the loads-only variant runs too and leaves the output untouched."""
    kvb = gpu
    kv, shape, lens, page, part, pool, varied = random_case(i)
    progress(f"[parity] random {i}: {kv} shape {shape} page {page} part {part} lens {lens}")
    w = kvb.Workload(kvb.Shape(*shape), kv, lens, seed=2000 + i, varied=varied and kv == "i8")
    c = kvb.PagedCache(w, page, 3000 + i, pool_factor=pool, poison=True)
    dev = kvb.DeviceCase(w, c)
    dev.out.fill(0xFF)
    dev.run(part)
    fused = dev.output()
    pb.check_output(kvb, oracle, w, c, fused)
    dev.out.fill(0xFF)
    dev.run_split(part)
    assert np.array_equal(dev.output(), fused)
    dev.out.fill(0xFF)
    dev.run(part, share_kv=False)
    pb.check_output(kvb, oracle, w, c, dev.output())
    eff = part if part else kvb.auto_part_tokens(w.shape.batch, w.shape.num_kv_heads, w.max_len)
    if page % 16 == 0 and eff % 16 == 0:
        dev.out.fill(0x7F)
        sentinel = dev.output()
        assert dev.run_loads(part) > 0
        assert np.array_equal(dev.output(), sentinel)
    dev.free()


@pytest.mark.parametrize("kv", ["f32", "f16", "i8"])
def test_non_finite_query_poisons_only_its_head(gpu, oracle, kv):
    """A NaN (or infinite) element of one head's q makes that head's output NaN, as floating point
    does, and leaves the other heads of its group exact to the tolerance."""
    kvb = gpu
    w = kvb.Workload(kvb.Shape(2, 8, 2, 128), kv, [300, 40], seed=61)
    c = kvb.PagedCache(w, 16, 9, pool_factor=1.5, poison=True)
    clean, tol = pb.expected(kvb, oracle, w, c)
    for bad in (np.nan, np.inf):
        w.q[0, 1, 17] = bad
        got = run(kvb, w, c, 64)
        assert np.isnan(got[0, 1]).all(), bad
        keep = np.ones(got.shape[:2], bool)
        keep[0, 1] = False
        assert np.abs(got[keep] - clean[keep]).max() <= tol, bad
        w.q[0, 1, 17] = 0.5


@pytest.mark.parametrize("kv", ["f32", "f16", "i8"])
def test_any_page_table_staged_and_not(gpu, oracle, kv):
    """The any-page path (page or partition not a multiple of 16) copies a workgroup's block ids
    into LDS when its range touches at most kTableStage (4096) blocks, and reads the table in
    memory otherwise. Page 1: a 4096-token partition stages exactly 4096 ids; a 5000-token one
    touches 5000 and does not; page 7 with a partition of 100 stages 16."""
    kvb = gpu
    for page, part, lens in ((1, 4096, [4096, 1000]), (1, 5000, [6000, 333]), (7, 100, [777, 50])):
        w = kvb.Workload(kvb.Shape(len(lens), 8, 2, 64), kv, lens, seed=page * 1000 + part, varied=(kv == "i8"))
        c = kvb.PagedCache(w, page, part + 3, pool_factor=1.25, poison=True)
        got = run(kvb, w, c, part)
        err = pb.check_output(kvb, oracle, w, c, got)
        progress(f"[any-page] {kv} page {page} part {part}: max err {err:.3g}")
