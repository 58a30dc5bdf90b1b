"""The decode path's parity checks, written once against a runner.

tests/test_gpu_parity.py runs them on the HIP kernels through the C ABI. tests/test_split_model.py
runs them on the oracle's CPU model of the same split-K kernel (kvbo_split_decode), where
tests/mutation/mutate.py plants the reference's kernel mistakes (scripts/mutation.sh:47-59): a
planted mistake counts as caught when these checks fail on it.

A runner is ``run(w, c, part, share_kv) -> out [B][H][D]`` (float32). The workspace check takes
``run_ws(w, c, part) -> (out, part_out [B][H][max_parts][D], part_ml [B][H][max_parts][2])``, with every
workspace slot NaN before the run.

Tolerance (the reference's tests/gpu_tests.cpp:13-17, scaled for |v| > 1): kernel vs oracle on the
same stored values <= 2e-5 * max(1, max|v|); fp32 storage also <= 1e-4 relative to max|out|. Gathers
through the block table and partition indexing are checked bit for bit.
"""
import glob
import os

import numpy as np

from conftest import ROOT

THREADS = 16
GOLDEN = sorted(glob.glob(os.path.join(ROOT, "tests", "golden", "*.npz")))
DOMINANT_LAYOUTS = [(16, 0), (16, 48), (64, 128), (1, 16), (3, 7), (24, 100)]
RAGGED_LENS = [0, 1, 15, 16, 17, 63, 64, 65, 129, 300, 2, 0]
RAGGED_LAYOUTS = [(1, 0), (3, 5), (8, 100), (16, 16), (32, 0), (48, 96), (64, 1)]
GQA_SHAPES = [(2, 8, 8, 128), (2, 12, 4, 64), (2, 32, 2, 128), (2, 6, 2, 64)]
MANY_PARTITIONS = [("f16", 16), ("f16", 32), ("f16", 64), ("f32", 16), ("i8", 16), ("i8", 32)]
# head_dim 128, 4 query heads per KV head, 128-token partitions: 64 and 24 partitions per sequence,
# the fused merge's batched form at its head_dim-128 batch size (the reference's own sweep runs 64
# partitions at 32k tokens)
MANY_PARTITIONS_D128 = [("f16", 128), ("f32", 128), ("i8", 128)]


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


def check_output(kvb, oracle, w, c, got):
    """A full output against the oracle: tolerance, fp32 relative bound, exact zeros of empty
    sequences. Returns the error."""
    want, tol = expected(kvb, oracle, w, c)
    err = oracle.max_abs_diff(got, want)
    assert err <= tol, f"max err {err:.3g} > tol {tol:.3g}"
    if w.kv_type == kvb.KV_F32:
        assert err <= 1e-4 * float(np.abs(want).max())
    for b in np.flatnonzero(w.lens == 0):
        assert not got[b].any()
    return err


def check_golden(kvb, oracle, run, path):
    """The reference-derived fixtures (tests/golden/make_golden.py) at three partition sizes."""
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
        got = run(w, c, part, True)
        assert oracle.max_abs_diff(got, g["out"]) <= 2e-5 * max(1.0, vmax), (part,)


def check_dominant_key(kvb, run, kv, page, part):
    """q = 1000 e_0 and a one-hot key make the softmax exactly one-hot: the output must be the hot
    token's V row bit for bit, through the shuffled block table and every partition merge."""
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
    got = run(w, c, part, True)
    vals = c.dequantized(w)[1] if kv == "i8" else w.v.astype(np.float32)
    for b, t in enumerate(hot):
        for h in range(16):
            assert np.array_equal(got[b, h], vals[b, h // 8, t]), (b, h)


def check_workspace_partitions(kvb, oracle, run_ws):
    """Every (sequence, head, partition) slot of the workspace: written with the oracle's (m, l, o)
    iff the partition holds tokens, untouched (NaN) otherwise."""
    lens, part = [200, 65, 0, 64], 64
    w = kvb.Workload(kvb.Shape(4, 8, 2, 128), "f32", lens, seed=21)
    c = kvb.PagedCache(w, 16, 5, pool_factor=2.0, poison=True)
    got, part_out, part_ml = run_ws(w, c, part)
    B, H, max_parts = 4, 8, part_out.shape[2]
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
    want = oracle.attention(w.shape, w.lens, w.max_len, w.q, w.k, w.v)
    assert oracle.max_abs_diff(got, want) <= 2e-5


def check_ragged(kvb, oracle, run, kv):
    """Lengths around tile, page and partition edges (0, 1, 15, 16, 17, ...), at seven page and
    partition sizes, with and without one workgroup per GQA group."""
    w = kvb.Workload(kvb.Shape(1, 8, 2, 64), kv, RAGGED_LENS, seed=31, varied=(kv == "i8"))
    for page, part in RAGGED_LAYOUTS:
        c = kvb.PagedCache(w, page, page * 7, pool_factor=3.0, poison=True)
        want, tol = expected(kvb, oracle, w, c)
        for share in (True, False):
            got = run(w, c, part, share)
            assert oracle.max_abs_diff(got, want) <= tol, (page, part, share)
            for b in np.flatnonzero(w.lens == 0):
                assert not got[b].any(), (page, part, share)


def check_gqa(kvb, oracle, run, shape):
    """Groups 1, 3, 16 and 3: query heads per workgroup chosen from {8,4,2,1} dividing the group."""
    w = kvb.Workload(kvb.Shape(*shape), "f16", [333, 1000], seed=41, dist="normal", q_amp=1.0)
    c = kvb.PagedCache(w, 16, 3, pool_factor=1.25, poison=True)
    want, tol = expected(kvb, oracle, w, c)
    assert oracle.max_abs_diff(run(w, c, 256, True), want) <= tol


def check_huge_and_tiny_queries(kvb, oracle, run, kv="f16"):
    """q far from 1 in magnitude, over the whole query and per head inside one GQA group: the fp16
    high/low split scales q by a power of two per wave, the int8 digits per head. With one scale
    for the group, the 1.0 head's int8 digits would be fixed point on the 8000 head's scale."""
    w = kvb.Workload(kvb.Shape(2, 8, 2, 128), kv, [500, 20], seed=51)
    c = kvb.PagedCache(w, 16, 3, poison=True)
    for amp in (8000.0, 1e-3, 3e-6, "mixed"):
        rng = np.random.Generator(np.random.PCG64(7))
        if amp == "mixed":  # the 4 heads of each group at 8000, 1, 1e-3 and 30
            a = np.array([8000.0, 1.0, 1e-3, 30.0] * 2, np.float32)
            w.q[:] = (rng.uniform(-1.0, 1.0, w.q.shape) * a[None, :, None]).astype(np.float32)
        else:
            w.q[:] = rng.uniform(-amp, amp, w.q.shape).astype(np.float32)
        want, tol = expected(kvb, oracle, w, c)
        assert oracle.max_abs_diff(run(w, c, 64, True), want) <= tol, amp


def check_huge_and_tiny_values(kvb, oracle, run, kv="i8"):
    """K and V far from 1 in magnitude (1e-7, 1e3): int8 p * v_scale is normalised by the wave's
    largest V-scale power of two before its fp16 split, which at 1e-7 would otherwise underflow;
    fp16 stores the values as subnormals or near its range. Tolerance relative to max|v|."""
    for amp in (1e-7, 1e3):
        base = kvb.Workload(kvb.Shape(2, 8, 2, 128), kv, [300, 77], seed=61, varied=(kv == "i8"))
        dt = base.k.dtype
        k = (base.k.astype(np.float32) * amp).astype(dt)
        v = (base.v.astype(np.float32) * amp).astype(dt)
        w = kvb.Workload.from_arrays(kv, base.lens, base.q, k, v)
        c = kvb.PagedCache(w, 16, 11, pool_factor=1.5, poison=True)
        want, _ = expected(kvb, oracle, w, c)
        vals = c.dequantized(w)[1] if kv == "i8" else w.v.astype(np.float32)
        vmax = max(float(np.abs(vals[b, :, :L]).max()) for b, L in enumerate(w.lens) if L)
        err = oracle.max_abs_diff(run(w, c, 64, True), want)
        assert err <= 2e-5 * vmax, (amp, err, vmax)


def check_storage_bound_f16(kvb, oracle, run):
    """c2's shape (8 x 4096 tokens, N(0,1)): the output against fp64 attention on the unrounded fp32
    data, within the derived fp16 storage bound (tests/gpu_tests.cpp:16-40)."""
    shape = kvb.Shape(8, 32, 8, 128)
    w = kvb.Workload(shape, "f16", [4096] * 8, seed=4096, q_amp=1.0, keep_f32=True, dist="normal", threads=THREADS)
    c = kvb.PagedCache(w, 16, 4096 * 131 + 16, pool_factor=1.5, poison=True)
    got = run(w, c, 512, True)
    exact = oracle.attention(w.shape, w.lens, w.max_len, w.q, w.k32, w.v32, threads=THREADS)
    bound = oracle.fp16_storage_bound(w.shape, w.lens, w.max_len, w.q, w.k32, w.v32)
    assert oracle.max_abs_diff(got, exact) <= bound


def check_storage_bound_i8(kvb, oracle, run):
    """c3's shape (16 x 8192 tokens, page 64, N(0,1)): within the derived int8 storage bound
    (tests/gpu_tests.cpp:42-62)."""
    shape = kvb.Shape(16, 32, 8, 128)
    w = kvb.Workload(shape, "i8", [8192] * 16, seed=8192, q_amp=1.0, dist="normal", threads=THREADS)
    c = kvb.PagedCache(w, 64, 8192 * 131 + 64, poison=True)
    got = run(w, c, 0, True)
    exact = oracle.attention(w.shape, w.lens, w.max_len, w.q, w.k, w.v, threads=THREADS)
    bound = oracle.i8_storage_bound(w.shape, w.lens, 64, c.table, w.q, c.k_scale, c.v_scale)
    assert oracle.max_abs_diff(got, exact) <= bound


def many_partitions_case(kvb, kv, head_dim=64):
    if head_dim == 128:
        w = kvb.Workload(kvb.Shape(2, 32, 8, 128), kv, [8192, 3001], seed=92)
        return w, kvb.PagedCache(w, 32, 92, pool_factor=1.25)
    w = kvb.Workload(kvb.Shape(2, 16, 2, 64), kv, [4096, 2049], seed=91)
    return w, kvb.PagedCache(w, 16, 91, pool_factor=1.25)


def check_many_partitions(kvb, oracle, run, kv, part, head_dim=64):
    """Up to 256 partitions per sequence: the merge over many partitions. Returns the output."""
    w, c = many_partitions_case(kvb, kv, head_dim)
    got = run(w, c, part, True)
    want, tol = expected(kvb, oracle, w, c)
    assert oracle.max_abs_diff(got, want) <= tol
    return got
