"""GQA groups other than 1, 2, 4 and 8 (3, 5, 6, 7, 9, 12, 14, 16, 32). One paged_decode workgroup serves
kvb_heads_per_workgroup query heads of a KV head: 16 or 32 where they divide the group (fp16 and
int8), else the largest divisor of the group that is at most 8, so it reads each K/V page once for
all of them (src/metal_attn.mm:64-80 builds its kernel with QG = GROUP for any group). Up to 8
heads it runs the kernel built for the next of 1, 2, 4 and 8 heads, whose MFMA columns past those
heads stay idle; 16 heads run as one 16-head wave per token stream, 32 as two head splits of
16-head waves (fp16: the two waves of a stream share each tile through LDS, one loading its K rows
and the other its V rows). Checked for every storage type:
- the output against the oracle, on the plain grid (fused merge, one and two partitions per
  workgroup), the ragged grid, and a layout whose page is not a tile multiple;
- the fused step against the two-kernel form, bit for bit;
- every workspace slot against the oracle's partition state;
- groups of 16: each 8 of the heads (of the one f16 or i8 workgroup of 16-head waves, or of the two
  f32 workgroups, which run on one XCD and read with ordinary loads) against a group-8 run of the
  same heads (f32 bit for bit, f16 and i8 to fp32 rounding);
- 16 and 32 heads per workgroup past 16 partitions (the fused merge's many-partition form, or
  paged_reduce where the group's output has more chunks than the workgroup has threads)."""
import numpy as np
import pytest

import parity_battery as pb
from conftest import progress

pytestmark = pytest.mark.gpu

# (B, H, Hkv, D) -> query heads per workgroup (f16 and i8; f32 caches take at most 8)
SHAPES = [
    ((2, 24, 8, 128), 3),   # the 4-head build, one column pair idle
    ((2, 10, 2, 64), 5),    # the 8-head build from here on
    ((2, 12, 2, 128), 6),
    ((2, 56, 8, 128), 7),
    ((1, 24, 2, 128), 6),   # group 12: two workgroups per KV head
    ((1, 28, 2, 64), 7),    # group 14: two workgroups per KV head
    ((1, 18, 2, 64), 3),    # group 9: three workgroups of 3 per KV head
    ((1, 32, 2, 128), 16),  # group 16: 16-head waves (f32: two workgroups of 8)
    ((1, 64, 2, 128), 32),  # group 32: two head splits of 16-head waves, f16 sharing tiles (f32: four of 8)
    ((2, 32, 1, 64), 32),   # group 32, one KV head, head_dim 64
]
IDS = [f"H{s[1]}-Hkv{s[2]}-D{s[3]}" for s, _ in SHAPES]

# lengths, page, partition: equal lengths over several partitions (fused merge; pair mode possible
# at 256), ragged lengths (longest-first work items), and a page that is not a multiple of 16 (each
# lane finds its own token's block)
LAYOUTS = [("equal", 16, 256), ("ragged", 32, 128), ("any-page", 24, 100)]


def lengths(kind, batch):
    if kind == "equal":
        return [1000] * batch
    if kind == "ragged":
        return [777, 65, 0, 1][:batch] if batch > 1 else [777]
    return [500, 201][:batch]


@pytest.fixture
def pair_restored(gpu):
    prev = gpu.set_pair_mode("auto")
    yield gpu
    gpu.set_pair_mode(prev)


@pytest.mark.parametrize("kv", ["f32", "f16", "i8"])
@pytest.mark.parametrize("shape,qg", SHAPES, ids=IDS)
def test_groups_match_the_oracle(pair_restored, oracle, shape, qg, kv):
    kvb = pair_restored
    s = kvb.Shape(*shape)
    qg = qg if kv != "f32" else min(qg, 8)
    assert kvb.heads_per_workgroup(s, kv) == qg
    for kind, page, part in LAYOUTS:
        w = kvb.Workload(s, kv, lengths(kind, s.batch), seed=qg * 97 + page, varied=(kv == "i8"))
        c = kvb.PagedCache(w, page, 13 * page + qg, pool_factor=1.5, poison=True)
        modes = ("off", "always") if kind == "equal" and kv != "f32" else ("auto",)
        outs = []
        for mode in modes:
            kvb.set_pair_mode(mode)
            dev = kvb.DeviceCase(w, c)
            dev.out.fill(0xFF)  # NaN: every output element must be written
            dev.run(part)
            fused = dev.output().copy()
            dev.out.fill(0xFF)
            dev.run_split(part)
            split = dev.output().copy()
            dev.free()
            assert np.array_equal(fused.view(np.uint32), split.view(np.uint32)), (kind, mode)
            outs.append(fused)
        for o in outs[1:]:  # two partitions per workgroup: the same bits as one
            assert np.array_equal(o.view(np.uint32), outs[0].view(np.uint32)), kind
        err = pb.check_output(kvb, oracle, w, c, outs[0])
        progress(f"[groups] {shape} {kv} {kind}: qg {qg}, max err {err:.3g}")


@pytest.mark.parametrize("kv", ["f16", "i8"])
@pytest.mark.parametrize("shape,qg", [SHAPES[i] for i in (0, 3, 5, 7, 9)], ids=[IDS[i] for i in (0, 3, 5, 7, 9)])
def test_groups_workspace_slots(gpu, oracle, shape, qg, kv):
    """Every (sequence, head, partition) slot: the oracle's (m, l, o) where the partition holds
    tokens, untouched (NaN) elsewhere. A head's slot depends on its own index only, so a workgroup
    of qg heads writes exactly its heads' slots."""
    kvb = gpu
    s = kvb.Shape(*shape)
    lens = [300, 65][: s.batch]
    part = 64
    w = kvb.Workload(s, kv, lens, seed=5 + qg, varied=(kv == "i8"))
    s = w.shape
    c = kvb.PagedCache(w, 16, 7, pool_factor=1.5, poison=True)
    dev = kvb.DeviceCase(w, c)
    max_parts = dev.max_parts(part)
    ws = kvb.Buffer(dev.workspace_bytes(part))
    ws.fill(0xFF)
    dev.run(part, workspace=ws)
    B, H, D = s.batch, s.num_heads, s.head_dim
    raw = ws.download(np.float32, ws.nbytes // 4)
    part_out = raw[: B * H * max_parts * D].reshape(B, H, max_parts, D)
    part_ml = raw[B * H * max_parts * D: B * H * max_parts * (D + 2)].reshape(B, H, max_parts, 2)
    dev.free()
    ws.free()
    kd, vd = c.dequantized(w) if kv == "i8" else (w.k, w.v)
    vmax = float(np.abs(np.asarray(vd, np.float32)).max())
    for b in range(B):
        for h in range(H):
            for p in range(max_parts):
                st = oracle.partition_state(s, w.lens, w.max_len, w.q, kd, vd, part, b, h, p)
                if st is None:
                    assert np.isnan(part_out[b, h, p]).all() and np.isnan(part_ml[b, h, p]).all(), (b, h, p)
                    continue
                m, l, o = st
                assert abs(part_ml[b, h, p, 0] - m) <= 1e-5 * max(1.0, abs(m)), (b, h, p)
                assert abs(part_ml[b, h, p, 1] - l) <= 1e-5 * l, (b, h, p)
                assert np.abs(part_out[b, h, p] - o).max() <= 2e-5 * max(1.0, vmax), (b, h, p)
    progress(f"[groups] workspace {shape} {kv}: qg {qg}, {B * H * max_parts} slots")


@pytest.mark.parametrize("kv", ["f16", "i8", "f32"])
# (KV head, sequence or work item, partition) units: 16, 32, 24 and 64 fill blocks of 8 (the
# sibling order); the ragged [500, 300, 120] at 160 has 2 x 7 = 14 (the plain order)
@pytest.mark.parametrize("lens,part", [([1000, 1000], 256), ([1000, 1000], 128), ([777, 65, 300, 1], 128),
                                       ([4096, 4096, 4096, 4096], 512), ([500, 300, 120], 160)])
def test_sibling_workgroups_give_group8_bits(gpu, kv, lens, part):
    """Group 16: f16 and i8 run one workgroup of 16-head waves per KV head (one head per score
    column, the high and low parts in separate MFMAs), f32 two workgroups of 8 (with the sibling
    order when the (KV head, sequence, partition) units fill blocks of 8, else without it). Each 8
    of the 16 heads give the result of a group-8 run over the same K/V with those heads as the group:
    bit for bit for f32; for f16 and i8 to fp32 rounding (2e-7 of max(1, max |v|)), as a 16-head wave
    rescales its accumulators lazily (the p are taken against a reference max that lags the running
    max by up to 2^8) and the compiler forms the int8 p split from the exact or the rounded product
    per build. (A high part the MFMA received that differed from the one its low part was taken
    against once showed here as 2.3e-6.)"""
    kvb = gpu
    B = len(lens)
    w16 = kvb.Workload(kvb.Shape(B, 32, 2, 128), kv, lens, seed=len(lens) * 31 + part)
    k, v = w16.k, w16.v  # as stored (fp16) or before quantisation (int8, fp32)
    c16 = kvb.PagedCache(w16, 16, 3, pool_factor=1.5, poison=True)
    dev = kvb.DeviceCase(w16, c16)
    dev.out.fill(0xFF)
    dev.run(part)
    out16 = dev.output().copy()
    units = 2 * B * dev.max_parts(part)
    dev.free()
    for half in (0, 1):
        heads = [16 * g + 8 * half + j for g in range(2) for j in range(8)]
        w8 = kvb.Workload.from_arrays(kv, lens, w16.q[:, heads], k, v)
        c8 = kvb.PagedCache(w8, 16, 5, pool_factor=1.5, poison=True)
        if kv == "i8":  # the same pages give the same bytes and scales
            assert np.array_equal(c8.dequantized(w8)[0], c16.dequantized(w16)[0])
        d8 = kvb.DeviceCase(w8, c8)
        d8.out.fill(0xFF)
        d8.run(part)
        out8 = d8.output()
        d8.free()
        if kv == "f32":
            assert np.array_equal(out16[:, heads].view(np.uint32), out8.view(np.uint32)), half
        else:
            vmax = float(np.abs(c16.dequantized(w16)[1] if kv == "i8" else v.astype(np.float32)).max())
            d = float(np.abs(out16[:, heads] - out8).max())
            progress(f"[groups]   {kv} 16-head against 8-head waves: max |diff| {d:.3g} (max |v| {vmax:.3g})")
            assert d <= 2e-7 * max(1.0, vmax), half
    progress(f"[groups] group 16 = 2 x group 8, {kv} lens {lens} part {part} ({units} units)")


@pytest.mark.parametrize("kv", ["f16", "i8"])
def test_sixteen_head_waves_keep_each_eight_heads_precision(gpu, kv):
    """A 16-head wave takes q's power-of-two scale per 8 heads (fp16; int8 per head), as two 8-head
    waves would. Heads 0-7 of each group with |q| near 2^10 and heads 8-15 near 2^-12, over K near
    2^10 so that the small heads' scores still spread their softmax: one scale for all 16 would put
    the small heads' low fp16 parts among the subnormals (about 1e-5 in their p). Each 8 of the 16
    heads against a group-8 run of the same heads, to fp32 rounding (2e-7 of max(1, max |v|))."""
    kvb = gpu
    rng = np.random.default_rng(2026 + len(kv))
    B, H, Hkv, D, lens = 2, 32, 2, 128, [700, 333]
    q = rng.standard_normal((B, H, D)).astype(np.float32)
    for g in range(H // 16):
        q[:, 16 * g:16 * g + 8] *= 2.0 ** 10
        q[:, 16 * g + 8:16 * g + 16] *= 2.0 ** -12
    k = (rng.standard_normal((B, Hkv, max(lens), D)) * 2.0 ** 10).astype(np.float32)
    v = rng.standard_normal((B, Hkv, max(lens), D)).astype(np.float32)
    w16 = kvb.Workload.from_arrays(kv, lens, q, k, v)
    assert kvb.heads_per_workgroup(w16.shape, kv) == 16
    c16 = kvb.PagedCache(w16, 16, 3, pool_factor=1.5, poison=True)
    dev = kvb.DeviceCase(w16, c16)
    dev.run(256)
    out16 = dev.output().copy()
    dev.free()
    vmax = float(np.abs(c16.dequantized(w16)[1] if kv == "i8" else w16.v.astype(np.float32)).max())
    for half in (0, 1):
        heads = [16 * g + 8 * half + j for g in range(H // 16) for j in range(8)]
        w8 = kvb.Workload.from_arrays(kv, lens, q[:, heads], w16.k, w16.v)
        c8 = kvb.PagedCache(w8, 16, 5, pool_factor=1.5, poison=True)
        d8 = kvb.DeviceCase(w8, c8)
        d8.run(256)
        out8 = d8.output()
        d8.free()
        d = float(np.abs(out16[:, heads] - out8).max())
        progress(f"[groups] {kv} heads of 2^10 and 2^-12 in one 16-head wave, half {half}: max |diff| {d:.3g}")
        assert d <= 2e-7 * max(1.0, vmax), half


@pytest.mark.parametrize("kv", ["f16", "i8"])
@pytest.mark.parametrize("heads,dim", [(32, 128), (64, 128), (64, 64)], ids=["g16", "g32", "g32-D64"])
def test_wide_groups_past_sixteen_partitions(gpu, oracle, kv, heads, dim):
    """16 and 32 heads per workgroup past 16 partitions. The fused merge of more than 16 gives each
    thread one chunk of the group's output; a workgroup with more chunks than threads (f16 16 or 32
    heads at head_dim 128, i8 32 heads at head_dim 128) leaves that merge to paged_reduce. Against
    the oracle, and fused (requested) equal to two-kernel."""
    kvb = gpu
    w = kvb.Workload(kvb.Shape(2, heads, 2, dim), kv, [1000, 333], seed=77 + heads + dim, varied=(kv == "i8"))
    assert kvb.heads_per_workgroup(w.shape, kv) == heads // 2
    c = kvb.PagedCache(w, 16, 9, pool_factor=1.5, poison=True)
    for part in (32, 64):  # 32 and 16 partitions
        dev = kvb.DeviceCase(w, c)
        dev.out.fill(0xFF)
        dev.run(part)
        fused = dev.output().copy()
        dev.out.fill(0xFF)
        dev.run_split(part)
        split = dev.output().copy()
        dev.free()
        assert np.array_equal(fused.view(np.uint32), split.view(np.uint32)), part
        err = pb.check_output(kvb, oracle, w, c, fused)
        progress(f"[groups] {heads // 2} heads, D {dim}, {kv}, part {part}: max err {err:.3g}")


# (B, H, Hkv, D), lengths, page, partitions
LONG_CASES = [
    ((2, 64, 2, 128), [4000, 2333], 16, (1024, 2048, 4096)),
    ((2, 64, 1, 64), [3000, 17], 128, (1024, 3072)),
    ((1, 128, 2, 128), [2500], 64, (1024, 2048)),  # group 64: two 32-head workgroups per KV head
    ((2, 64, 2, 128), [1500, 900], 24, (512, 1024)),  # a page that is not a multiple of 16
]


@pytest.mark.parametrize("kv", ["f16", "i8"])
@pytest.mark.parametrize("case", range(len(LONG_CASES)))
def test_shared_tiles_long_partitions(gpu, oracle, case, kv):
    """Groups of 32 and 64 over partitions of up to eight tiles per stream, whose streams end their
    walks at different steps (fp16: the two head splits of a stream share each tile through LDS,
    the stream's two slots reused round after round). Against the oracle; fused equal to
    two-kernel."""
    kvb = gpu
    shape, lens, page, parts = LONG_CASES[case]
    w = kvb.Workload(kvb.Shape(*shape), kv, lens, seed=501 + case, varied=(kv == "i8"))
    assert kvb.heads_per_workgroup(w.shape, kv) == 32
    c = kvb.PagedCache(w, page, 11 * page + case, pool_factor=1.5, poison=True)
    for part in parts:
        dev = kvb.DeviceCase(w, c)
        dev.out.fill(0xFF)
        dev.run(part)
        fused = dev.output().copy()
        dev.out.fill(0xFF)
        dev.run_split(part)
        split = dev.output().copy()
        dev.free()
        assert np.array_equal(fused.view(np.uint32), split.view(np.uint32)), part
        err = pb.check_output(kvb, oracle, w, c, fused)
        progress(f"[shared tiles] {kv} {shape} lens {lens} page {page} part {part}: max err {err:.3g}")


@pytest.mark.parametrize("kv", ["f16", "i8"])
@pytest.mark.parametrize("heads", [32, 64])
def test_loads_only_wide_groups(gpu, kv, heads):
    """kvb_run_paged_loads on 16- and 32-head workgroups (fp16 32: the shared tiles' half-tile
    loads) reports a GPU time, leaves the output untouched, and a decode step afterwards is
    unchanged."""
    kvb = gpu
    w = kvb.Workload(kvb.Shape(2, heads, 2, 128), kv, [2048, 700], seed=61 + heads)
    c = kvb.PagedCache(w, 16, 7, pool_factor=1.5)
    dev = kvb.DeviceCase(w, c)
    dev.run(512)
    want = dev.output()
    dev.out.fill(0x7F)
    sentinel = dev.output()
    progress(f"[shared tiles] loads-only {kv} {heads // 2} heads per workgroup")
    assert dev.run_loads(512) > 0
    assert np.array_equal(dev.output(), sentinel, equal_nan=True)
    dev.run(512)
    assert np.array_equal(dev.output(), want)
    dev.free()
