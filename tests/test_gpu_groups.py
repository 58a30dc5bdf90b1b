"""GQA groups that are not powers of two (3, 5, 6, 7, 12, 14). One paged_decode workgroup serves
kvb_heads_per_workgroup query heads of a KV head, the largest divisor of the group that is at most
8, so it reads each K/V page once for all of them (src/metal_attn.mm:64-80 builds its kernel with
QG = GROUP for any group). It runs the kernel built for the next of 1, 2, 4 and 8 heads, whose
MFMA columns past those heads stay idle. Checked for every storage type:
- the output against the oracle, on the plain grid (fused merge, one and two partitions per
  workgroup), the ragged grid, and a layout whose page is not a tile multiple;
- the fused step against the two-kernel form, bit for bit;
- every workspace slot against the oracle's partition state."""
import numpy as np
import pytest

import parity_battery as pb
from conftest import progress

pytestmark = pytest.mark.gpu

# (B, H, Hkv, D) -> query heads per workgroup
SHAPES = [
    ((2, 24, 8, 128), 3),   # the 4-head build, one column pair idle
    ((2, 10, 2, 64), 5),    # the 8-head build from here on
    ((2, 12, 2, 128), 6),
    ((2, 56, 8, 128), 7),
    ((1, 24, 2, 128), 6),   # group 12: two workgroups per KV head
    ((1, 28, 2, 64), 7),    # group 14: two workgroups per KV head
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
    assert kvb.heads_per_workgroup(s) == qg
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
@pytest.mark.parametrize("shape,qg", [SHAPES[0], SHAPES[3], SHAPES[5]], ids=[IDS[0], IDS[3], IDS[5]])
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
