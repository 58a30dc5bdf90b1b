"""Two partitions per decode workgroup (kvb_set_pair_mode): the same bits as one partition per
workgroup, for odd partition counts, partial last partitions and a second partition of one token,
in the fused step, the two-kernel form and every workspace slot; and parity with the oracle."""
import numpy as np
import pytest

import parity_battery as pb
from conftest import progress

pytestmark = pytest.mark.gpu

# (B, H, Hkv, D), storage, lengths (equal, so the grid is the plain one), page, partition
CASES = [
    ((1, 8, 2, 128), "f16", [1000], 16, 128),              # 8 partitions, the last partial
    ((1, 8, 2, 128), "f16", [640], 32, 128),               # 5: the last workgroup holds one
    ((2, 16, 2, 64), "i8", [700, 700], 64, 256),           # GQA 8, head_dim 64, 3 partitions
    ((3, 8, 4, 128), "i8", [513, 513, 513], 16, 128),      # one token in the fifth partition
    ((2, 32, 8, 128), "f16", [4096, 4096], 16, 512),       # c2's shape, two sequences
    ((1, 4, 4, 128), "f16", [300], 128, 128),              # one query head per group, page 128
    ((2, 8, 2, 128), "f16", [256, 256], 64, 128),          # exactly two full partitions
    ((1, 8, 1, 64), "i8", [129], 16, 128),                 # the second partition holds one token
    ((2, 16, 4, 128), "i8", [2048, 2048], 64, 512),        # c3-like, int8 scales per page
]


def run_all(kvb, w, c, part):
    """(fused out, two-kernel out, part_out, part_ml) with NaN-filled outputs and workspace."""
    dev = kvb.DeviceCase(w, c)
    ws = kvb.Buffer(dev.workspace_bytes(part))
    ws.fill(0xFF)
    dev.out.fill(0xFF)
    dev.run(part, workspace=ws)
    fused = dev.output().copy()
    B, H, D = w.shape.batch, w.shape.num_heads, w.shape.head_dim
    mp = dev.max_parts(part)
    raw = ws.download(np.float32, ws.nbytes // 4)
    part_out = raw[: B * H * mp * D].reshape(B, H, mp, D).copy()
    part_ml = raw[B * H * mp * D: B * H * mp * (D + 2)].reshape(B, H, mp, 2).copy()
    dev.out.fill(0xFF)
    dev.run_split(part)
    split = dev.output().copy()
    dev.free()
    ws.free()
    return fused, split, part_out, part_ml


@pytest.fixture
def pair_mode(gpu):
    prev = gpu.set_pair_mode("auto")
    yield gpu
    gpu.set_pair_mode(prev)


@pytest.mark.parametrize("shape,kv,lens,page,part", CASES)
def test_pair_gives_the_same_bits(pair_mode, oracle, shape, kv, lens, page, part):
    kvb = pair_mode
    w = kvb.Workload(kvb.Shape(*shape), kv, lens, seed=sum(lens) + page, varied=(kv == "i8"))
    c = kvb.PagedCache(w, page, 17 * page + part, pool_factor=1.5, poison=True)
    kvb.set_pair_mode("off")
    one = run_all(kvb, w, c, part)
    kvb.set_pair_mode("always")
    two = run_all(kvb, w, c, part)
    for name, a, b in zip(("fused", "two-kernel", "part_out", "part_ml"), one, two):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), name
    assert np.array_equal(one[0].view(np.uint32), one[1].view(np.uint32))
    err = pb.check_output(kvb, oracle, w, c, two[0])
    progress(f"[pair] {shape} {kv} len {lens[0]} page {page} part {part}: same bits, max err {err:.3g}")


def test_pair_mode_setting(gpu):
    prev = gpu.set_pair_mode("off")
    try:
        assert gpu.set_pair_mode("always") == "off"
        assert gpu.set_pair_mode("auto") == "always"
        assert gpu.hip.kvb_set_pair_mode(7) == -1
        assert gpu.set_pair_mode("auto") == "auto"
    finally:
        gpu.set_pair_mode(prev)


def test_c2_runs_paired_with_the_same_bits(pair_mode):
    """c2 at full size: the automatic choice (two partitions per workgroup: 512 single-partition
    workgroups on 256 CUs) against one partition per workgroup."""
    kvb = pair_mode
    w, c, cfg = kvb.make_config("c2", threads=pb.THREADS)
    part = kvb.config_part(cfg, w)
    auto = run_all(kvb, w, c, part)
    kvb.set_pair_mode("off")
    off = run_all(kvb, w, c, part)
    for name, a, b in zip(("fused", "two-kernel", "part_out", "part_ml"), auto, off):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), name
