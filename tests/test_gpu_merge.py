"""Where a decode step merges its partitions (kvb_set_merge_mode): fused into paged_decode, or
paged_reduce as a second kernel. Through kvb_run_paged, every setting gives the same bits, for
partition counts from 2 to 64, and the output is within the oracle's bound."""
import numpy as np
import pytest

import parity_battery as pb
from conftest import progress

pytestmark = pytest.mark.gpu

# (B, H, Hkv, D), storage, lengths, page, partition
CASES = [
    ((2, 32, 8, 128), "f16", [8192, 3001], 32, 128),      # 64 and 24 partitions
    ((2, 32, 8, 128), "i8", [8192, 8192], 16, 256),       # 32 each, the plain grid
    ((2, 32, 8, 128), "f32", [4096, 1000], 16, 128),      # 32 and 8
    ((2, 16, 2, 64), "i8", [4096, 2049], 16, 64),         # 64 and 33, head_dim 64, GQA 8
    ((3, 8, 4, 128), "f16", [700, 700, 700], 16, 128),    # 6 each
    ((4, 32, 8, 128), "f16", [5000, 0, 17, 3000], 64, 256),  # ragged, with an empty sequence
]


@pytest.fixture
def merge_mode(gpu):
    prev = gpu.set_merge_mode("auto")
    yield gpu
    gpu.set_merge_mode(prev)


@pytest.mark.parametrize("shape,kv,lens,page,part", CASES)
def test_merge_modes_give_the_same_bits(merge_mode, oracle, shape, kv, lens, page, part):
    kvb = merge_mode
    w = kvb.Workload(kvb.Shape(*shape), kv, lens, seed=sum(lens) + page, varied=(kv == "i8"))
    c = kvb.PagedCache(w, page, 13 * page + part, pool_factor=1.5, poison=True)
    dev = kvb.DeviceCase(w, c)
    outs = {}
    for mode in ("fused", "separate", "auto"):
        kvb.set_merge_mode(mode)
        dev.out.fill(0xFF)
        dev.run(part)
        outs[mode] = dev.output().copy()
    dev.free()
    for mode in ("separate", "auto"):
        assert np.array_equal(outs["fused"].view(np.uint32), outs[mode].view(np.uint32)), mode
    err = pb.check_output(kvb, oracle, w, c, outs["fused"])
    progress(f"[merge] {shape} {kv} lens {lens} page {page} part {part}: same bits, max err {err:.3g}")


def test_merge_mode_setting(gpu):
    prev = gpu.set_merge_mode("fused")
    try:
        assert gpu.set_merge_mode("separate") == "fused"
        assert gpu.set_merge_mode("auto") == "separate"
        assert gpu.hip.kvb_set_merge_mode(7) == -1
        assert gpu.set_merge_mode("auto") == "auto"
        with pytest.raises(KeyError):
            gpu.set_merge_mode("sometimes")
    finally:
        gpu.set_merge_mode(prev)
