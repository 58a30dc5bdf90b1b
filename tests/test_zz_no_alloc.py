"""kvb_run_paged_noalloc: kvb_run_paged's decode step with the split-K workspace and the fused-merge
counters in the library's static device scratch (no allocation, no events, no wait). It runs the
same kernels in the same order as kvb_run_paged, so its output must be the same bits: checked on
two calls in a row, the second with a smaller input, then the first again. Its refusals are host
checks and run no GPU work."""
import ctypes

import numpy as np
import pytest

from conftest import progress

pytestmark = pytest.mark.gpu


def noalloc(kvb, dev, part):
    a = dev.args(part)
    kvb.check(kvb.hip.kvb_run_paged_noalloc(ctypes.byref(a)), "run_paged_noalloc")
    kvb.synchronize()


def test_noalloc_matches_run_paged(gpu):
    kvb = gpu
    cases = [
        # GQA 8, c4's shape at a quarter of its length: 4 partitions per sequence, fused merge
        (kvb.Shape(4, 64, 8, 128), "f16", [8192] * 4, 128, 2048),
        # smaller: int8, ragged (longest-first order), an empty sequence
        (kvb.Shape(3, 32, 8, 128), "i8", [3000, 17, 0], 64, 512),
    ]
    devs = []
    for shape, kv, lens, page, part in cases:
        w = kvb.Workload(shape, kv, lens, seed=5, q_amp=2.0, varied=(kv == "i8"))
        dev = kvb.DeviceCase(w, kvb.PagedCache(w, page, 11, pool_factor=1.5))
        dev.out.fill(0xFF)
        dev.run(part)
        devs.append((dev, part, dev.output()))
    try:
        for i in (0, 1, 0):
            dev, part, want = devs[i]
            progress(f"[noalloc] case {i}: B={dev.w.shape.batch} {kvb.KV_NAMES[dev.w.kv_type]} part {part}")
            dev.out.fill(0xFF)
            noalloc(kvb, dev, part)
            got = dev.output()
            assert np.array_equal(got, want), f"case {i}: max diff {np.nanmax(np.abs(got - want))}"
    finally:
        for dev, _, _ in devs:
            dev.free()


def test_noalloc_refusals(gpu):
    """Sizes past the scratch and a caller workspace are refused before any GPU work, and the output
    is left as it was."""
    kvb = gpu
    w = kvb.Workload(kvb.Shape(2, 8, 2, 64), "f16", [100, 40], seed=2)
    dev = kvb.DeviceCase(w, kvb.PagedCache(w, 16, 3))
    try:
        dev.out.fill(0x7F)
        before = dev.output()
        ws = kvb.Buffer(dev.workspace_bytes(16))
        a = dev.args(16, workspace=ws)
        assert kvb.hip.kvb_run_paged_noalloc(ctypes.byref(a)) == kvb.KVB_EINVAL
        assert b"no workspace" in kvb.hip.kvb_last_error()
        ws.free()
        a = dev.args(16)
        a.max_len = 64000  # 4000 partitions of 16: 2 x 8 x 4000 slots x 264 B, past the scratch's 16 MiB
        assert kvb.hip.kvb_run_paged_noalloc(ctypes.byref(a)) == kvb.KVB_EINVAL
        assert b"KVB_NOALLOC_WORKSPACE_BYTES" in kvb.hip.kvb_last_error()
        assert np.array_equal(dev.output(), before, equal_nan=True)
    finally:
        dev.free()
    # more (sequence, head) pairs than the scratch has counters: 130 x 128 = 16640 > 16384, with a
    # workspace (one partition each) well inside the scratch
    w = kvb.Workload(kvb.Shape(130, 128, 16, 64), "f16", [1] * 130, seed=4)
    dev = kvb.DeviceCase(w, kvb.PagedCache(w, 16, 5))
    try:
        assert dev.workspace_bytes(16) < (16 << 20)
        dev.out.fill(0x7F)
        before = dev.output()
        a = dev.args(16)
        assert kvb.hip.kvb_run_paged_noalloc(ctypes.byref(a)) == kvb.KVB_EINVAL
        err = kvb.hip.kvb_last_error()
        assert b"KVB_NOALLOC_MAX_GROUPS" in err and b"16640" in err, err
        assert np.array_equal(dev.output(), before, equal_nan=True)
    finally:
        dev.free()
