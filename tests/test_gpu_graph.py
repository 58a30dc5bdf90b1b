"""Decode steps captured into a HIP graph (kvb_graph_capture_paged): every replay gives the eager
step's bits, with the program's own eager work and synchronisations between the replays, for the
fused step, the ragged order, two partitions per workgroup and the two-kernel form; and the
refusals, which run no GPU work."""
import ctypes

import numpy as np
import pytest

from conftest import progress

pytestmark = pytest.mark.gpu


def cases(kvb):
    return [
        # fused merge, GQA 8, four partitions per sequence
        (kvb.Shape(4, 64, 8, 128), "f16", [8192] * 4, 128, 2048),
        # int8, ragged (longest-first order), an empty sequence
        (kvb.Shape(3, 32, 8, 128), "i8", [3000, 17, 0], 64, 512),
        # two partitions per workgroup (512 single-partition workgroups on 256 CUs)
        (kvb.Shape(8, 32, 8, 128), "f16", [4096] * 8, 16, 512),
        # 563 partitions x 4 query heads: more (m, l) pairs than the fused merge stages, so each
        # captured step is paged_decode then paged_reduce
        (kvb.Shape(1, 8, 2, 64), "f16", [9000], 16, 16),
    ]


def make(kvb, shape, kv, lens, page, part):
    w = kvb.Workload(shape, kv, lens, seed=sum(lens) % 997, q_amp=2.0, varied=(kv == "i8"))
    return kvb.DeviceCase(w, kvb.PagedCache(w, page, 13, pool_factor=1.5))


def test_graph_replays_match_eager(gpu):
    kvb = gpu
    all_cases = cases(kvb)
    devs = []
    try:
        for shape, kv, lens, page, part in all_cases:
            dev = make(kvb, shape, kv, lens, page, part)
            dev.out.fill(0xFF)
            dev.run(part)
            devs.append((dev, part, dev.output()))
        for i, (dev, part, want) in enumerate(devs):
            progress(f"[graph] case {i}: B={dev.w.shape.batch} {kvb.KV_NAMES[dev.w.kv_type]} part {part}")
            graph = dev.capture_graph(part, steps=3)
            try:
                for rep in range(4):
                    dev.out.fill(0xFF)  # an eager fill kernel between the replays
                    if rep == 2:  # and another case's eager step, waited for
                        other, opart, owant = devs[(i + 1) % len(devs)]
                        other.out.fill(0xFF)
                        other.run(opart)
                        assert np.array_equal(other.output(), owant)
                    ms = graph.launch()
                    kvb.synchronize()
                    assert ms > 0.0
                    got = dev.output()
                    assert np.array_equal(got, want), f"case {i} replay {rep}: max diff {np.nanmax(np.abs(got - want))}"
            finally:
                graph.free()
    finally:
        for dev, _, _ in devs:
            dev.free()


def test_graph_refusals(gpu):
    kvb = gpu
    dev = make(kvb, kvb.Shape(2, 8, 2, 64), "f16", [100, 40], 16, 16)
    try:
        h = ctypes.c_void_p()
        a = dev.args(16)
        assert kvb.hip.kvb_graph_capture_paged(ctypes.byref(a), 0, ctypes.byref(h)) == kvb.KVB_EINVAL
        assert not h.value
        ws = kvb.Buffer(dev.workspace_bytes(16))
        a = dev.args(16, workspace=ws)
        assert kvb.hip.kvb_graph_capture_paged(ctypes.byref(a), 1, ctypes.byref(h)) == kvb.KVB_EINVAL
        assert b"owns its own" in kvb.hip.kvb_last_error()
        ws.free()
        a = dev.args(16)
        a.max_len = 30  # shorter than a sequence: the same refusal as kvb_run_paged
        assert kvb.hip.kvb_graph_capture_paged(ctypes.byref(a), 1, ctypes.byref(h)) == kvb.KVB_EINVAL
        ms = ctypes.c_double()
        assert kvb.hip.kvb_graph_launch(None, ctypes.byref(ms)) == kvb.KVB_EINVAL
        assert kvb.hip.kvb_graph_destroy(None) == kvb.KVB_OK
    finally:
        dev.free()
