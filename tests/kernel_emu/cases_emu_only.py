"""Cases for the CPU emulation of the kernels only (tests/kernel_emu/run_gpu_tests.py runs them with
the GPU test files; on a GPU they skip).

Device lengths that disagree with the host's. The host checks its copy of the lengths and sizes the
launch from it; the kernels read the device copy and clamp it to what the launch holds (live_len in
kv-cache-bench_amd/csrc/kvb_kernels.hpp). These cases hand the kernels lengths the host did not check:
negative, past the table rows, past max_len. That is nothing to run on a GPU on purpose. The emulation
checks every buffer access against its allocation and, in the AddressSanitizer build
(run_gpu_tests.py --asan), every plain load and store too, so a run that returns at all has kept
every access inside the buffers. On top of that:
- a sequence whose device length is 0 or negative gets exactly 0 (plain grid);
- the step after a disagreeing one, with the lengths agreeing again, gives the bits of a fresh run:
  no merge counter was left short (a ragged launch whose device lengths make a different number of
  work items than the host counted does nothing at all).
Reference: the reference's kernel reads seq_lens as given (src/kernels.metal:44-47) and its host
refuses lengths past the capacity (src/metal_attn.mm:107-117); the output for lengths that disagree
is unspecified in both.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

DEVICE_LENS = [(-5, 1000), (1000, -5), (48, 48), (0, 0), (1000, 1000), (2**31 - 1, -(2**31))]


@pytest.fixture(scope="module")
def emu(gpu):
    if "CPU emulation" not in gpu.device_name():
        pytest.skip("emulation only: these cases hand the kernels lengths the host did not check")
    return gpu


@pytest.mark.parametrize("kv", ["f32", "f16", "i8"])
@pytest.mark.parametrize("page,part", [(16, 16), (16, 64), (32, 32), (3, 7), (1, 8)])
@pytest.mark.parametrize("host_lens", [(40, 17), (40, 40)], ids=["ragged", "plain"])
def test_device_lengths_that_disagree_stay_in_bounds(emu, kv, page, part, host_lens):
    kvb = emu
    shape = kvb.Shape(2, 8, 2, 64)
    w = kvb.Workload(shape, kv, list(host_lens), seed=3, q_amp=2.0, varied=(kv == "i8"))
    c = kvb.PagedCache(w, page, 5, pool_factor=1.5, poison=True)
    dev = kvb.DeviceCase(w, c)
    try:
        dev.out.fill(0xFF)
        dev.run(part)
        fresh = dev.output()
        for lens in DEVICE_LENS:
            dev.lens.upload(np.array(lens, np.int32))
            dev.out.fill(0xFF)
            dev.run(part)  # returns only if every access stayed inside the buffers
            got = dev.output()
            if host_lens[0] == host_lens[1]:  # the plain grid: a non-positive length gives exactly 0
                for b, L in enumerate(lens):
                    if L <= 0:
                        assert not got[b].any(), (lens, b)
            dev.lens.upload(np.asarray(w.lens, np.int32))
            dev.out.fill(0xFF)
            dev.run(part)
            np.testing.assert_array_equal(dev.output(), fresh, err_msg=f"the step after device lengths {lens}")
    finally:
        dev.free()


@pytest.mark.parametrize("kv", ["f16", "i8"])
def test_graph_replay_with_device_lengths_that_disagree(emu, kv):
    """A captured graph keeps the grid and the work order that the host's lengths gave at capture.
    Ragged (lengths not all equal): device lengths that make a different number of work items turn
    every replay into a no-op (the output keeps what it held), and the replay after the lengths agree
    again gives the bits of a fresh step. Plain (equal lengths at capture): shorter device lengths are
    clamped and served like an eager step with the same device lengths."""
    kvb = emu
    part = 16
    for host_lens, dev_lens in (((40, 17), (40, 40)), ((40, 40), (17, 40))):
        w = kvb.Workload(kvb.Shape(2, 8, 2, 64), kv, list(host_lens), seed=7, q_amp=2.0, varied=(kv == "i8"))
        dev = kvb.DeviceCase(w, kvb.PagedCache(w, 16, 9, pool_factor=1.5, poison=True))
        graph = None
        try:
            dev.out.fill(0xFF)
            dev.run(part)
            fresh = dev.output()
            graph = dev.capture_graph(part, 1)
            dev.out.fill(0xFF)
            graph.launch()
            np.testing.assert_array_equal(dev.output(), fresh)
            dev.lens.upload(np.array(dev_lens, np.int32))
            if host_lens[0] != host_lens[1]:
                dev.out.fill(0x7F)
                before = dev.output()
                graph.launch()
                np.testing.assert_array_equal(dev.output(), before, err_msg="a disagreeing ragged replay wrote")
            else:
                dev.out.fill(0xFF)
                dev.run(part)
                eager = dev.output()
                dev.out.fill(0xFF)
                graph.launch()
                np.testing.assert_array_equal(dev.output(), eager)
                assert not np.array_equal(eager[0], fresh[0])
            dev.lens.upload(np.asarray(w.lens, np.int32))
            dev.out.fill(0xFF)
            graph.launch()
            np.testing.assert_array_equal(dev.output(), fresh, err_msg="the replay after the lengths agree again")
        finally:
            if graph is not None:
                graph.free()
            dev.free()
