"""The GPU cache writers (kvb_write_paged) against the host writers: scatter_to_paged for f32/f16
and quantize_to_paged_i8 for int8 (the reference's src/reference.hpp:60-68 and
src/reference.cpp:32-51, whose host restatements are pinned bit for bit against the reference's
own code in the oracle tests). Every byte of the pool and every scale must come out as the host
writes them: live rows written, everything else left as it was."""
import ctypes

import numpy as np
import pytest

from conftest import progress

pytestmark = pytest.mark.gpu


def _bytes(a):
    return np.ascontiguousarray(a).view(np.uint8)


def _elems(a):
    """The array as unsigned integers of its element size (bitwise, NaNs included)."""
    a = np.ascontiguousarray(a)
    return a.view({1: np.uint8, 2: np.uint16, 4: np.uint32}[a.dtype.itemsize])


def check_writer(kvb, w, page, seed, pool_factor):
    want = kvb.PagedCache(w, page, seed, pool_factor=pool_factor, poison=True)
    plain = kvb.PagedCache(w, page, seed, pool_factor=pool_factor, poison=False)
    table = kvb.Buffer.from_array(want.table)
    lens = kvb.Buffer.from_array(w.lens)
    total = 0.0
    for src, pool_want, pool_plain, sc_want, sc_plain in (
            (w.k, want.k, plain.k, want.k_scale, plain.k_scale),
            (w.v, want.v, plain.v, want.v_scale, plain.v_scale)):
        # the pool before the write: the host result, with every live element (equal in the poisoned
        # and the plain pool) overwritten
        before = _elems(pool_want).copy()
        live = before == _elems(pool_plain)
        before[live] = 0x5A5A5A5A & np.iinfo(before.dtype).max
        contig = kvb.Buffer.from_array(src)
        paged = kvb.Buffer.from_array(before)
        scales = None
        if sc_want is not None:
            sc_before = _elems(sc_want).copy()
            sc_before[sc_before == _elems(sc_plain)] = 0x5A5A5A5A
            scales = kvb.Buffer.from_array(sc_before)
        total += kvb.write_paged(w, want, contig, paged, table, lens, scales)
        got = paged.download(before.dtype, before.size)
        bad = np.flatnonzero(got != _elems(pool_want).ravel())
        assert bad.size == 0, f"{bad.size} pool elements differ, first at {bad[:4]} (live: {live.ravel()[bad[:4]]})"
        if scales is not None:
            got_s = scales.download(np.uint32, sc_before.size)
            assert np.array_equal(got_s, _elems(sc_want).ravel()), "scales"
            scales.free()
        contig.free()
        paged.free()
    table.free()
    lens.free()
    return total, want


@pytest.mark.parametrize("kv", ["f32", "f16", "i8"])
@pytest.mark.parametrize("page", [1, 3, 16, 64])
def test_writer_matches_host_bytes(gpu, kv, page):
    kvb = gpu
    lens = [0, 1, 15, 16, 17, 63, 64, 65, 129, 300, 2, 0]
    w = kvb.Workload(kvb.Shape(len(lens), 8, 2, 64), kv, lens, seed=41, varied=(kv == "i8"))
    check_writer(kvb, w, page, page * 5 + 1, 2.0)


@pytest.mark.parametrize("kv", ["f16", "i8"])
def test_writer_c5_shape(gpu, kv):
    """BASELINE c5's ragged batch (page 64, 3x pool, N(0,1)): the GPU-written pool and scales are the
    host's, byte for byte."""
    kvb = gpu
    lens = kvb.c5_lengths()
    w = kvb.Workload(kvb.Shape(len(lens), 32, 8, 128), kv, lens, seed=16384, q_amp=1.0, dist="normal", threads=16)
    ms, _ = check_writer(kvb, w, 64, 16384 * 131 + 64, 3.0)
    progress(f"[writer] c5 {kv}: K+V written in {ms * 1e3:.1f} us "
             f"({w.min_bytes() / (ms * 1e-3) / 1e9:.0f} GB/s of cache bytes)")


def test_writer_refusals_leave_the_pool(gpu):
    kvb = gpu
    w = kvb.Workload(kvb.Shape(2, 8, 2, 64), "i8", [32, 40], seed=3)
    c = kvb.PagedCache(w, 16, 1, poison=False)
    contig = kvb.Buffer.from_array(w.k)
    paged = kvb.Buffer(c.k.nbytes)
    paged.fill(0x33)
    table, lens = kvb.Buffer.from_array(c.table), kvb.Buffer.from_array(w.lens)
    with pytest.raises(kvb.KvbInvalidArgument):
        kvb.write_paged(w, c, contig, paged, table, lens, None)  # int8 without scales
    assert (paged.download(np.uint8, c.k.nbytes) == 0x33).all()
    for b in (contig, paged, table, lens):
        b.free()
