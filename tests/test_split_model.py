"""The oracle's CPU model of the split-K decode kernel (kvbo_split_decode) through the parity
battery that the GPU kernels pass (parity_battery.py), on the CPU.

The model is where the mutation harness (tests/mutation/mutate.py) plants the reference's kernel
mistakes, since no deliberately broken kernel runs on a GPU. Unmutated, it must pass every check
here; each planted mistake must fail at least one. Full-size configurations, the fused-merge and
timing checks are GPU-only and are not part of this battery."""
import numpy as np
import pytest

import parity_battery as pb


@pytest.fixture(scope="module")
def model(oracle):
    def run_ws(w, c, part):
        return oracle.split_decode(w.shape, c.page_size, c.table, w.lens, w.max_len, w.q, c.k, c.v,
                                   c.k_scale, c.v_scale, part_tokens=part, threads=8)

    def run(w, c, part, share_kv):
        # share_kv picks how many query heads a workgroup serves; per head the arithmetic is the same
        return run_ws(w, c, part)[0]

    return run, run_ws


@pytest.mark.parametrize("path", pb.GOLDEN, ids=[p.rsplit("/", 1)[-1] for p in pb.GOLDEN])
def test_golden(kvb, oracle, model, path):
    pb.check_golden(kvb, oracle, model[0], path)


@pytest.mark.parametrize("kv", ["f32", "f16", "i8"])
@pytest.mark.parametrize("page,part", pb.DOMINANT_LAYOUTS)
def test_dominant_key_gather_is_exact(kvb, model, kv, page, part):
    pb.check_dominant_key(kvb, model[0], kv, page, part)


def test_workspace_partition_indexing(kvb, oracle, model):
    pb.check_workspace_partitions(kvb, oracle, model[1])


@pytest.mark.parametrize("kv", ["f32", "f16", "i8"])
def test_ragged_any_page_and_partition(kvb, oracle, model, kv):
    pb.check_ragged(kvb, oracle, model[0], kv)


@pytest.mark.parametrize("shape", pb.GQA_SHAPES)
def test_gqa_groups(kvb, oracle, model, shape):
    pb.check_gqa(kvb, oracle, model[0], shape)


@pytest.mark.parametrize("kv", ["f32", "f16", "i8"])
def test_huge_and_tiny_queries(kvb, oracle, model, kv):
    pb.check_huge_and_tiny_queries(kvb, oracle, model[0], kv)


@pytest.mark.parametrize("kv", ["f16", "i8"])
def test_huge_and_tiny_values(kvb, oracle, model, kv):
    pb.check_huge_and_tiny_values(kvb, oracle, model[0], kv)


def test_storage_bounds_c2_f16(kvb, oracle, model):
    pb.check_storage_bound_f16(kvb, oracle, model[0])


def test_storage_bounds_c3_i8(kvb, oracle, model):
    pb.check_storage_bound_i8(kvb, oracle, model[0])


@pytest.mark.parametrize("kv,part", pb.MANY_PARTITIONS)
def test_many_partitions(kvb, oracle, model, kv, part):
    pb.check_many_partitions(kvb, oracle, model[0], kv, part)


def test_model_refuses_bad_arguments(kvb, oracle):
    w = kvb.Workload(kvb.Shape(1, 4, 2, 64), "f32", [10], seed=1)
    c = kvb.PagedCache(w, 16, 1, poison=False)
    with pytest.raises(ValueError):
        oracle.split_decode(w.shape, c.page_size, c.table, w.lens, w.max_len, w.q, c.k, c.v, waves=9)
    qc = kvb.PagedCache(kvb.Workload(kvb.Shape(1, 4, 2, 64), "i8", [10], seed=1), 16, 1, poison=False)
    with pytest.raises(ValueError):  # int8 without scales
        oracle.split_decode(w.shape, 16, qc.table, w.lens, w.max_len, w.q, qc.k, qc.v)
    out, part_out, part_ml = oracle.split_decode(w.shape, 16, c.table, w.lens, w.max_len, w.q, c.k, c.v)
    assert part_out.shape == (1, 4, 1, 64) and np.isfinite(out).all()


@pytest.mark.parametrize("kv", ["f32", "f16", "i8"])
def test_device_lengths_that_disagree_stay_in_bounds(kvb, oracle, kv):
    """The kernels' length clamp (live_len), on the CPU model. The host sized the launch for lengths
    [40, 17] (max_len 40, part 16: 3 partitions; page 16: table rows of 3 blocks, capacity 48); the
    device copy of the lengths says otherwise. The model counts every table read outside a sequence's
    row and every merge past its partitions, and refuses (-2, a ValueError here) if there is one: so
    returning at all shows the clamp keeps them in. A negative length gives exactly 0; a length past
    the cap computes as the cap, with the row's unused (-1) entries read as zeros."""
    shape = kvb.Shape(2, 8, 2, 64)
    w = kvb.Workload(shape, kv, [40, 17], seed=3, q_amp=2.0, varied=(kv == "i8"))
    c = kvb.PagedCache(w, 16, 5, pool_factor=1.5, poison=False)

    def decode(dev_lens):
        return oracle.split_decode(shape, 16, c.table, np.array(dev_lens, np.int32), 40, w.q, c.k, c.v,
                                   c.k_scale, c.v_scale, part_tokens=16, threads=2)

    out, _, _ = decode([-5, 1000])
    assert (out[0] == 0).all()
    capped, _, _ = decode([48, 48])  # the cap itself: every table entry of both rows
    assert np.isfinite(capped).all()
    np.testing.assert_array_equal(out[1], capped[1])
    np.testing.assert_array_equal(decode([1000, 48])[0], capped)
    # agreeing lengths are untouched by the clamp: the same as the host's own lengths
    np.testing.assert_array_equal(decode([40, 17])[0], decode(w.lens)[0])
