"""The host layer (libkvb_host.so: generator, layout, scatter, int8 quantiser, poison) against the
oracle bit for bit, and the C ABI's refusals, which happen before any GPU work (no GPU needed)."""
import ctypes

import numpy as np
import pytest


def test_layout_equals_oracle(kvb, oracle):
    lens = [0, 1, 63, 64, 65, 2047, 2048, 2049, 300]
    w = kvb.Workload(kvb.Shape(1, 4, 2, 64), "f32", lens, seed=1)
    for page in (1, 3, 16, 64, 128):
        for pool in (1.0, 1.25, 1.5, 2.0, 3.0):
            for seed in (0, 5, 2 ** 63 + 11):
                c = kvb.PagedCache(w, page, seed, pool_factor=pool, poison=False)
                want = oracle.make_paged_layout(lens, page, seed, pool)
                assert np.array_equal(c.table, want)
                assert c.num_blocks == oracle.layout_dims(lens, page, pool)[2]


@pytest.mark.parametrize("kv", ["f32", "f16", "i8"])
def test_paged_cache_equals_oracle(kvb, oracle, kv):
    lens = [37, 0, 70, 16]
    w = kvb.Workload(kvb.Shape(1, 8, 2, 64), kv, lens, seed=3, varied=(kv == "i8"))
    c = kvb.PagedCache(w, 16, 77, pool_factor=2.0, poison=False)
    if kv == "i8":
        for src, pool, sc in ((w.k, c.k, c.k_scale), (w.v, c.v, c.v_scale)):
            op, osc = oracle.quantize(w.shape, 16, c.table, lens, w.max_len, src, c.num_blocks)
            assert np.array_equal(op, pool) and np.array_equal(osc.view(np.uint32), sc.view(np.uint32))
        kd, vd = c.dequantized(w)
        assert np.array_equal(kd, oracle.dequantize(w.shape, 16, c.table, lens, w.max_len, c.k, c.k_scale))
    else:
        for src, pool in ((w.k, c.k), (w.v, c.v)):
            assert np.array_equal(oracle.scatter(w.shape, 16, c.table, lens, w.max_len, src, c.num_blocks).view(np.uint8),
                                  pool.view(np.uint8))


def test_f16_workload_is_rne_of_f32(kvb):
    w = kvb.Workload(kvb.Shape(1, 8, 2, 128), "f16", [300, 41], seed=9, keep_f32=True, dist="normal")
    assert np.array_equal(w.k32.astype(np.float16).view(np.uint16), w.k.view(np.uint16))
    assert np.array_equal(w.v32.astype(np.float16).view(np.uint16), w.v.view(np.uint16))


def test_workload_deterministic_and_distributions(kvb):
    a = kvb.Workload(kvb.Shape(1, 8, 2, 128), "f32", [1000, 5], seed=4, threads=1)
    b = kvb.Workload(kvb.Shape(1, 8, 2, 128), "f32", [1000, 5], seed=4, threads=7)
    assert np.array_equal(a.k, b.k) and np.array_equal(a.v, b.v) and np.array_equal(a.q, b.q)
    assert np.abs(a.k).max() < 1 and abs(a.k[0].mean()) < 0.01 and not a.k[1, :, 5:].any()
    n = kvb.Workload(kvb.Shape(1, 8, 2, 128), "f32", [4000], seed=4, q_amp=1.0, dist="normal")
    live = n.k[0].ravel()
    assert abs(live.mean()) < 0.01 and abs(live.std() - 1) < 0.01 and abs(n.q.std() - 1) < 0.1
    assert 0 < np.abs(n.k - kvb.Workload(kvb.Shape(1, 8, 2, 128), "f32", [4000], seed=5, dist="normal").k).max()


def test_poison_marks_every_unowned_element(kvb):
    lens = [1, 16, 17, 100, 0]
    for kv, bad in (("f32", np.isnan), ("f16", np.isnan), ("i8", lambda x: x == -128)):
        w = kvb.Workload(kvb.Shape(1, 4, 2, 64), kv, lens, seed=2)
        c = kvb.PagedCache(w, 16, 9, pool_factor=3.0, poison=True)
        owned = np.zeros(c.k.shape[:3], bool)  # [block][kvh][row]
        for b, ln in enumerate(lens):
            for t in range(ln):
                owned[c.table[b, t // 16], :, t % 16] = True
        marked = bad(c.k).all(axis=-1)
        assert np.array_equal(marked, ~owned), kv
        if kv == "i8":
            used = set(c.table[c.table >= 0].tolist())
            for blk in range(c.num_blocks):
                assert np.isnan(c.k_scale[blk]).all() == (blk not in used)


def test_mi355x_partition_policy(kvb):
    # c4 (B 4, 64/8 heads, 32k): 4 * 8 workgroups per partition -> 256 at part 4096
    assert kvb.mi355x_part_tokens(kvb.Shape(4, 64, 8, 128), 32768) == 4096
    assert kvb.mi355x_part_tokens(kvb.Shape(4, 64, 8, 128), 32768, min_groups=kvb.mi355x_min_groups(kvb.KV_I8)) == 4096
    # int8 at head_dim 64 (64-byte rows) asks for two workgroups per CU
    assert [kvb.mi355x_min_groups(t, d) for t in (kvb.KV_F32, kvb.KV_F16, kvb.KV_I8) for d in (64, 128)] == \
        [256, 256, 256, 256, 512, 256]
    assert kvb.mi355x_part_tokens(kvb.Shape(4, 64, 8, 64), 32768, min_groups=kvb.mi355x_min_groups(kvb.KV_I8, 64)) == 2048
    assert kvb.mi355x_part_tokens(kvb.Shape(4, 64, 8, 128), 32768, min_groups=512) == 2048
    assert kvb.mi355x_part_tokens(kvb.Shape(4, 64, 8, 128), 32768, min_groups=1024) == 1024
    # short or small: the floor
    assert kvb.mi355x_part_tokens(kvb.Shape(1, 32, 8, 128), 512) == 256
    # c3 (B 16, 32/8 heads, 8k): 16 * 8 workgroups per partition
    assert kvb.mi355x_part_tokens(kvb.Shape(16, 32, 8, 128), 8192) == 4096
    assert kvb.mi355x_part_tokens(kvb.Shape(16, 32, 8, 128), 8192, min_groups=512) == 2048
    # a ragged batch (lengths not all equal) caps the partition at 2048 while its longest sequence is
    # under 2 x 3584 tokens, 4096 from 7 x 4096, 3584 between: c5's lengths -> 3584; c4's equal
    # lengths keep 4096; the cap yields to a larger min_part; an all-empty batch gets the floor
    c5 = kvb.Shape(72, 32, 8, 128)
    assert max(kvb.c5_lengths()) >= 2 * 3584
    assert kvb.mi355x_part_tokens_for(c5, kvb.c5_lengths()) == 3584
    assert kvb.mi355x_part_tokens_for(c5, kvb.c5_lengths(), min_part=4096) == 4096
    s64 = kvb.Shape(64, 32, 8, 128)
    for longest, cap in ((4096, 2048), (7167, 2048), (7168, 3584), (28671, 3584), (28672, 4096), (65536, 4096)):
        lens = [100] * 63 + [longest]
        assert kvb.mi355x_part_tokens_for(s64, lens) == cap, (longest, cap)
    assert kvb.mi355x_part_tokens_for(kvb.Shape(4, 64, 8, 128), [32768] * 4) == 4096
    assert kvb.mi355x_part_tokens_for(kvb.Shape(2, 64, 8, 128), [32768, 100]) == 2048
    assert kvb.mi355x_part_tokens_for(kvb.Shape(3, 8, 2, 64), [0, 0, 0]) == 256
    assert kvb.mi355x_part_tokens_for(c5, kvb.c5_lengths(), max_part=1024) == 1024
    assert kvb.host.kvbh_mi355x_part_tokens_lens(2, 8, 2, 64, None, 256, 256, 4096) == -1
    # BASELINE names c1's and c2's partitions; the policy is used where it leaves the choice
    assert kvb.CONFIGS["c1"]["part"] == 128 and kvb.CONFIGS["c2"]["part"] == 512
    assert all(kvb.CONFIGS[n]["part"] == "mi355x" for n in ("c3", "c4", "c5f16", "c5i8"))


# The ragged batches the cap was measured on (32 q / 8 KV heads, head_dim 128, page 64): B lengths
# ~U[1, L] drawn with numpy's default_rng, three from seed 5 and three from seed 11 in this order,
# with each batch's longest sequence and token count as drawn, and the partition that ran fastest of
# 2048 / 3584 / 4096 on MI355X (fp16 and int8 agree; 128 x U[1, 8192] is the one batch where the
# cap's 3584 is not the fastest: 4096 was 1.1% faster in fp16).
RAGGED_BATCHES = (
    (5, ((64, 4096, 4093, 127111, 2048), (64, 8192, 8032, 260108, 3584), (64, 32768, 32496, 1089010, 4096))),
    (11, ((32, 16384, 16295, 269525, 3584), (128, 8192, 8163, 520274, 3584), (16, 65536, 65478, 615616, 4096))),
)


def test_ragged_cap_on_the_measured_batches(kvb):
    for seed, batches in RAGGED_BATCHES:
        rng = np.random.default_rng(seed)
        for B, L, longest, tokens, want in batches:
            lens = [int(x) for x in rng.integers(1, L + 1, size=B)]
            assert (max(lens), sum(lens)) == (longest, tokens), (seed, B, L)  # the same draw as measured
            assert kvb.mi355x_part_tokens_for(kvb.Shape(B, 32, 8, 128), lens) == want, (B, L)


class TestRefusals:
    """kvb_check_paged / kvb_run_paged refuse what the reference's run_paged refuses
    (src/metal_attn.mm:72-73, 107-117, 199-201), with no GPU involved."""

    def args(self, kvb, **kw):
        a = kvb.PagedArgsC()
        a.batch, a.num_heads, a.num_kv_heads, a.head_dim = 2, 8, 2, 128
        a.kv_type, a.page_size, a.max_blocks, a.max_len, a.part_tokens, a.share_kv = kvb.KV_F32, 16, 2, 32, 16, 1
        self.lens = np.array(kw.pop("lens", [32, 32]), np.int32)
        a.host_seq_lens = self.lens.ctypes.data
        for name in ("q", "k", "v", "block_table", "seq_lens", "out"):
            setattr(a, name, 0x1000)
        for k, v in kw.items():
            setattr(a, k, v)
        return a

    def status(self, kvb, a):
        return kvb.hip.kvb_check_paged(ctypes.byref(a))

    def test_valid_passes(self, kvb):
        assert self.status(kvb, self.args(kvb)) == kvb.KVB_OK
        assert self.status(kvb, self.args(kvb, lens=[0, 0], max_len=0)) == kvb.KVB_OK

    @pytest.mark.parametrize("kw", [dict(lens=[33, 33], max_len=64), dict(lens=[32, 33], max_len=64),
                                    dict(lens=[33, 33]), dict(lens=[32, 32], max_len=31), dict(lens=[-1, 32]),
                                    dict(max_len=-1), dict(page_size=0), dict(part_tokens=-1), dict(head_dim=96),
                                    dict(num_heads=6, num_kv_heads=4), dict(kv_type=2), dict(kv_type=7),
                                    dict(max_blocks=-1), dict(host_seq_lens=None), dict(q=None), dict(out=None),
                                    dict(workspace=0x1000, workspace_bytes=16),
                                    # launch-grid limits (y = batch, z = partitions <= 65535)
                                    dict(part_tokens=1, max_len=70000), dict(lens=[0] * 65536, batch=65536)])
    def test_refused(self, kvb, kw):
        a = self.args(kvb, **kw)
        assert self.status(kvb, a) == kvb.KVB_EINVAL, kvb.hip.kvb_last_error()
        ms = ctypes.c_double(-1)
        assert kvb.hip.kvb_run_paged(ctypes.byref(a), ctypes.byref(ms)) == kvb.KVB_EINVAL
        assert ms.value == 0.0
        ms.value = -1
        assert kvb.hip.kvb_run_paged_loads(ctypes.byref(a), ctypes.byref(ms)) == kvb.KVB_EINVAL
        assert ms.value == 0.0

    @pytest.mark.parametrize("kw", [dict(page_size=8, max_blocks=4), dict(part_tokens=24)])
    def test_loads_only_needs_tile_aligned_pages(self, kvb, kw):
        """kvb_run_paged_loads measures the tile-aligned decode only: a page or partition that is
        not a multiple of 16 tokens is refused before any GPU work (kvb_run_paged accepts both)."""
        a = self.args(kvb, **kw)
        assert self.status(kvb, a) == kvb.KVB_OK
        ms = ctypes.c_double(-1)
        assert kvb.hip.kvb_run_paged_loads(ctypes.byref(a), ctypes.byref(ms)) == kvb.KVB_EINVAL
        assert b"multiples of 16" in kvb.hip.kvb_last_error()
        assert ms.value == 0.0

    def test_capacity_message_names_the_sequence(self, kvb):
        self.status(kvb, self.args(kvb, lens=[32, 33], max_len=64))
        assert b"sequence 1 has length 33" in kvb.hip.kvb_last_error()

    def test_naive_refuses_int8_and_long(self, kvb):
        a = kvb.NaiveArgsC()
        a.batch, a.num_heads, a.num_kv_heads, a.head_dim, a.kv_type, a.max_len = 2, 8, 2, 128, kvb.KV_F32, 32
        lens = np.array([32, 33], np.int32)
        a.host_seq_lens = lens.ctypes.data
        for name in ("q", "k", "v", "seq_lens", "out"):
            setattr(a, name, 0x1000)
        assert kvb.hip.kvb_check_naive(ctypes.byref(a)) == kvb.KVB_EINVAL
        lens[1] = 32
        assert kvb.hip.kvb_check_naive(ctypes.byref(a)) == kvb.KVB_OK
        a.kv_type = kvb.KV_I8
        assert kvb.hip.kvb_check_naive(ctypes.byref(a)) == kvb.KVB_EINVAL

    def test_writer_refusals(self, kvb):
        """kvb_check_write_paged: the cache writer's argument checks, before any GPU work."""
        lens = np.array([32, 20], np.int32)

        def args(**kw):
            a = kvb.CacheArgsC()
            a.batch, a.num_kv_heads, a.head_dim, a.kv_type = 2, 2, 128, kvb.KV_I8
            a.page_size, a.max_blocks, a.max_len = 16, 2, 32
            a.host_seq_lens = lens.ctypes.data
            for name in ("contig", "paged", "scales", "block_table", "seq_lens"):
                setattr(a, name, 0x1000)
            for k, v in kw.items():
                setattr(a, k, v)
            return kvb.hip.kvb_check_write_paged(ctypes.byref(a))

        assert args() == kvb.KVB_OK
        assert args(kv_type=kvb.KV_F16, scales=None) == kvb.KVB_OK
        for kw in (dict(scales=None), dict(head_dim=96), dict(page_size=0), dict(max_len=31), dict(max_blocks=1),
                   dict(kv_type=5), dict(paged=None), dict(host_seq_lens=None), dict(num_kv_heads=0)):
            assert args(**kw) == kvb.KVB_EINVAL, kw

    def test_valid_without_gpu_is_no_device(self, kvb):
        if kvb.gpu_available():
            pytest.skip("a GPU is present")
        ms = ctypes.c_double()
        assert kvb.hip.kvb_run_paged(ctypes.byref(self.args(kvb)), ctypes.byref(ms)) == kvb.KVB_ENODEV

    def test_workspace_size(self, kvb):
        a = self.args(kvb, part_tokens=0, max_len=32)
        # auto part for B 2, Hkv 2, 32 tokens is 64 -> one partition; slots 2*8*1
        assert kvb.hip.kvb_paged_max_parts(ctypes.byref(a)) == 1
        assert kvb.hip.kvb_paged_workspace_bytes(ctypes.byref(a)) == 16 * (128 * 4 + 8)
        a.part_tokens = 5
        assert kvb.hip.kvb_paged_max_parts(ctypes.byref(a)) == 7


def test_c_abi_auto_part_tokens_thresholds(kvb, oracle):
    """kvb_auto_part_tokens (the C ABI's) on the threshold table of the reference's
    tests/boundary_tests.cpp:86-92 (16 (sequence, KV head) pairs: thresholds at 32 partitions), and
    equal to the oracle's over a sweep of shapes and lengths."""
    for length, part in [(0, 64), (1, 64), (3968, 64), (3969, 128), (7936, 128), (7937, 256), (15872, 256),
                         (15873, 512), (1 << 20, 512)]:
        assert kvb.auto_part_tokens(2, 8, length) == part
    for b in (1, 2, 3, 16):
        for hkv in (1, 2, 8):
            for L in list(range(0, 5000, 37)) + [32768, 100000]:
                assert kvb.auto_part_tokens(b, hkv, L) == oracle.auto_part_tokens(b, hkv, L)


def test_heads_per_workgroup(kvb):
    """kvb_heads_per_workgroup: one workgroup reads each K/V page for this many query heads. 32 or
    16 for a group that is a multiple of 32 or 16 with an f16 or i8 cache (16-head waves: one
    workgroup of four, or two head splits), else the largest divisor of the group that is at most 8;
    1 without share_kv; -1 for shapes the decode refuses. Spot values, then every group to 64
    against a brute-force search."""
    spot = {1: 1, 2: 2, 3: 3, 4: 4, 5: 5, 6: 6, 7: 7, 8: 8, 9: 3, 10: 5, 11: 1, 12: 6, 13: 1, 14: 7, 15: 5,
            16: 8, 18: 6, 20: 5, 21: 7, 24: 8, 28: 7, 32: 8, 40: 8, 48: 8, 64: 8}
    F32, F16, I8 = kvb.KV_F32, kvb.KV_F16, kvb.KV_I8

    def wide(g, want):  # f16 and i8
        return 32 if g % 32 == 0 else 16 if g % 16 == 0 else want

    for g, want in spot.items():
        assert kvb.hip.kvb_heads_per_workgroup(g * 8, 8, F32, 1) == want, g
        assert kvb.hip.kvb_heads_per_workgroup(g * 8, 8, F16, 1) == wide(g, want), g
        assert kvb.hip.kvb_heads_per_workgroup(g * 8, 8, I8, 1) == wide(g, want), g
        for kv in (F32, F16, I8):
            assert kvb.hip.kvb_heads_per_workgroup(g * 8, 8, kv, 0) == 1
    for g in range(1, 65):
        for kv in (F32, F16, I8):
            got = kvb.hip.kvb_heads_per_workgroup(g * 2, 2, kv, 1)
            if kv != F32 and g % 16 == 0:
                assert got == (32 if g % 32 == 0 else 16), g
                continue
            assert g % got == 0 and got <= 8
            assert all(g % d != 0 for d in range(got + 1, 9)), g
    for h, hkv in ((8, 0), (0, 8), (12, 8), (-8, 8), (8, -2)):
        assert kvb.hip.kvb_heads_per_workgroup(h, hkv, F16, 1) == -1, (h, hkv)
    assert kvb.hip.kvb_heads_per_workgroup(16, 8, 3, 1) == -1
    assert kvb.heads_per_workgroup(kvb.Shape(2, 56, 8, 128)) == 7
    assert kvb.heads_per_workgroup(kvb.Shape(1, 16, 1, 128), "f32") == 8
    assert kvb.heads_per_workgroup(kvb.Shape(1, 16, 1, 128), "i8") == 16
    assert kvb.heads_per_workgroup(kvb.Shape(1, 16, 1, 128), "f16") == 16
    assert kvb.heads_per_workgroup(kvb.Shape(1, 64, 1, 128), "i8") == 32


def test_partition_policy_counts_live_heads(kvb):
    """The MI355X partition policy counts workgroups with kvb_heads_per_workgroup. Group 3, batch 1,
    8 KV heads: one workgroup per KV head, so 8 per partition index, and 256 workgroups need 32
    partitions of 256 tokens at 8192 tokens (counting a workgroup per query head, 24 per partition
    index, would stop at 512). Groups 7 and 8 at c4's size both give 4096-token partitions."""
    s3 = kvb.Shape(1, 24, 8, 128)
    assert kvb.mi355x_part_tokens(s3, 8192) == 256
    s7 = kvb.Shape(4, 56, 8, 128)
    s8 = kvb.Shape(4, 64, 8, 128)
    assert kvb.mi355x_part_tokens(s7, 32768) == kvb.mi355x_part_tokens(s8, 32768) == 4096
