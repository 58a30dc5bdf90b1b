"""Pins the CPU oracle (oracle/kvb_oracle.c) before anything is checked against it: known-answer
tests, closed forms, an independent fp64 evaluation (scipy's softmax), the reference's own CPU code
built into oracle/_ref, and the golden fixtures under tests/golden/ (made from oracle/_ref)."""
import glob
import os

import numpy as np
import pytest
from scipy.special import softmax

from conftest import ROOT

GOLDEN = sorted(glob.glob(os.path.join(ROOT, "tests", "golden", "*.npz")))


class S:
    def __init__(self, b, h, hkv, d):
        self.batch, self.num_heads, self.num_kv_heads, self.head_dim = b, h, hkv, d


def rand(shape, seed, lo=-1.0, hi=1.0):
    return np.random.Generator(np.random.PCG64(seed)).uniform(lo, hi, shape).astype(np.float32)


def scipy_attention(s, lens, q, k, v):
    """Textbook softmax(q k^T / sqrt(D)) v in fp64 with scipy's softmax; 0 for an empty sequence."""
    G = s.num_heads // s.num_kv_heads
    scale = float(np.float32(1) / np.float32(np.sqrt(np.float32(s.head_dim))))
    out = np.zeros((s.batch, s.num_heads, s.head_dim))
    for b in range(s.batch):
        L = int(lens[b])
        if L == 0:
            continue
        for h in range(s.num_heads):
            K = k[b, h // G, :L].astype(np.float64)
            V = v[b, h // G, :L].astype(np.float64)
            p = softmax(K @ q[b, h].astype(np.float64) * scale)
            out[b, h] = p @ V
    return out


def test_mt19937_64_known_answer(oracle):
    # The C++ standard fixes the 10000th output of a default-seeded mt19937_64 ([rand.predef]).
    assert oracle.mt64_stream(5489, 10000)[-1] == 9981545732273789042


def test_f16_rounding_matches_numpy(oracle):
    # Every binary16 value round-trips, and random / boundary floats round like numpy (RNE).
    for bits in range(0, 1 << 16, 7):
        h = np.array([bits], np.uint16).view(np.float16)[0]
        if np.isnan(h):
            continue
        assert oracle.f32_to_f16_bits(float(h)) == bits
    x = np.concatenate([rand(20000, 1, -70000, 70000), rand(20000, 2, -1e-4, 1e-4), rand(20000, 3, -8, 8),
                        np.array([65504, 65519.99, 65520, 6.1035156e-05, 5.9604645e-08, 2.9802322e-08, 2.98e-08,
                                  0.0, -0.0, np.inf, -np.inf], np.float32)])
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    got = np.array([oracle.f32_to_f16_bits(float(v)) for v in x], np.uint16)
    assert np.array_equal(got, want)


def test_max_abs_diff_known_answers(oracle):
    a, b, c = np.array([1, np.nan, 3], np.float32), np.array([1, 2, 3], np.float32), np.array([1, 2, 3.5], np.float32)
    assert np.isinf(oracle.max_abs_diff(a, b)) and np.isinf(oracle.max_abs_diff(a, a))
    assert oracle.max_abs_diff(b, c) == 0.5


def test_auto_part_tokens_thresholds(oracle):
    # tests/boundary_tests.cpp:86-92: 16 (sequence, KV head) pairs -> thresholds at 32 partitions.
    for length, part in [(0, 64), (1, 64), (3968, 64), (3969, 128), (7936, 128), (7937, 256), (15872, 256),
                         (15873, 512), (1 << 20, 512)]:
        assert oracle.auto_part_tokens(2, 8, length) == part


@pytest.mark.skipif(not os.path.exists(os.path.join(ROOT, "oracle", "_ref", "libkvbref.so")), reason="oracle/_ref not built")
def test_auto_part_tokens_matches_reference(oracle):
    for b in (1, 2, 3, 16):
        for hkv in (1, 2, 8):
            for L in list(range(0, 5000, 37)) + [32768, 100000]:
                assert oracle.auto_part_tokens(b, hkv, L) == oracle.ref.kvbref_auto_part_tokens(b, 32, hkv, 128, L)


@pytest.mark.parametrize("shape,lens", [((2, 4, 2, 64), [37, 5]), ((3, 8, 2, 128), [1, 0, 70]),
                                        ((1, 16, 2, 64), [33]), ((2, 4, 4, 64), [0, 0])])
def test_attention_matches_scipy_softmax(oracle, shape, lens):
    s = S(*shape)
    L = max(lens)
    q = rand((s.batch, s.num_heads, s.head_dim), 5, -3, 3)
    k = rand((s.batch, s.num_kv_heads, L, s.head_dim), 6)
    v = rand((s.batch, s.num_kv_heads, L, s.head_dim), 7)
    got = oracle.attention(s, lens, L, q, k, v, threads=3)
    want = scipy_attention(s, lens, q, k, v)
    assert np.abs(got - want).max() <= 2e-7
    for b, ln in enumerate(lens):  # an empty sequence gives exactly 0
        if ln == 0:
            assert not got[b].any()


def test_attention_closed_forms(oracle):
    s = S(2, 4, 2, 64)
    lens, L = [37, 5], 37
    k, v = rand((2, 2, L, 64), 1), rand((2, 2, L, 64), 2)
    # zero query: the mean of V
    out = oracle.attention(s, lens, L, np.zeros((2, 4, 64), np.float32), k, v)
    for b in range(2):
        for h in range(4):
            assert np.abs(out[b, h] - v[b, h // 2, :lens[b]].astype(np.float64).mean(0)).max() < 1e-6
    # a dominant key: exactly that V row
    q = np.zeros((2, 4, 64), np.float32)
    q[:, :, 0] = 1000.0
    kk = np.zeros_like(k)
    hot = [11, 4]
    for b in range(2):
        kk[b, :, hot[b], 0] = 1.0
    out = oracle.attention(s, lens, L, q, kk, v)
    for b in range(2):
        for h in range(4):
            assert np.array_equal(out[b, h], v[b, h // 2, hot[b]])
    # huge scores stay finite and convex
    out = oracle.attention(s, lens, L, rand((2, 4, 64), 3) * 8000, k, v)
    assert np.isfinite(out).all() and np.abs(out).max() <= 1.0


def test_f16_storage_reads_stored_values(oracle):
    s = S(2, 8, 2, 64)
    lens, L = [50, 9], 50
    q = rand((2, 8, 64), 9, -3, 3)
    k, v = rand((2, 2, L, 64), 10).astype(np.float16), rand((2, 2, L, 64), 11).astype(np.float16)
    got = oracle.attention(s, lens, L, q, k, v)
    want = oracle.attention(s, lens, L, q, k.astype(np.float32), v.astype(np.float32))
    assert np.array_equal(got, want)


def test_partition_states_merge_to_attention(oracle):
    # The split-K identity the decode/reduce kernels rely on: merging partitions with weights
    # l_i exp(m_i - M) reproduces the whole softmax.
    s = S(2, 8, 2, 64)
    lens, L, part = [200, 65], 200, 64
    q = rand((2, 8, 64), 12, -3, 3)
    k, v = rand((2, 2, L, 64), 13), rand((2, 2, L, 64), 14)
    full = oracle.attention(s, lens, L, q, k, v)
    for b in range(2):
        for h in range(8):
            states = [oracle.partition_state(s, lens, L, q, k, v, part, b, h, p) for p in range(4)]
            live = [x for x in states if x is not None]
            assert len(live) == -(-lens[b] // part) and all(x is None for x in states[len(live):])
            M = max(m for m, _, _ in live)
            w = np.array([l * np.exp(m - M) for m, l, _ in live])
            merged = (w[:, None] * np.array([o for _, _, o in live])).sum(0) / w.sum()
            assert np.abs(merged - full[b, h]).max() < 1e-6


def test_layout_invariants(oracle):
    lens = [1, 16, 17, 100]
    t = oracle.make_paged_layout(lens, 16, 7)
    live = t[t >= 0]
    assert t.shape == (4, 7) and len(set(live.tolist())) == 11 and live.max() == 10
    assert oracle.make_paged_layout([0, 9, 0], 16, 3).ravel().tolist() == [-1, 0, -1]
    assert oracle.make_paged_layout([0, 0], 16, 3).size == 0
    t3 = oracle.make_paged_layout(lens + [0], 16, 9, 3.0)
    assert oracle.layout_dims(lens + [0], 16, 3.0) == (7, 11, 33)
    assert len(set(t3[t3 >= 0].tolist())) == 11 and t3.max() < 33
    # each sequence's blocks in order: rows of the table list only its own count of ids, then -1
    for b, ln in enumerate(lens):
        nb = -(-ln // 16)
        assert (t[b, :nb] >= 0).all() and (t[b, nb:] == -1).all()


def test_quantizer_closed_form(oracle):
    s = S(4, 2, 2, 64)
    lens, L = [1, 16, 17, 40], 40
    table = oracle.make_paged_layout(lens, 16, 11)
    src = rand((4, 2, L, 64), 12)
    src[3, 1, :16] *= 8
    src[3, 1, 32:] = 0
    paged, scales = oracle.quantize(s, 16, table, lens, L, src, 7)
    back = oracle.dequantize(s, 16, table, lens, L, paged, scales)
    for b in range(4):
        for kvh in range(2):
            for t in range(lens[b]):
                sc = scales[table[b, t // 16], kvh]
                # s/2 in exact arithmetic, plus the fp32 rounding of x / s and of q * s (2 ulps of x)
                slack = 2 * np.spacing(np.abs(src[b, kvh, t]))
                assert (np.abs(back[b, kvh, t] - src[b, kvh, t]) <= 0.5 * sc + slack).all()
    assert np.abs(paged).max() == 127 and paged.min() >= -127
    big, small, zero = (scales[table[3, i], 1] for i in range(3))
    assert big > 6 * small > 0 and zero == 0


def test_fp16_storage_bound_sound_where_each_term_is_needed(oracle):
    """The fp16 storage-error bound (tests/gpu_tests.cpp:19-40) holds on two constructed cases,
    each of which exceeds what the bound would be without one of its terms."""
    u = 2.0 ** -11
    # (a) q = 0 (no score error) and every V element the tie 1 + 2^-11, which rounds down to 1:
    # the output moves by exactly u, more than the fp32 tolerance alone.
    s = S(1, 2, 1, 64)
    q = np.zeros((1, 2, 64), np.float32)
    k32 = rand((1, 1, 5, 64), 21)
    v32 = np.full((1, 1, 5, 64), 1 + u, np.float32)
    exact = oracle.attention(s, [5], 5, q, k32, v32)
    stored = oracle.attention(s, [5], 5, q, k32.astype(np.float16), v32.astype(np.float16))
    err = oracle.max_abs_diff(stored, exact)
    assert err == u
    assert err <= oracle.fp16_storage_bound(s, [5], 5, q, k32, v32)
    # (b) two K rows that round to the same fp16 row from either side (1 + 2^-11 down, 1 - 2^-12 up,
    # a tie to even) under a large query: the stored scores tie, the exact ones differ by
    # x (2^-11 + 2^-12) with x = scale * sum q = 1000, and with V = +1 / -1 the output moves by
    # tanh(x * 3 * 2^-13), about 0.35: far beyond u max|v|.
    s = S(1, 1, 1, 128)
    q = np.full((1, 1, 128), 1000 / np.sqrt(128), np.float32)
    k32 = np.stack([np.full(128, 1 + u), np.full(128, 1 - u / 2)]).astype(np.float32).reshape(1, 1, 2, 128)
    v32 = np.stack([np.ones(128), -np.ones(128)]).astype(np.float32).reshape(1, 1, 2, 128)
    assert np.array_equal(k32[0, 0, 0].astype(np.float16), k32[0, 0, 1].astype(np.float16))
    exact = oracle.attention(s, [2], 2, q, k32, v32)
    stored = oracle.attention(s, [2], 2, q, k32.astype(np.float16), v32.astype(np.float16))
    err = oracle.max_abs_diff(stored, exact)
    assert abs(err - np.tanh(1000 * 3 * 2.0 ** -13)) < 1e-3 and not stored.any()
    assert err <= oracle.fp16_storage_bound(s, [2], 2, q, k32, v32)


def test_i8_storage_bound_sound_where_each_term_is_needed(oracle):
    """The int8 storage-error bound (tests/gpu_tests.cpp:42-62) likewise: two tokens in one page,
    so one scale per K and per V."""
    s = S(1, 1, 1, 64)
    table = oracle.make_paged_layout([2], 2, 5)

    def err_and_bound(q, k32, v32):
        kq, ks = oracle.quantize(s, 2, table, [2], 2, k32, 1)
        vq, vs = oracle.quantize(s, 2, table, [2], 2, v32, 1)
        kd = oracle.dequantize(s, 2, table, [2], 2, kq, ks)
        vd = oracle.dequantize(s, 2, table, [2], 2, vq, vs)
        err = oracle.max_abs_diff(oracle.attention(s, [2], 2, q, kd, vd), oracle.attention(s, [2], 2, q, k32, v32))
        return err, oracle.i8_storage_bound(s, [2], 2, table, q, ks, vs)

    # (a) q = 0: one token's V row sets the scale 1/127, the other's 0.49/127 all round to 0; the
    # mean moves by 0.49/127/2, about the V term s_v / 2 = 1/254 and far beyond the fp32 tolerance.
    q = np.zeros((1, 1, 64), np.float32)
    k32 = rand((1, 1, 2, 64), 22)
    v32 = np.stack([np.ones(64), np.full(64, 0.49 / 127)]).astype(np.float32).reshape(1, 1, 2, 64)
    err, bound = err_and_bound(q, k32, v32)
    assert abs(err - 0.49 / 127 / 2) < 1e-6 and err <= bound
    # (b) K rows [1, 0.49/127 ...] and [1, 0 ...] quantise to the same row, so the stored scores tie;
    # with q = 30 on dims 1..63 the exact scores differ by 30 * 63 * 0.49 / 127 / 8, about 0.91, and
    # with V = +1 / -1 the output moves by tanh(0.455): far beyond the V term.
    q = np.zeros((1, 1, 64), np.float32)
    q[0, 0, 1:] = 30
    k32 = np.zeros((1, 1, 2, 64), np.float32)
    k32[0, 0, :, 0] = 1
    k32[0, 0, 0, 1:] = 0.49 / 127
    v32 = np.stack([np.ones(64), -np.ones(64)]).astype(np.float32).reshape(1, 1, 2, 64)
    err, bound = err_and_bound(q, k32, v32)
    assert abs(err - np.tanh(30 * 63 * 0.49 / 127 / 8 / 2)) < 1e-3 and err <= bound


@pytest.mark.skipif(not os.path.exists(os.path.join(ROOT, "oracle", "_ref", "libkvbref.so")), reason="oracle/_ref not built")
class TestAgainstReferenceBuild:
    """The reference's own src/reference.cpp, compiled into oracle/_ref, on the same inputs."""

    @pytest.mark.parametrize("shape,lens,f16", [((2, 8, 2, 128), [70, 3], False), ((3, 4, 4, 64), [5, 0, 33], True),
                                                ((1, 16, 2, 64), [257], False)])
    def test_attention_identical(self, oracle, shape, lens, f16):
        s = S(*shape)
        L = max(lens)
        q = rand((s.batch, s.num_heads, s.head_dim), 21, -8, 8)
        k = rand((s.batch, s.num_kv_heads, L, s.head_dim), 22)
        v = rand((s.batch, s.num_kv_heads, L, s.head_dim), 23)
        if f16:
            k, v = k.astype(np.float16), v.astype(np.float16)
        ours = oracle.attention(s, lens, L, q, k, v, threads=2)
        theirs = oracle.ref_attention(s, lens, L, q, k, v, threads=1)
        assert np.array_equal(ours, theirs)

    def test_layout_invariants_and_quantiser_identical(self, oracle):
        import ctypes
        lens = np.array([1, 16, 17, 100, 0, 64], np.int32)
        table = np.full(6 * 7, -7, np.int32)
        mb = ctypes.c_int()
        nb = oracle.ref.kvbref_make_paged_layout(lens.ctypes.data, 6, 16, 5, table.ctypes.data, table.size,
                                                 ctypes.byref(mb))
        table = table[: 6 * mb.value].reshape(6, mb.value)
        ours = oracle.make_paged_layout(lens, 16, 5)
        assert (nb, mb.value) == (15, 7) and np.array_equal(table < 0, ours < 0)
        assert sorted(table[table >= 0].tolist()) == sorted(ours[ours >= 0].tolist()) == list(range(15))
        # quantiser on the reference's own table: identical bytes and scales
        s = S(6, 2, 2, 64)
        src = rand((6, 2, 100, 64), 31)
        src[2] *= 5
        paged, scales = oracle.quantize(s, 16, table, lens, 100, src, nb)
        rp = np.zeros_like(paged)
        rs = np.zeros_like(scales)
        oracle.ref.kvbref_quantize_to_paged_i8(6, 2, 2, 64, 16, mb.value, nb, table.ctypes.data, lens.ctypes.data, 100,
                                               src.ctypes.data, rp.ctypes.data, rs.ctypes.data)
        assert np.array_equal(paged, rp) and np.array_equal(scales.view(np.uint32), rs.view(np.uint32))
        back = oracle.dequantize(s, 16, table, lens, 100, paged, scales)
        rback = np.zeros_like(back)
        oracle.ref.kvbref_dequantize_paged_i8(6, 2, 2, 64, 16, mb.value, nb, table.ctypes.data, lens.ctypes.data, 100,
                                              paged.ctypes.data, scales.ctypes.data, rback.ctypes.data)
        assert np.array_equal(back, rback)
        # scatter
        ps = oracle.scatter(s, 16, table, lens, 100, src, nb)
        rps = np.zeros_like(ps)
        oracle.ref.kvbref_scatter_to_paged_f32(6, 2, 2, 64, 16, mb.value, nb, table.ctypes.data, lens.ctypes.data, 100,
                                               src.ctypes.data, rps.ctypes.data)
        assert np.array_equal(ps, rps)

    def test_max_abs_diff_identical(self, oracle):
        a = rand(1000, 41)
        b = rand(1000, 42)
        b[17] = np.nan
        for x, y in ((a, a), (a, b), (b, b), (a, a + 1e-3)):
            r = oracle.ref.kvbref_max_abs_diff(x.ctypes.data, np.ascontiguousarray(y).ctypes.data, x.size)
            assert oracle.max_abs_diff(x, y) == r or (np.isinf(r) and np.isinf(oracle.max_abs_diff(x, y)))


@pytest.mark.parametrize("path", GOLDEN, ids=[os.path.basename(p) for p in GOLDEN])
def test_oracle_against_golden(oracle, path):
    g = np.load(path, allow_pickle=False)
    s = S(*g["shape"].tolist())
    lens, L = g["lens"], int(g["max_len"])
    if "k_deq" in g:  # int8 case: the reference dequantised its own quantisation
        paged, scales = oracle.quantize(s, int(g["page"]), g["table"], lens, L, g["k"], int(g["num_blocks"]))
        assert np.array_equal(paged, g["k_paged"]) and np.array_equal(scales, g["k_scale"])
        got = oracle.attention(s, lens, L, g["q"], g["k_deq"], g["v_deq"])
    else:
        got = oracle.attention(s, lens, L, g["q"], g["k"], g["v"])
    assert np.array_equal(got, g["out"]), np.abs(got - g["out"]).max()
