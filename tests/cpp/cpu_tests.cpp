// Properties of the fp64 oracle and of the host layer's layout, scatter and quantiser that hold
// exactly (no GPU needed): the reference's tests/cpu_tests.cpp:32-152, plus the host layer against
// the oracle, bit for bit.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <random>
#include <set>

#include "kvb/rng.hpp"
#include "kvb_host.h"
#include "test_util.hpp"

using namespace kvbt;

namespace {

int failed = 0, passed = 0;

void expect(bool ok, const char* what) {
    ok ? ++passed : ++failed;
    std::printf("%s %s\n", ok ? "ok  " : "FAIL", what);
}

std::vector<float> random_vec(size_t n, uint64_t seed) {
    std::mt19937_64 g(seed);
    std::vector<float> x(n);
    for (auto& e : x) e = rng::uniform_pm1(g());
    return x;
}

double max_diff(const std::vector<float>& a, const std::vector<float>& b) { return max_abs_diff(a.data(), b.data(), a.size()); }

void attention(const Shape& s, const std::vector<int>& lens, int max_len, const float* q, const float* k, const float* v,
               float* out, float scale, int threads = 1) {
    const kvbo_shape os = oshape(s);
    kvbo_attention_f32(&os, lens.data(), max_len, q, k, v, out, scale, threads);
}

}  // namespace

int main() {
    const Shape s{2, 4, 2, 64};
    const std::vector<int> lens{37, 5};
    const int max_len = 37, D = s.head_dim;
    const float scale = 1.0f / std::sqrt(float(D));
    const size_t nkv = size_t(s.batch) * s.num_kv_heads * max_len * D, nq = size_t(s.batch) * s.num_heads * D;
    const auto k = random_vec(nkv, 1), v = random_vec(nkv, 2);

    {  // q = 0: every score is 0, so the output is the plain mean of V over the sequence.
        std::vector<float> q(nq, 0.0f), out(nq), want(nq);
        attention(s, lens, max_len, q.data(), k.data(), v.data(), out.data(), scale);
        for (int b = 0; b < s.batch; ++b)
            for (int h = 0; h < s.num_heads; ++h)
                for (int d = 0; d < D; ++d) {
                    double sum = 0;
                    for (int t = 0; t < lens[b]; ++t) sum += v[contig_index(s, max_len, b, h / s.group(), t, d)];
                    want[(b * s.num_heads + h) * D + d] = float(sum / lens[b]);
                }
        expect(max_diff(out, want) < 1e-6, "zero query gives the mean of V");
    }
    {  // One key aligned with a huge query dominates: the output is that token's V row, exactly.
        std::vector<float> q(nq, 0.0f), kk(nkv, 0.0f), out(nq), want(nq);
        for (size_t i = 0; i < nq; i += D) q[i] = 1000.0f;
        const int hot[] = {11, 4};
        for (int b = 0; b < s.batch; ++b)
            for (int kvh = 0; kvh < s.num_kv_heads; ++kvh) kk[contig_index(s, max_len, b, kvh, hot[b], 0)] = 1.0f;
        attention(s, lens, max_len, q.data(), kk.data(), v.data(), out.data(), scale);
        for (int b = 0; b < s.batch; ++b)
            for (int h = 0; h < s.num_heads; ++h)
                for (int d = 0; d < D; ++d)
                    want[(b * s.num_heads + h) * D + d] = v[contig_index(s, max_len, b, h / s.group(), hot[b], d)];
        expect(max_diff(out, want) == 0.0, "a dominant key selects its V row");
    }
    {  // Scores near +-1000 overflow exp() without the max shift; the output stays a convex combination.
        std::vector<float> q = random_vec(nq, 3), out(nq);
        for (auto& e : q) e *= 8000.0f;
        attention(s, lens, max_len, q.data(), k.data(), v.data(), out.data(), scale);
        bool bounded = true;
        for (float o : out) bounded &= std::isfinite(o) && std::fabs(o) <= 1.0f;
        expect(bounded, "huge scores stay finite (max-shifted softmax)");
    }
    {  // GQA: query heads that share a KV head and a query give identical outputs.
        std::vector<float> q = random_vec(nq, 5), out(nq);
        for (int b = 0; b < s.batch; ++b)
            for (int d = 0; d < D; ++d) q[(b * s.num_heads + 1) * D + d] = q[(b * s.num_heads + 0) * D + d];
        attention(s, lens, max_len, q.data(), k.data(), v.data(), out.data(), scale, 3);
        bool same = true;
        for (int b = 0; b < s.batch; ++b)
            for (int d = 0; d < D; ++d) same &= out[(b * s.num_heads + 0) * D + d] == out[(b * s.num_heads + 1) * D + d];
        expect(same, "query heads 0 and 1 share KV head 0");
    }
    {  // The block table is a permutation of the pool, and scatter + indexed read is the identity.
        const std::vector<int> plens{1, 16, 17, 100};
        const Shape ps{4, 2, 2, 64};
        const PagedLayout L = make_paged_layout(plens, 16, 7);
        std::set<int> used;
        int live = 0;
        for (size_t b = 0; b < plens.size(); ++b)
            for (int i = 0; i < (plens[b] + 15) / 16; ++i, ++live) used.insert(L.block_table[b * L.max_blocks + i]);
        expect(L.num_blocks == 1 + 1 + 2 + 7 && int(used.size()) == live && *used.rbegin() == L.num_blocks - 1,
               "block table maps logical blocks onto distinct physical blocks");
        const auto src = random_vec(size_t(4) * 2 * 100 * 64, 8);
        std::vector<float> dst(size_t(L.num_blocks) * 2 * 16 * 64, 0.0f);
        scatter_to_paged<float>(ps, L, plens, 100, src.data(), dst.data());
        bool same = true;
        for (int b = 0; b < 4; ++b)
            for (int kvh = 0; kvh < 2; ++kvh)
                for (int t = 0; t < plens[b]; ++t)
                    for (int d = 0; d < 64; ++d) same &= dst[paged_index(ps, L, b, kvh, t, d)] == src[contig_index(ps, 100, b, kvh, t, d)];
        expect(same, "paged scatter round-trips through paged_index");
    }
    {  // An oversized pool: live ids are distinct and within the pool, the unused ones are poisoned.
        const std::vector<int> plens{1, 16, 17, 100, 0};
        const Shape ps{5, 2, 2, 64};
        const PagedLayout L = make_paged_layout(plens, 16, 9, 3.0);
        std::set<int> used;
        bool in_pool = true;
        for (int32_t id : L.block_table)
            if (id >= 0) used.insert(id), in_pool &= id < L.num_blocks;
        expect(L.live_blocks == 11 && L.num_blocks == 33 && int(used.size()) == 11 && in_pool,
               "3x pool: 11 live blocks of 33, distinct and inside the pool");
        std::vector<float> pool(size_t(L.num_blocks) * 2 * 16 * 64, 0.0f);
        poison_paged(ps, L, plens, 4, pool.data(), nullptr);
        size_t nans = 0;
        for (float x : pool) nans += std::isnan(x);
        const size_t live_rows = 1 + 16 + 17 + 100;
        expect(nans == (size_t(33) * 16 - live_rows) * 2 * 64, "poison marks exactly the rows no live token owns");
    }
    {  // The host layer's block table equals the oracle's, bit for bit, for any pool factor.
        bool same = true;
        for (double pf : {1.0, 1.25, 1.5, 2.0, 3.0})
            for (uint64_t seed : {0ull, 1ull, 77ull, 0x9e3779b97f4a7c15ull}) {
                const std::vector<int> plens{0, 1, 63, 64, 65, 2047, 2048, 2049, 300};
                const PagedLayout L = make_paged_layout(plens, 64, seed, pf);
                std::vector<int32_t> ot(L.block_table.size());
                kvbo_make_paged_layout(plens.data(), int(plens.size()), 64, pf, seed, ot.data());
                same &= ot == L.block_table;
            }
        expect(same, "block tables equal the oracle's for pool factors 1..3");
    }
    {  // fp16 storage: the oracle reads half values exactly; the result stays near the fp32 one.
        std::vector<uint16_t> kh(nkv), vh(nkv);
        for (size_t i = 0; i < nkv; ++i) kh[i] = kvbo_f32_to_f16(k[i]), vh[i] = kvbo_f32_to_f16(v[i]);
        std::vector<float> q = random_vec(nq, 9), o32(nq), o16(nq);
        attention(s, lens, max_len, q.data(), k.data(), v.data(), o32.data(), scale);
        const kvbo_shape os = oshape(s);
        kvbo_attention_f16(&os, lens.data(), max_len, q.data(), kh.data(), vh.data(), o16.data(), scale, 1);
        const double d = max_diff(o32, o16);
        expect(d > 0 && d < 5e-3, "fp16 storage reference differs from fp32 only by rounding");
    }
    {  // The host layer's fp16 rounding (the compiler's conversion) equals the oracle's, exhaustively
       // over every float whose top 20 bits vary (all exponents, signs, and the rounding bits).
        bool same = true;
        for (uint32_t hi = 0; hi < (1u << 20) && same; ++hi) {
            for (uint32_t lo : {0u, 0xfffu, 0x1000u, 0x1001u, 0x17ffu}) {
                const uint32_t bits = (hi << 12) | lo;
                float f;
                std::memcpy(&f, &bits, 4);
                if (std::isnan(f)) continue;
                const half_t h = half_t(f);
                uint16_t hb;
                std::memcpy(&hb, &h, 2);
                same &= hb == kvbo_f32_to_f16(f);
            }
        }
        expect(same, "fp16 rounding equals the oracle's round-to-nearest-even");
    }
    {  // int8 storage: each (block, KV head) slice round-trips within half its scale, its largest
       // value maps to +-127, an all-zero slice stays zero, and the host quantiser equals the oracle's.
        const std::vector<int> plens{1, 16, 17, 40};
        const Shape ps{4, 2, 2, 64};
        const PagedLayout L = make_paged_layout(plens, 16, 11);
        auto src = random_vec(size_t(4) * 2 * 40 * 64, 12);
        for (int t = 0; t < 40; ++t)  // sequence 3, KV head 1: a slice 8x larger, and one of zeros
            for (int d = 0; d < 64; ++d) {
                src[contig_index(ps, 40, 3, 1, t, d)] *= t < 16 ? 8.0f : 1.0f;
                if (t >= 32) src[contig_index(ps, 40, 3, 1, t, d)] = 0.0f;
            }
        const size_t n = size_t(L.num_blocks) * 2 * 16 * 64;
        std::vector<int8_t> q8(n, 0), o8(n, 0);
        std::vector<float> scales(size_t(L.num_blocks) * 2, -1.0f), oscales(scales), back(src.size(), 0.0f);
        quantize_to_paged_i8(ps, L, plens, 40, src.data(), q8.data(), scales.data());
        dequantize_paged_i8(ps, L, plens, 40, q8.data(), scales.data(), back.data());
        bool within = true;
        for (int b = 0; b < 4; ++b)
            for (int kvh = 0; kvh < 2; ++kvh)
                for (int t = 0; t < plens[b]; ++t) {
                    const float sc = scales[size_t(L.block_table[b * L.max_blocks + t / 16]) * 2 + kvh];
                    for (int d = 0; d < 64; ++d) {
                        const size_t i = contig_index(ps, 40, b, kvh, t, d);
                        within &= std::fabs(back[i] - src[i]) <= 0.5f * sc * (1 + 1e-6f);
                    }
                }
        int peak = 0;
        for (int8_t x : q8) peak = std::max(peak, std::abs(int(x)));
        const float big = scales[size_t(L.block_table[3 * L.max_blocks + 0]) * 2 + 1];
        const float small = scales[size_t(L.block_table[3 * L.max_blocks + 1]) * 2 + 1];
        const float zero = scales[size_t(L.block_table[3 * L.max_blocks + 2]) * 2 + 1];
        expect(within && peak == 127, "int8 blocks round-trip within scale / 2, the largest value maps to 127");
        expect(big > 6 * small && small > 0 && zero == 0.0f, "int8 scale is per (block, KV head)");
        const kvbo_shape os = oshape(ps);
        kvbo_quantize_to_paged_i8(&os, 16, L.max_blocks, L.block_table.data(), plens.data(), 40, src.data(), o8.data(),
                                  oscales.data());
        expect(o8 == q8 && std::memcmp(oscales.data(), scales.data(), scales.size() * 4) == 0,
               "host int8 quantiser equals the oracle's bit for bit");
    }
    {  // The reference's comparison KAT and the auto_part_tokens thresholds (tests/boundary_tests.cpp:80-92).
        const float a[] = {1.0f, NAN, 3.0f}, b[] = {1.0f, 2.0f, 3.0f}, c[] = {1.0f, 2.0f, 3.5f};
        expect(std::isinf(max_abs_diff(a, b, 3)) && std::isinf(max_abs_diff(a, a, 3)) && max_abs_diff(b, c, 3) == 0.5,
               "max_abs_diff: NaN counts as infinite, finite values compare");
        const Shape as{2, 32, 8, 128};
        const int want[][2] = {{0, 64}, {1, 64}, {3968, 64}, {3969, 128}, {7936, 128}, {7937, 256}, {15872, 256}, {15873, 512}, {1 << 20, 512}};
        bool ok = true;
        for (const auto& [len, part] : want)
            ok &= auto_part_tokens(as, len) == part && kvb_auto_part_tokens(2, 8, len) == part &&
                  kvbo_auto_part_tokens(2, 8, len) == part;
        expect(ok, "auto_part_tokens thresholds (host, C ABI and oracle)");
    }
    {  // An empty sequence attends to nothing: exactly 0, and its neighbour is untouched; it takes no block.
        const Shape es{3, 4, 2, 64};
        const std::vector<int> elens{0, 9, 0}, alone{9};
        const size_t ekv = size_t(3) * 2 * 9 * 64, eq = size_t(3) * 4 * 64, row = size_t(4) * 64;
        std::vector<float> q(eq, 0.5f), kk(ekv, 0.25f), vv(ekv), out(eq, NAN), one(row);
        for (size_t i = 0; i < ekv; ++i) vv[i] = float(i % 7) / 7;
        attention(es, elens, 9, q.data(), kk.data(), vv.data(), out.data(), 0.125f);
        attention({1, 4, 2, 64}, alone, 9, q.data(), kk.data() + size_t(2) * 9 * 64, vv.data() + size_t(2) * 9 * 64,
                  one.data(), 0.125f);
        const std::vector<float> zero(row, 0.0f);
        expect(max_abs_diff(out.data(), zero.data(), row) == 0 && max_abs_diff(out.data() + 2 * row, zero.data(), row) == 0,
               "oracle: an empty sequence gives exactly 0");
        expect(max_abs_diff(out.data() + row, one.data(), row) == 0, "oracle: an empty neighbour changes nothing");
        const PagedLayout L = make_paged_layout(elens, 16, 3), none = make_paged_layout(std::vector<int>{0, 0}, 16, 3);
        expect(L.num_blocks == 1 && L.max_blocks == 1 && L.block_table == std::vector<int32_t>{-1, 0, -1},
               "layout: an empty sequence takes no block");
        expect(none.num_blocks == 0 && none.max_blocks == 0 && none.block_table.empty(), "layout: an all-empty batch has no blocks");
    }
    {  // The workload generator is deterministic and its streams do not depend on the other lengths.
        const Shape ws{2, 8, 2, 64};
        const int la[] = {40, 7}, lb[] = {40, 30};
        const size_t n = size_t(2) * 2 * 40 * 64;
        std::vector<float> qa(2 * 8 * 64), qb(qa.size()), ka(n), va(n), kb(n), vb(n), ka2(n), va2(n);
        kvbh_fill_workload(2, 8, 2, 64, la, 40, KVB_KV_F32, 5, 3.0f, 0, KVBH_UNIFORM, qa.data(), ka.data(), va.data(), nullptr, nullptr, 1);
        kvbh_fill_workload(2, 8, 2, 64, lb, 40, KVB_KV_F32, 5, 3.0f, 0, KVBH_UNIFORM, qb.data(), kb.data(), vb.data(), nullptr, nullptr, 4);
        kvbh_fill_workload(2, 8, 2, 64, la, 40, KVB_KV_F32, 5, 3.0f, 0, KVBH_UNIFORM, qa.data(), ka2.data(), va2.data(), nullptr, nullptr, 3);
        bool same = qa == qb && ka == ka2 && va == va2;
        for (int kvh = 0; kvh < 2; ++kvh)
            for (int t = 0; t < 40; ++t)
                for (int d = 0; d < 64; ++d) same &= ka[contig_index(ws, 40, 0, kvh, t, d)] == kb[contig_index(ws, 40, 0, kvh, t, d)];
        bool bounded = true;
        for (float x : ka) bounded &= x > -1.0f && x < 1.0f;
        for (int t = 7; t < 40; ++t)
            for (int d = 0; d < 64; ++d) bounded &= ka[contig_index(ws, 40, 1, 0, t, d)] == 0.0f;
        expect(same && bounded, "workload streams are per (sequence, KV head), in (-1, 1), 0 past a length");
    }

    std::printf("%d passed, %d failed\n", passed, failed);
    return failed ? 1 : 0;
}
