// The workload generator and the C ABI of include/kvb_host.h over the host layer's cache writers.
#include "kvb_host.h"

#include <algorithm>
#include <atomic>
#include <cmath>
#include <exception>
#include <thread>
#include <vector>

#include "kvb/hip_attn.hpp"
#include "kvb/layout.hpp"
#include "kvb/rng.hpp"

namespace {

kvb::Shape shape(int B, int H, int Hkv, int D) { return kvb::Shape{B, H, Hkv, D}; }

kvb::PagedLayout layout_view(int page, int max_blocks, int pool, const int32_t* table, int batch) {
    kvb::PagedLayout L;
    L.page_size = page;
    L.max_blocks = max_blocks;
    L.num_blocks = pool;
    L.block_table.assign(table, table + size_t(batch) * max_blocks);
    return L;
}

template <class F>
int guarded(F&& f) {
    try {
        f();
        return 0;
    } catch (const std::exception&) {
        return -1;
    }
}

// Runs fn(i) for i in [0, n) on `threads` workers.
template <class F>
void parallel_for(size_t n, int threads, F&& fn) {
    if (threads <= 0) threads = int(std::max(1u, std::thread::hardware_concurrency()));
    threads = int(std::min<size_t>(size_t(threads), std::max<size_t>(n, 1)));
    std::atomic<size_t> next{0};
    auto work = [&] {
        for (size_t i; (i = next.fetch_add(1)) < n;) fn(i);
    };
    std::vector<std::thread> pool;
    for (int t = 1; t < threads; ++t) pool.emplace_back(work);
    work();
    for (auto& th : pool) th.join();
}

}  // namespace

extern "C" {

int kvbh_fill_workload(int batch, int num_heads, int num_kv_heads, int head_dim, const int* lens, int max_len,
                       int kv_type, uint64_t seed, float q_amp, int varied, int dist, float* q, void* k, void* v,
                       float* k32, float* v32, int threads) {
    using namespace kvb::rng;
    if (batch < 0 || num_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 || max_len < 0 || !q || (batch && !lens) ||
        (dist != KVBH_UNIFORM && dist != KVBH_NORMAL) || kv_type < KVB_KV_F32 || kv_type > KVB_KV_I8)
        return -1;
    for (int b = 0; b < batch; ++b)
        if (lens[b] < 0 || lens[b] > max_len) return -1;
    const bool f16 = kv_type == KVB_KV_F16, normal = dist == KVBH_NORMAL;
    const size_t D = size_t(head_dim), HD = size_t(num_heads) * D;

    for (int b = 0; b < batch; ++b) {
        std::mt19937_64 g = stream(seed, kQuery, uint64_t(b));
        float* qb = q + size_t(b) * HD;
        if (normal) {
            for (size_t i = 0; i < HD; i += 2) {
                float z0, z1;
                normal_pair(g(), g(), z0, z1);
                qb[i] = q_amp * z0;
                if (i + 1 < HD) qb[i + 1] = q_amp * z1;
            }
        } else {
            for (size_t i = 0; i < HD; ++i) qb[i] = q_amp * uniform_pm1(g());
        }
    }
    if (max_len == 0 || batch == 0) return 0;
    if (!k || !v) return -1;

    const size_t pairs = size_t(batch) * num_kv_heads, row_elems = size_t(max_len) * D;
    parallel_for(pairs, threads, [&](size_t pidx) {
        const int b = int(pidx / size_t(num_kv_heads));
        const int len = lens[b];
        std::mt19937_64 g = stream(seed, kKeyValue, pidx);
        std::mt19937_64 ga = stream(seed, kAmplitude, pidx);
        const size_t base = pidx * row_elems;
        float ak = 1.0f, av = 1.0f;
        for (int t = 0; t < max_len; ++t) {
            const bool live = t < len;
            if (live && varied && t % 16 == 0) {
                ak = std::exp2(-1.5f * (uniform_pm1(ga()) + 1.0f));
                av = std::exp2(-1.5f * (uniform_pm1(ga()) + 1.0f));
            }
            for (size_t d = 0; d < D; ++d) {
                float kf = 0.0f, vf = 0.0f;
                if (live) {
                    if (normal) normal_pair(g(), g(), kf, vf);
                    else kf = uniform_pm1(g()), vf = uniform_pm1(g());
                    kf *= ak;
                    vf *= av;
                }
                const size_t i = base + size_t(t) * D + d;
                if (f16) {
                    static_cast<kvb::half_t*>(k)[i] = kvb::half_t(kf);
                    static_cast<kvb::half_t*>(v)[i] = kvb::half_t(vf);
                } else {
                    static_cast<float*>(k)[i] = kf;
                    static_cast<float*>(v)[i] = vf;
                }
                if (k32) k32[i] = kf;
                if (v32) v32[i] = vf;
            }
        }
    });
    return 0;
}

int kvbh_layout_dims(const int* lens, int batch, int page_size, double pool_factor, int* max_blocks, int* live_blocks,
                     int* pool_blocks) {
    if (batch < 0 || (batch && !lens) || page_size <= 0 || !(pool_factor >= 1.0)) return -1;
    long long mx = 0, live = 0;
    for (int b = 0; b < batch; ++b) {
        if (lens[b] < 0) return -1;
        const long long blocks = ((long long)lens[b] + page_size - 1) / page_size;
        mx = std::max(mx, blocks);
        live += blocks;
    }
    const long long pool = std::max(live, (long long)std::ceil(double(live) * pool_factor));
    if (pool > 0x7fffffffLL) return -1;
    if (max_blocks) *max_blocks = int(mx);
    if (live_blocks) *live_blocks = int(live);
    if (pool_blocks) *pool_blocks = int(pool);
    return 0;
}

int kvbh_make_paged_layout(const int* lens, int batch, int page_size, double pool_factor, uint64_t seed,
                           int32_t* table) {
    if (batch < 0 || (batch && !lens)) return -1;
    return guarded([&] {
        const kvb::PagedLayout L =
            kvb::make_paged_layout(std::span<const int>(lens, size_t(batch)), page_size, seed, pool_factor);
        std::copy(L.block_table.begin(), L.block_table.end(), table);
    });
}

int kvbh_scatter_to_paged(int batch, int num_kv_heads, int head_dim, int page_size, int max_blocks,
                          const int32_t* table, const int* lens, int max_len, size_t elem_size, const void* contig,
                          void* paged) {
    if (batch < 0 || page_size <= 0 || (elem_size != 2 && elem_size != 4)) return -1;
    return guarded([&] {
        const kvb::Shape s = shape(batch, num_kv_heads, num_kv_heads, head_dim);
        const kvb::PagedLayout L = layout_view(page_size, max_blocks, 0, table, batch);
        const std::span<const int> ls(lens, size_t(batch));
        if (elem_size == 4)
            kvb::scatter_to_paged<float>(s, L, ls, max_len, static_cast<const float*>(contig), static_cast<float*>(paged));
        else
            kvb::scatter_to_paged<uint16_t>(s, L, ls, max_len, static_cast<const uint16_t*>(contig),
                                            static_cast<uint16_t*>(paged));
    });
}

int kvbh_quantize_to_paged_i8(int batch, int num_kv_heads, int head_dim, int page_size, int max_blocks,
                              const int32_t* table, const int* lens, int max_len, const float* contig, int8_t* paged,
                              float* scales) {
    if (batch < 0 || page_size <= 0) return -1;
    return guarded([&] {
        kvb::quantize_to_paged_i8(shape(batch, num_kv_heads, num_kv_heads, head_dim),
                                  layout_view(page_size, max_blocks, 0, table, batch),
                                  std::span<const int>(lens, size_t(batch)), max_len, contig, paged, scales);
    });
}

int kvbh_dequantize_paged_i8(int batch, int num_kv_heads, int head_dim, int page_size, int max_blocks,
                             const int32_t* table, const int* lens, int max_len, const int8_t* paged,
                             const float* scales, float* contig) {
    if (batch < 0 || page_size <= 0) return -1;
    return guarded([&] {
        kvb::dequantize_paged_i8(shape(batch, num_kv_heads, num_kv_heads, head_dim),
                                 layout_view(page_size, max_blocks, 0, table, batch),
                                 std::span<const int>(lens, size_t(batch)), max_len, paged, scales, contig);
    });
}

int kvbh_poison_paged(int batch, int num_kv_heads, int head_dim, int page_size, int max_blocks, int pool_blocks,
                      const int32_t* table, const int* lens, size_t elem_size, void* paged, float* scales) {
    if (batch < 0 || page_size <= 0 || pool_blocks < 0) return -1;
    return guarded([&] {
        kvb::poison_paged(shape(batch, num_kv_heads, num_kv_heads, head_dim),
                          layout_view(page_size, max_blocks, pool_blocks, table, batch),
                          std::span<const int>(lens, size_t(batch)), elem_size, paged, scales);
    });
}

int kvbh_mi355x_part_tokens_lens(int batch, int num_heads, int num_kv_heads, int head_dim, const int* lens,
                                 int min_groups, int min_part, int max_part) {
    if (batch < 0 || (batch > 0 && !lens) || num_heads <= 0 || num_kv_heads <= 0 || min_part <= 0 || max_part < min_part)
        return -1;
    return kvb::mi355x_part_tokens(shape(batch, num_heads, num_kv_heads, head_dim), std::span<const int>(lens, size_t(batch)),
                                   min_groups, min_part, max_part);
}

int kvbh_mi355x_part_tokens(int batch, int num_heads, int num_kv_heads, int head_dim, int max_len, int min_groups,
                            int min_part, int max_part) {
    if (batch < 0 || num_heads <= 0 || num_kv_heads <= 0 || min_part <= 0 || max_part < min_part) return -1;
    return kvb::mi355x_part_tokens(shape(batch, num_heads, num_kv_heads, head_dim), max_len, min_groups, min_part,
                                   max_part);
}

}  // extern "C"
