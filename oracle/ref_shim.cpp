// ref_shim.cpp -- TEST INFRASTRUCTURE ONLY. C entry points over the reference's own CPU code
// (chipontix/kv-cache-bench src/reference.cpp and the inline auto_part_tokens of
// src/metal_attn.hpp:47-51), compiled from the sources where they lie under /root/reference by
// oracle/Makefile into oracle/_ref/libkvbref.so. Used only by tests/ (to pin the C oracle) and by
// bench.py's cpu_baseline leg (to time the reference's own fp64 path).
#include <cstdint>
#include <cstring>
#include <span>
#include <vector>

#include "metal_attn.hpp"  // declarations only: Buffer & co are never defined or called here
#include "reference.hpp"

using kvb::half_t;

namespace {
kvb::Shape shape(int B, int H, int Hkv, int D) { return kvb::Shape{B, H, Hkv, D}; }
kvb::PagedLayout layout(int page, int max_blocks, int num_blocks, const int32_t* table, int B) {
    kvb::PagedLayout L;
    L.page_size = page;
    L.max_blocks = max_blocks;
    L.num_blocks = num_blocks;
    L.block_table.assign(table, table + size_t(B) * max_blocks);
    return L;
}
}  // namespace

extern "C" {

void kvbref_attention_f32(int B, int H, int Hkv, int D, const int* lens, int max_len, const float* q,
                          const float* k, const float* v, float* out, float scale, int threads) {
    kvb::attention_reference<float>(shape(B, H, Hkv, D), std::span<const int>(lens, size_t(B)), max_len, q, k, v,
                                    out, scale, threads);
}

void kvbref_attention_f16(int B, int H, int Hkv, int D, const int* lens, int max_len, const float* q,
                          const uint16_t* k, const uint16_t* v, float* out, float scale, int threads) {
    static_assert(sizeof(half_t) == sizeof(uint16_t));
    kvb::attention_reference<half_t>(shape(B, H, Hkv, D), std::span<const int>(lens, size_t(B)), max_len, q,
                                     reinterpret_cast<const half_t*>(k), reinterpret_cast<const half_t*>(v), out,
                                     scale, threads);
}

// Returns num_blocks; fills max_blocks and, if table_cap is large enough, the table.
int kvbref_make_paged_layout(const int* lens, int B, int page, uint64_t seed, int32_t* table, size_t table_cap,
                             int* max_blocks) {
    const kvb::PagedLayout L = kvb::make_paged_layout(std::span<const int>(lens, size_t(B)), page, seed);
    *max_blocks = L.max_blocks;
    if (table && L.block_table.size() <= table_cap)
        std::memcpy(table, L.block_table.data(), L.block_table.size() * sizeof(int32_t));
    return L.num_blocks;
}

void kvbref_quantize_to_paged_i8(int B, int H, int Hkv, int D, int page, int max_blocks, int num_blocks,
                                 const int32_t* table, const int* lens, int max_len, const float* contig,
                                 int8_t* paged, float* scales) {
    kvb::quantize_to_paged_i8(shape(B, H, Hkv, D), layout(page, max_blocks, num_blocks, table, B),
                              std::span<const int>(lens, size_t(B)), max_len, contig, paged, scales);
}

void kvbref_dequantize_paged_i8(int B, int H, int Hkv, int D, int page, int max_blocks, int num_blocks,
                                const int32_t* table, const int* lens, int max_len, const int8_t* paged,
                                const float* scales, float* contig) {
    kvb::dequantize_paged_i8(shape(B, H, Hkv, D), layout(page, max_blocks, num_blocks, table, B),
                             std::span<const int>(lens, size_t(B)), max_len, paged, scales, contig);
}

void kvbref_scatter_to_paged_f32(int B, int H, int Hkv, int D, int page, int max_blocks, int num_blocks,
                                 const int32_t* table, const int* lens, int max_len, const float* contig,
                                 float* paged) {
    kvb::scatter_to_paged<float>(shape(B, H, Hkv, D), layout(page, max_blocks, num_blocks, table, B),
                                 std::span<const int>(lens, size_t(B)), max_len, contig, paged);
}

double kvbref_max_abs_diff(const float* a, const float* b, size_t n) { return kvb::max_abs_diff(a, b, n); }

int kvbref_auto_part_tokens(int B, int H, int Hkv, int D, int max_len) {
    return kvb::auto_part_tokens(shape(B, H, Hkv, D), max_len);
}

}  // extern "C"
