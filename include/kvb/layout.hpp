// Shapes, the paged block table and the cache writers of the host layer (the layout half of the
// reference's src/reference.hpp:11-81). The fp64 attention reference of that file is declared in
// kvb/reference.hpp and defined by the reference's own CPU code, not by this build's libraries.
#pragma once

#include <algorithm>
#include <cmath>
#include <cstddef>
#include <cstdint>
#include <span>
#include <vector>

namespace kvb {

using half_t = _Float16;

// One decode step: every sequence has one new query token per query head and attends to its
// whole KV history. Query head h reads KV head h / group() (src/reference.hpp:15-23).
struct Shape {
    int batch = 1;
    int num_heads = 32;    // query heads, H
    int num_kv_heads = 8;  // KV heads, Hkv; H % Hkv == 0
    int head_dim = 128;    // D
    int group() const { return num_heads / num_kv_heads; }
};

// max |a[i] - b[i]| in fp64, +inf if any difference is NaN (src/reference.hpp:25-35): a plain
// maximum would call an output full of NaN equal to anything.
inline double max_abs_diff(const float* a, const float* b, size_t n) {
    double m = 0;
    for (size_t i = 0; i < n; ++i) {
        const double e = std::fabs(double(a[i]) - double(b[i]));
        if (std::isnan(e)) return INFINITY;
        m = std::max(m, e);
    }
    return m;
}

// Contiguous cache layout [B][Hkv][max_len][D] (src/reference.hpp:37-40).
inline size_t contig_index(const Shape& s, int max_len, int b, int kvh, int t, int d) {
    return ((size_t(b) * s.num_kv_heads + kvh) * max_len + t) * s.head_dim + d;
}

// Paged cache: a pool of physical blocks, each [Hkv][page_size][D]; logical block i of sequence b
// lives in physical block block_table[b * max_blocks + i] (src/reference.hpp:42-58).
struct PagedLayout {
    int page_size = 16;
    int max_blocks = 0;   // row stride of block_table
    int num_blocks = 0;   // physical blocks in the pool (live + unused)
    std::vector<int32_t> block_table;
    int live_blocks = 0;  // blocks some sequence uses; num_blocks - live_blocks are never read
};

// Assigns physical blocks in a shuffled order so the kernel cannot rely on logically adjacent
// blocks being adjacent in memory (src/reference.cpp:11-30). The pool holds
// ceil(live * pool_factor) blocks (pool_factor 1 is the reference's exact pool); ids 0..pool-1 are
// shuffled by Fisher-Yates driven by std::mt19937_64(seed) (for i = pool-1..1: swap(i, j) with
// j = (draw * (i+1)) >> 64), and handed out in sequence order. Unused table entries are -1; an
// empty sequence takes no block. The reference's std::shuffle stream is implementation-defined, so
// this explicit one keeps tables identical on every standard library.
PagedLayout make_paged_layout(std::span<const int> seq_lens, int page_size, uint64_t seed, double pool_factor = 1.0);

inline size_t paged_index(const Shape& s, const PagedLayout& L, int b, int kvh, int t, int d) {
    const size_t blk = size_t(L.block_table[size_t(b) * L.max_blocks + t / L.page_size]);
    return ((blk * s.num_kv_heads + kvh) * L.page_size + t % L.page_size) * s.head_dim + d;
}

// One page of one KV head of one sequence: the `rows` live tokens from token t0 of sequence b (t0 a
// multiple of the page size), held in physical block `block`. Its rows are one contiguous run in both
// layouts: from contig_index(b, kvh, t0, 0) in the contiguous cache, from row 0 of (block, kvh) in the
// pool. The cache writers below work slice by slice.
struct PageSlice {
    int b, kvh, t0, rows;
    int32_t block;
    size_t elems(const Shape& s) const { return size_t(rows) * s.head_dim; }
    size_t contig_at(const Shape& s, int max_len) const { return contig_index(s, max_len, b, kvh, t0, 0); }
    size_t paged_at(const Shape& s, const PagedLayout& L) const {
        return (size_t(block) * s.num_kv_heads + kvh) * L.page_size * s.head_dim;
    }
};

// Calls fn(PageSlice) for every live (sequence, logical block, KV head), sequences in order.
template <class Fn>
void for_each_page_slice(const Shape& s, const PagedLayout& L, std::span<const int> seq_lens, Fn&& fn) {
    for (int b = 0; b < s.batch; ++b) {
        const int32_t* blocks = L.block_table.data() + size_t(b) * L.max_blocks;
        for (int t0 = 0; t0 < seq_lens[b]; t0 += L.page_size) {
            const int rows = std::min(L.page_size, seq_lens[b] - t0);
            for (int kvh = 0; kvh < s.num_kv_heads; ++kvh) fn(PageSlice{b, kvh, t0, rows, blocks[t0 / L.page_size]});
        }
    }
}

// Copies every live token of the contiguous cache into the pool (src/reference.hpp:60-68).
template <class T>
void scatter_to_paged(const Shape& s, const PagedLayout& L, std::span<const int> seq_lens, int max_len,
                      const T* contig, T* paged) {
    for_each_page_slice(s, L, seq_lens, [&](const PageSlice& p) {
        std::copy_n(contig + p.contig_at(s, max_len), p.elems(s), paged + p.paged_at(s, L));
    });
}

// int8 storage: the live page_size x D values of one (physical block, KV head) become int8 with one
// fp32 scale max|x| / 127, q = clamp(nearbyint(x / scale), -127, 127) (0 if the scale is 0), so
// x ~= q * scale within scale / 2 (src/reference.cpp:32-51). scales is [num_blocks][Hkv].
void quantize_to_paged_i8(const Shape& s, const PagedLayout& L, std::span<const int> seq_lens, int max_len,
                          const float* contig, int8_t* paged, float* scales);

// The values the kernel computes with for an int8 cache: float(q) * scale on live tokens, in the
// contiguous layout (src/reference.cpp:53-63).
void dequantize_paged_i8(const Shape& s, const PagedLayout& L, std::span<const int> seq_lens, int max_len,
                         const int8_t* paged, const float* scales, float* contig);

// Marks every pool element no live token owns -- unused blocks, and rows past a sequence's length in
// its last block -- so a kernel that reads one shows it: NaN for f32/f16 (elem_size 4/2); for int8
// (elem_size 1) the byte -128, which the quantiser never writes, and a NaN scale for unused blocks.
void poison_paged(const Shape& s, const PagedLayout& L, std::span<const int> seq_lens, size_t elem_size, void* paged,
                  float* scales);

}  // namespace kvb
