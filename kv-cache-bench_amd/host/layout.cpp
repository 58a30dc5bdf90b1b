// Paged layout, int8 quantiser and pool poisoning of the host layer (src/reference.cpp:11-63).
#include "kvb/layout.hpp"

#include <algorithm>
#include <cstring>
#include <numeric>
#include <stdexcept>

#include "kvb/rng.hpp"

namespace kvb {

PagedLayout make_paged_layout(std::span<const int> seq_lens, int page_size, uint64_t seed, double pool_factor) {
    if (page_size <= 0) throw std::invalid_argument("make_paged_layout: page_size <= 0");
    if (!(pool_factor >= 1.0)) throw std::invalid_argument("make_paged_layout: pool_factor < 1");
    PagedLayout L;
    L.page_size = page_size;
    long long live = 0;
    for (int len : seq_lens) {
        if (len < 0) throw std::invalid_argument("make_paged_layout: negative length");
        const int blocks = (len + page_size - 1) / page_size;
        L.max_blocks = std::max(L.max_blocks, blocks);
        live += blocks;
    }
    const long long pool = std::max(live, (long long)std::ceil(double(live) * pool_factor));
    if (pool > 0x7fffffffLL) throw std::invalid_argument("make_paged_layout: pool larger than 2^31 blocks");
    L.live_blocks = int(live);
    L.num_blocks = int(pool);

    std::vector<int32_t> phys(static_cast<size_t>(pool));
    std::iota(phys.begin(), phys.end(), 0);
    std::mt19937_64 g(seed);
    for (long long i = pool - 1; i > 0; --i) std::swap(phys[size_t(i)], phys[rng::below(g(), uint64_t(i) + 1)]);

    // the shuffled ids are handed out in sequence order, a run of ceil(len / page) per sequence
    L.block_table.assign(seq_lens.size() * size_t(L.max_blocks), -1);
    auto next = phys.cbegin();
    for (size_t b = 0; b < seq_lens.size(); ++b) {
        const auto run = (seq_lens[b] + page_size - 1) / page_size;
        std::copy(next, next + run, L.block_table.begin() + std::ptrdiff_t(b * size_t(L.max_blocks)));
        next += run;
    }
    return L;
}

namespace {

// The reference's rounding of one value (src/reference.cpp:44-47): IEEE division, round half to
// even, clamp to +-127; a zero scale (an all-zero slice) stores 0.
int8_t quantize_one(float x, float scale) {
    return scale > 0 ? int8_t(std::clamp(std::nearbyint(x / scale), -127.0f, 127.0f)) : int8_t(0);
}

// max |x| over a slice; a NaN never becomes the running value (std::max keeps its first argument).
float slice_amax(std::span<const float> x) {
    return std::accumulate(x.begin(), x.end(), 0.0f, [](float m, float v) { return std::max(m, std::fabs(v)); });
}

}  // namespace

void quantize_to_paged_i8(const Shape& s, const PagedLayout& L, std::span<const int> seq_lens, int max_len,
                          const float* contig, int8_t* paged, float* scales) {
    for_each_page_slice(s, L, seq_lens, [&](const PageSlice& p) {
        const std::span<const float> x(contig + p.contig_at(s, max_len), p.elems(s));
        const float scale = slice_amax(x) / 127.0f;
        scales[size_t(p.block) * s.num_kv_heads + p.kvh] = scale;
        std::transform(x.begin(), x.end(), paged + p.paged_at(s, L), [scale](float v) { return quantize_one(v, scale); });
    });
}

void dequantize_paged_i8(const Shape& s, const PagedLayout& L, std::span<const int> seq_lens, int max_len,
                         const int8_t* paged, const float* scales, float* contig) {
    for_each_page_slice(s, L, seq_lens, [&](const PageSlice& p) {
        const float scale = scales[size_t(p.block) * s.num_kv_heads + p.kvh];
        const int8_t* q = paged + p.paged_at(s, L);
        std::transform(q, q + p.elems(s), contig + p.contig_at(s, max_len), [scale](int8_t v) { return float(v) * scale; });
    });
}

void poison_paged(const Shape& s, const PagedLayout& L, std::span<const int> seq_lens, size_t elem_size, void* paged,
                  float* scales) {
    if (elem_size != 1 && elem_size != 2 && elem_size != 4) throw std::invalid_argument("poison_paged: elem_size");
    // live rows of every physical block; unused blocks keep 0
    std::vector<int> live_rows(size_t(L.num_blocks), 0);
    for (size_t b = 0; b < seq_lens.size(); ++b)
        for (int i = 0; i * L.page_size < seq_lens[b]; ++i)
            live_rows[size_t(L.block_table[b * L.max_blocks + i])] = std::min(L.page_size, seq_lens[b] - i * L.page_size);
    const size_t row_elems = size_t(s.head_dim);
    unsigned char* base = static_cast<unsigned char*>(paged);
    const uint32_t nan32 = 0x7fc00000u;
    const uint16_t nan16 = 0x7e00u;
    const float fnan = std::numeric_limits<float>::quiet_NaN();
    for (int blk = 0; blk < L.num_blocks; ++blk)
        for (int kvh = 0; kvh < s.num_kv_heads; ++kvh) {
            if (live_rows[size_t(blk)] == 0 && scales) scales[size_t(blk) * s.num_kv_heads + kvh] = fnan;
            for (int r = live_rows[size_t(blk)]; r < L.page_size; ++r) {
                unsigned char* row = base + ((size_t(blk) * s.num_kv_heads + kvh) * L.page_size + r) * row_elems * elem_size;
                if (elem_size == 1) std::memset(row, 0x80, row_elems);
                else if (elem_size == 2)
                    for (size_t d = 0; d < row_elems; ++d) std::memcpy(row + 2 * d, &nan16, 2);
                else
                    for (size_t d = 0; d < row_elems; ++d) std::memcpy(row + 4 * d, &nan32, 4);
            }
        }
}

}  // namespace kvb
