// Paged layout, int8 quantiser and pool poisoning of the host layer (src/reference.cpp:11-63).
#include "kvb/layout.hpp"

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

    L.block_table.assign(seq_lens.size() * size_t(L.max_blocks), -1);
    size_t next = 0;
    for (size_t b = 0; b < seq_lens.size(); ++b) {
        const int blocks = (seq_lens[b] + page_size - 1) / page_size;
        for (int i = 0; i < blocks; ++i) L.block_table[b * L.max_blocks + i] = phys[next++];
    }
    return L;
}

void quantize_to_paged_i8(const Shape& s, const PagedLayout& L, std::span<const int> seq_lens, int max_len,
                          const float* contig, int8_t* paged, float* scales) {
    const int P = L.page_size, D = s.head_dim;
    for (int b = 0; b < s.batch; ++b)
        for (int i = 0; i * P < seq_lens[b]; ++i)
            for (int kvh = 0; kvh < s.num_kv_heads; ++kvh) {
                const int t0 = i * P, t1 = std::min(seq_lens[b], t0 + P);
                float amax = 0;
                for (int t = t0; t < t1; ++t) {
                    const float* row = contig + contig_index(s, max_len, b, kvh, t, 0);
                    for (int d = 0; d < D; ++d) amax = std::max(amax, std::fabs(row[d]));
                }
                const float scale = amax / 127.0f;
                scales[size_t(L.block_table[size_t(b) * L.max_blocks + i]) * s.num_kv_heads + kvh] = scale;
                for (int t = t0; t < t1; ++t) {
                    const float* row = contig + contig_index(s, max_len, b, kvh, t, 0);
                    int8_t* dst = paged + paged_index(s, L, b, kvh, t, 0);
                    for (int d = 0; d < D; ++d)
                        dst[d] = scale > 0 ? int8_t(std::clamp(std::nearbyint(row[d] / scale), -127.0f, 127.0f)) : 0;
                }
            }
}

void dequantize_paged_i8(const Shape& s, const PagedLayout& L, std::span<const int> seq_lens, int max_len,
                         const int8_t* paged, const float* scales, float* contig) {
    for (int b = 0; b < s.batch; ++b)
        for (int kvh = 0; kvh < s.num_kv_heads; ++kvh)
            for (int t = 0; t < seq_lens[b]; ++t) {
                const float scale =
                    scales[size_t(L.block_table[size_t(b) * L.max_blocks + t / L.page_size]) * s.num_kv_heads + kvh];
                const int8_t* src = paged + paged_index(s, L, b, kvh, t, 0);
                float* dst = contig + contig_index(s, max_len, b, kvh, t, 0);
                for (int d = 0; d < s.head_dim; ++d) dst[d] = float(src[d]) * scale;
            }
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
