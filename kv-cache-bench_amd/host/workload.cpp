// Workload and PagedCache (src/workload.hpp:26-146) over the host layer's generator and cache writers.
#include "kvb/workload.hpp"

#include <algorithm>
#include <cstring>
#include <stdexcept>

#include "kvb_host.h"

namespace kvb {

Workload::Workload(Shape s, KvType t, std::vector<int> lens_, uint64_t seed, float q_amp, bool keep_f32, bool varied,
                   Dist dist)
    : shape(s), type(t), lens(std::move(lens_)), max_len(lens.empty() ? 0 : *std::max_element(lens.begin(), lens.end())) {
    shape.batch = int(lens.size());
    const size_t nq = size_t(shape.batch) * shape.num_heads * shape.head_dim;
    const size_t nkv = size_t(shape.batch) * shape.num_kv_heads * max_len * shape.head_dim;
    q = std::make_unique<Buffer>(nq * sizeof(float));
    seq_lens = std::make_unique<Buffer>(lens.size() * sizeof(int));
    std::copy(lens.begin(), lens.end(), seq_lens->as<int>());
    with_type(t, [&]<class T>(T) {
        k = std::make_unique<Buffer>(nkv * sizeof(T));
        v = std::make_unique<Buffer>(nkv * sizeof(T));
    });
    if (keep_f32) k32.resize(nkv), v32.resize(nkv);
    const int c_type = t == KvType::f32 ? KVB_KV_F32 : t == KvType::f16 ? KVB_KV_F16 : KVB_KV_I8;
    if (kvbh_fill_workload(shape.batch, shape.num_heads, shape.num_kv_heads, shape.head_dim, lens.data(), max_len,
                           c_type, seed, q_amp, varied ? 1 : 0, dist == Dist::normal ? KVBH_NORMAL : KVBH_UNIFORM,
                           q->as<float>(), k->data(), v->data(), keep_f32 ? k32.data() : nullptr,
                           keep_f32 ? v32.data() : nullptr, 0) != 0)
        throw std::invalid_argument("Workload: bad shape or lengths");
}

double Workload::min_bytes() const {
    size_t tokens = 0;
    for (int l : lens) tokens += size_t(l);
    return double(tokens) * shape.num_kv_heads * shape.head_dim * 2 * elem_size(type) +
           double(out_floats()) * 2 * sizeof(float);
}

NaiveArgs Workload::naive_args(const Buffer& out) const {
    return {shape, type, max_len, q.get(), k.get(), v.get(), seq_lens.get(), &out};
}

PagedCache::PagedCache(const Workload& w, int page_size, uint64_t seed, bool contiguous, double pool_factor, bool poison) {
    if (contiguous) {
        layout.page_size = std::max(w.max_len, 1);
        layout.max_blocks = 1;
        layout.num_blocks = w.shape.batch;
        layout.live_blocks = w.shape.batch;
        for (int b = 0; b < w.shape.batch; ++b) layout.block_table.push_back(b);
    } else {
        layout = make_paged_layout(w.lens, page_size, seed, pool_factor);
    }
    const Shape& s = w.shape;
    const size_t n = size_t(layout.num_blocks) * s.num_kv_heads * layout.page_size * s.head_dim;
    const size_t esz = elem_size(w.type);
    k = std::make_unique<Buffer>(n * esz);
    v = std::make_unique<Buffer>(n * esz);
    table = std::make_unique<Buffer>(layout.block_table.size() * sizeof(int32_t));
    std::copy(layout.block_table.begin(), layout.block_table.end(), table->as<int32_t>());
    const bool i8 = w.type == KvType::i8;
    if (i8) {
        const size_t ns = size_t(layout.num_blocks) * s.num_kv_heads;
        k_scale = std::make_unique<Buffer>(ns * sizeof(float));
        v_scale = std::make_unique<Buffer>(ns * sizeof(float));
    }
    if (poison) {
        poison_paged(s, layout, w.lens, esz, k->data(), i8 ? k_scale->as<float>() : nullptr);
        poison_paged(s, layout, w.lens, esz, v->data(), i8 ? v_scale->as<float>() : nullptr);
    }
    if (i8) {
        quantize_to_paged_i8(s, layout, w.lens, w.max_len, static_cast<const float*>(w.k->host()), k->as<int8_t>(),
                             k_scale->as<float>());
        quantize_to_paged_i8(s, layout, w.lens, w.max_len, static_cast<const float*>(w.v->host()), v->as<int8_t>(),
                             v_scale->as<float>());
        return;
    }
    with_type(w.type, [&]<class T>(T) {
        scatter_to_paged<T>(s, layout, w.lens, w.max_len, static_cast<const T*>(w.k->host()), k->as<T>());
        scatter_to_paged<T>(s, layout, w.lens, w.max_len, static_cast<const T*>(w.v->host()), v->as<T>());
    });
}

size_t PagedCache::bytes() const { return k->size() + v->size() + (k_scale ? k_scale->size() + v_scale->size() : 0); }

double PagedCache::scale_bytes(const Workload& w) const {
    if (!k_scale) return 0;
    size_t blocks = 0;
    for (int l : w.lens) blocks += size_t((l + layout.page_size - 1) / layout.page_size);
    return double(blocks) * w.shape.num_kv_heads * 2 * sizeof(float);
}

PagedArgs PagedCache::args(const Workload& w, int part_tokens, const Buffer& out) const {
    PagedArgs a{w.shape, w.type, layout.page_size, layout.max_blocks, w.max_len, part_tokens,
                w.q.get(), k.get(), v.get(), table.get(), w.seq_lens.get(), &out};
    a.k_scale = k_scale.get();
    a.v_scale = v_scale.get();
    return a;
}

}  // namespace kvb
