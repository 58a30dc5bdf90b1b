// Shared helpers of the C++ test programs: the fp64 oracle (oracle/kvb_oracle.h, test
// infrastructure) applied to the host layer's workloads, and the tolerance of the reference's tests.
#pragma once

#include <cmath>
#include <cstdio>
#include <thread>
#include <vector>

#include "kvb/workload.hpp"
#include "kvb_oracle.h"

namespace kvbt {

using namespace kvb;

// Kernel vs oracle on the same stored values (tests/gpu_tests.cpp:13-17, for |v| <= 1). For data
// with larger |v| (the N(0,1) configs) it scales with max|v|: the output is a convex combination of
// V rows and every error term of the argument is relative to |v|.
constexpr double kTolKernel = 2e-5;

inline int hw_threads() { return int(std::max(1u, std::min(16u, std::thread::hardware_concurrency()))); }

inline kvbo_shape oshape(const Shape& s) { return kvbo_shape{s.batch, s.num_heads, s.num_kv_heads, s.head_dim}; }

inline float softmax_scale(const Shape& s) { return 1.0f / std::sqrt(float(s.head_dim)); }

// fp64 oracle on the workload's contiguous cache: the stored fp16 values for f16, the fp32 values
// (unquantised) for f32 and i8 (Workload::reference, src/workload.hpp:76-83).
inline void reference(const Workload& w, float* out, int threads = 1) {
    const kvbo_shape s = oshape(w.shape);
    const float* q = static_cast<const float*>(w.q->host());
    if (w.type == KvType::f16)
        kvbo_attention_f16(&s, w.lens.data(), w.max_len, q, static_cast<const uint16_t*>(w.k->host()),
                           static_cast<const uint16_t*>(w.v->host()), out, softmax_scale(w.shape), threads);
    else
        kvbo_attention_f32(&s, w.lens.data(), w.max_len, q, static_cast<const float*>(w.k->host()),
                           static_cast<const float*>(w.v->host()), out, softmax_scale(w.shape), threads);
}

// The oracle's dequantised contiguous copy of an int8 cache (zeros past each length).
inline void dequantized(const Workload& w, const PagedCache& c, std::vector<float>& kd, std::vector<float>& vd) {
    const kvbo_shape s = oshape(w.shape);
    const size_t n = size_t(w.shape.batch) * w.shape.num_kv_heads * w.max_len * w.shape.head_dim;
    kd.assign(n, 0.0f);
    vd.assign(n, 0.0f);
    const int32_t* table = static_cast<const int32_t*>(c.table->host());
    kvbo_dequantize_paged_i8(&s, c.layout.page_size, c.layout.max_blocks, table, w.lens.data(), w.max_len,
                             static_cast<const int8_t*>(c.k->host()), static_cast<const float*>(c.k_scale->host()),
                             kd.data());
    kvbo_dequantize_paged_i8(&s, c.layout.page_size, c.layout.max_blocks, table, w.lens.data(), w.max_len,
                             static_cast<const int8_t*>(c.v->host()), static_cast<const float*>(c.v_scale->host()),
                             vd.data());
}

// fp64 oracle on the values the kernel reads: the dequantised cache for i8, otherwise reference()
// (PagedCache::reference, src/workload.hpp:128-137).
inline void paged_reference(const Workload& w, const PagedCache& c, float* out, int threads = 1) {
    if (w.type != KvType::i8) return reference(w, out, threads);
    std::vector<float> kd, vd;
    dequantized(w, c, kd, vd);
    const kvbo_shape s = oshape(w.shape);
    kvbo_attention_f32(&s, w.lens.data(), w.max_len, static_cast<const float*>(w.q->host()), kd.data(), vd.data(), out,
                       softmax_scale(w.shape), threads);
}

// max |v| over the live V values the kernel reads (1 for the reference's U(-1,1) data or less).
inline double vmax_live(const Workload& w, const PagedCache* c = nullptr) {
    std::vector<float> kd, vd;
    const float* v32 = nullptr;
    std::vector<float> tmp;
    if (w.type == KvType::i8 && c) {
        dequantized(w, *c, kd, vd);
        v32 = vd.data();
    } else if (w.type == KvType::f16) {
        const size_t n = w.v->size() / 2;
        tmp.resize(n);
        const uint16_t* h = static_cast<const uint16_t*>(w.v->host());
        for (size_t i = 0; i < n; ++i) tmp[i] = kvbo_f16_to_f32(h[i]);
        v32 = tmp.data();
    } else {
        v32 = static_cast<const float*>(w.v->host());
    }
    double m = 0;
    const Shape& s = w.shape;
    for (int b = 0; b < s.batch; ++b)
        for (int kvh = 0; kvh < s.num_kv_heads; ++kvh)
            for (int t = 0; t < w.lens[b]; ++t)
                for (int d = 0; d < s.head_dim; ++d)
                    m = std::max(m, double(std::fabs(v32[contig_index(s, w.max_len, b, kvh, t, d)])));
    return m;
}

// The kernel tolerance for this workload: 2e-5 * max(1, max|v|).
inline double kernel_tol(const Workload& w, const PagedCache* c = nullptr) {
    return kTolKernel * std::max(1.0, vmax_live(w, c));
}

}  // namespace kvbt
