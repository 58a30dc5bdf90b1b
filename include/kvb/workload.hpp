// Random decode workloads shared by the tests and the benchmark (the reference's src/workload.hpp).
#pragma once

#include <cmath>
#include <cstdint>
#include <memory>
#include <vector>

#include "kvb/hip_attn.hpp"

namespace kvb {

// Calls f with a value of the contiguous cache's element type: half for f16, float otherwise (an
// i8 workload keeps its unquantised fp32 values; PagedCache quantises them per block).
template <class F>
void with_type(KvType t, F&& f) {
    if (t == KvType::f16) f(half_t{});
    else f(float{});
}

// Value distribution. uniform: q ~ q_amp * U(-1, 1), K and V ~ U(-1, 1) (the reference's,
// src/workload.hpp:21-25). normal: q ~ q_amp * N(0, 1), K and V ~ N(0, 1) (the BASELINE configs).
enum class Dist { uniform, normal };

// Stream layout (rng.hpp): q of sequence b comes from stream (seed, kQuery, b); K and V of
// (b, kvh) from stream (seed, kKeyValue, b * Hkv + kvh), drawn token by token, K element then V
// element; with `varied`, every 16-token chunk of a (b, kvh) scales its K and its V by factors
// 2^-U(0,3) from stream (seed, kAmplitude, b * Hkv + kvh), so blocks and heads differ in magnitude
// and an int8 scale applied to the wrong block or head shows (src/workload.hpp:21-25, 46-49).
// Rows past a sequence's length are 0.
struct Workload {
    Shape shape;
    KvType type;
    std::vector<int> lens;
    int max_len;
    std::unique_ptr<Buffer> q, k, v, seq_lens;  // k, v: contiguous [B][Hkv][max_len][D] (with_type)
    std::vector<float> k32, v32;                // fp32 originals, kept only if asked (fp16 checks)

    Workload(Shape s, KvType t, std::vector<int> lens, uint64_t seed, float q_amp, bool keep_f32 = false,
             bool varied = false, Dist dist = Dist::uniform);

    size_t out_floats() const { return size_t(shape.batch) * shape.num_heads * shape.head_dim; }

    // Bytes a decode step must move at minimum: K and V of every live token, q and out
    // (src/workload.hpp:68-74; int8 scales not included).
    double min_bytes() const;

    // Fills `out` (out_floats() floats) with the fp64 attention reference on the contiguous cache:
    // the stored fp16 values for f16, the unquantised fp32 values for f32 and i8
    // (src/workload.hpp:76-83). attention_reference is the reference's own CPU code, linked by the
    // caller (kvb/reference.hpp); nothing in this build's libraries calls this.
    void reference(float* out, int threads = 1) const {
        with_type(type, [&]<class T>(T) {
            attention_reference<T>(shape, lens, max_len, static_cast<const float*>(q->host()),
                                   static_cast<const T*>(k->host()), static_cast<const T*>(v->host()), out,
                                   1.0f / std::sqrt(float(shape.head_dim)), threads);
        });
    }

    NaiveArgs naive_args(const Buffer& out) const;
};

// The workload's cache in the paged layout, in a shuffled block order; for i8, quantised per
// (block, KV head). With `contiguous`, one block per sequence in order (page = max_len), the
// layout [B][Hkv][max_len][D] of a plain contiguous cache read by the same kernel. pool_factor
// oversizes the pool (ceil(live * factor) blocks, the unused ones shuffled in among the live
// ones); with `poison` every element no live token owns is poisoned (poison_paged), so a kernel
// that reads one fails its test (src/workload.hpp:90-146).
struct PagedCache {
    PagedLayout layout;
    std::unique_ptr<Buffer> k, v, table, k_scale, v_scale;  // scales: i8 only

    PagedCache(const Workload& w, int page_size, uint64_t seed, bool contiguous = false, double pool_factor = 1.0,
               bool poison = true);

    // Bytes of the K and V pools, scales included.
    size_t bytes() const;
    // Bytes of the int8 scales of live blocks a decode step reads (0 for f32/f16).
    double scale_bytes(const Workload& w) const;

    // fp64 reference on the values the kernel reads: the dequantised cache for i8, otherwise
    // Workload::reference (src/workload.hpp:128-137).
    void reference(const Workload& w, float* out, int threads = 1) const {
        if (w.type != KvType::i8) return w.reference(out, threads);
        std::vector<float> kd(w.k->size() / sizeof(float)), vd(kd.size());
        dequantize_paged_i8(w.shape, layout, w.lens, w.max_len, static_cast<const int8_t*>(k->host()),
                            static_cast<const float*>(k_scale->host()), kd.data());
        dequantize_paged_i8(w.shape, layout, w.lens, w.max_len, static_cast<const int8_t*>(v->host()),
                            static_cast<const float*>(v_scale->host()), vd.data());
        attention_reference<float>(w.shape, w.lens, w.max_len, static_cast<const float*>(w.q->host()), kd.data(),
                                   vd.data(), out, 1.0f / std::sqrt(float(w.shape.head_dim)), threads);
    }

    PagedArgs args(const Workload& w, int part_tokens, const Buffer& out) const;
};

}  // namespace kvb
