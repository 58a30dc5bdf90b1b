// paged_reduce, the naive three-pass baseline, the read-bandwidth probe and the cache-flush fill.
#include <type_traits>

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include "kvb_kernels.hpp"

namespace kvbk {
namespace {

constexpr float kNegBigR = -1e30f;

// Merges the partitions of one (sequence, query head) (src/kernels.metal:123-147): weights
// l_i * exp(m_i - M) over the ceil(len / part) written slots; an empty sequence gives exactly 0, and
// a sequence of one partition takes that partition's output as it is.
// Grid (H, B), D threads: each thread owns one output element.
template <int D>
__global__ __launch_bounds__(D) void paged_reduce_kernel(ReduceParams p) {
    const int h = blockIdx.x, b = blockIdx.y, d = threadIdx.x, H = p.num_heads;
    const int parts = (live_len(p.seq_lens, b, p.len_cap) + p.part_tokens - 1) / p.part_tokens;  // <= max_parts
    float* o = p.out + ((size_t)b * H + h) * D;
    if (parts <= 0) {
        o[d] = 0.0f;
        return;
    }
    const size_t base = ((size_t)b * H + h) * p.max_parts;
    if (parts == 1) {  // one partition: its normalised output is the output (the fused step writes it so)
        o[d] = p.part_out[base * D + d];
        return;
    }
    // The (m, l) pairs and rows of up to U partitions are loaded in one round trip (U = 16 or 64, the
    // smallest that holds them: the loads of a batch go out together, clamped to the last partition
    // so that no branch sits between them); the max and then the sums run in partition order, so the
    // result keeps the bits of a one-by-one walk. Past 64 partitions the rest follow in batches of
    // 64. (One partition at a time, 64 partitions took 20 us on MI355X: a round trip each.)
    auto batch = [&](auto u) -> float {
        constexpr int U = decltype(u)::value;
        float2 ml[U];
        float v[U];
        for (int j = 0; j < U; ++j) {
            const size_t i = base + (size_t)min(j, parts - 1);
            ml[j] = p.part_ml[i];
            v[j] = p.part_out[i * D + d];
        }
        float M = kNegBigR;
        for (int j = 0; j < U; ++j)
            if (j < parts) M = fmaxf(M, ml[j].x);
        for (int i0 = U; i0 < parts; i0 += U)  // (uniform: more than U partitions)
            for (int j = 0; j < U; ++j) M = fmaxf(M, p.part_ml[base + min(i0 + j, parts - 1)].x);
        float L = 0.0f, acc = 0.0f;
        for (int j = 0; j < U; ++j)
            if (j < parts) {
                const float w = partition_weight(ml[j].x, ml[j].y, M);
                L += w;
                acc = __builtin_fmaf(w, v[j], acc);
            }
        for (int i0 = U; i0 < parts; i0 += U) {
            for (int j = 0; j < U; ++j) {
                const size_t i = base + (size_t)min(i0 + j, parts - 1);
                ml[j] = p.part_ml[i];
                v[j] = p.part_out[i * D + d];
            }
            for (int j = 0; j < U; ++j)
                if (i0 + j < parts) {
                    const float w = partition_weight(ml[j].x, ml[j].y, M);
                    L += w;
                    acc = __builtin_fmaf(w, v[j], acc);
                }
        }
        return acc * (1.0f / L);  // (the fused merge normalises the same way: the same bits)
    };
    o[d] = parts <= 16 ? batch(std::integral_constant<int, 16>{}) : batch(std::integral_constant<int, 64>{});
}

template <int KIND>
__device__ __forceinline__ float kv_at(const void* base, size_t i) {
    if constexpr (KIND == KV_F16) return (float)static_cast<const _Float16*>(base)[i];
    else return static_cast<const float*>(base)[i];
}

// ---- naive three-pass baseline (the reference's run_naive, src/kernels.metal:149-218) ----------
// The comparison point for paged_decode: the same attention in three launches with the scores in
// global memory, over the contiguous cache [B][Hkv][max_len][D] (f32 or f16). The passes are laid out
// for wave64 here: one wave per 16 tokens (scores), per row (softmax) and per row (P V).

template <int CTRL>
__device__ __forceinline__ float dpp_f(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float wave_max_f(float x) {
    for (int o = 32; o > 0; o >>= 1) x = fmaxf(x, __shfl_xor(x, o));
    return x;
}
__device__ __forceinline__ float wave_sum_f(float x) {
    for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o);
    return x;
}

// Pass 1, scores[b][h][t] = scale * q . k_t. Grid (ceil(max_len / 16), H, B), one wave each: the
// lanes of quad k take token 16 x + k, lane 4k + j the j-th quarter of its row (D / 4 contiguous
// elements in 16-byte loads, so a quad reads the whole row), and the quad's partial dot products
// are summed by two DPP quad swaps.
template <int KIND, int D>
__global__ __launch_bounds__(64) void naive_scores_kernel(NaiveParams p, int G) {
    constexpr int ESZ = KIND == KV_F16 ? 2 : 4, QD = D / 4, PER = 16 / ESZ, NL = QD / PER;
    const int lane = threadIdx.x, h = blockIdx.y, b = blockIdx.z, H = p.num_heads;
    const int len = live_len(p.seq_lens, b, p.max_len);
    if ((int)blockIdx.x * 16 >= len) return;  // uniform
    const int t = blockIdx.x * 16 + (lane >> 2), qd = lane & 3;
    const bool live = t < len;
    const int ts = live ? t : 0;  // lanes past the end read row 0 and write nothing
    const float* qh = p.q + ((size_t)b * H + h) * D + qd * QD;
    const char* krow = static_cast<const char*>(p.k) +
                       ((((size_t)b * p.num_kv_heads + h / G) * p.max_len + ts) * D + qd * QD) * ESZ;
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < NL; ++i) {
        const uint4 w = *reinterpret_cast<const uint4*>(krow + 16 * i);
        if constexpr (KIND == KV_F16) {
            const _Float16* x = reinterpret_cast<const _Float16*>(&w);
#pragma unroll
            for (int e = 0; e < PER; ++e) s = __builtin_fmaf(qh[i * PER + e], (float)x[e], s);
        } else {
            const float* x = reinterpret_cast<const float*>(&w);
#pragma unroll
            for (int e = 0; e < PER; ++e) s = __builtin_fmaf(qh[i * PER + e], x[e], s);
        }
    }
    s += dpp_f<0xB1>(s);  // quad_perm [1,0,3,2]
    s += dpp_f<0x4E>(s);  // quad_perm [2,3,0,1]
    if (live && qd == 0) p.scores[((size_t)b * H + h) * p.max_len + t] = s * p.scale;
}

// Pass 2, softmax in place. Grid (H, B), one wave per row: max, exp and sum, scale, each a sweep of
// the row 64 tokens at a time with the wave's reductions by lane shuffles.
__global__ __launch_bounds__(64) void naive_softmax_kernel(NaiveParams p) {
    const int h = blockIdx.x, b = blockIdx.y, lane = threadIdx.x;
    const int len = live_len(p.seq_lens, b, p.max_len);
    float* row = p.scores + ((size_t)b * p.num_heads + h) * p.max_len;
    float mx = kNegBigR;
    for (int t = lane; t < len; t += 64) mx = fmaxf(mx, row[t]);
    mx = wave_max_f(mx);
    float sum = 0.0f;
    for (int t = lane; t < len; t += 64) {
        const float e = __expf(row[t] - mx);
        row[t] = e;
        sum += e;
    }
    const float inv = 1.0f / wave_sum_f(sum);
    for (int t = lane; t < len; t += 64) row[t] *= inv;
}

// Pass 3, out[b][h] = sum_t p_t v_t. Grid (H, B), one wave per row: lane l owns D / 64 adjacent
// elements, so each token's V row is one contiguous read across the wave; p_t is the same for every
// lane. An empty sequence writes 0.
template <int KIND, int D>
__global__ __launch_bounds__(64) void naive_pv_kernel(NaiveParams p, int G) {
    constexpr int DL = D / 64;
    const int lane = threadIdx.x, h = blockIdx.x, b = blockIdx.y, H = p.num_heads;
    const int len = live_len(p.seq_lens, b, p.max_len);
    const float* pr = p.scores + ((size_t)b * H + h) * p.max_len;
    const size_t vbase = ((size_t)b * p.num_kv_heads + h / G) * p.max_len * D + (size_t)lane * DL;
    float o[DL];
#pragma unroll
    for (int j = 0; j < DL; ++j) o[j] = 0.0f;
    for (int t = 0; t < len; ++t) {
        const float pt = pr[t];
#pragma unroll
        for (int j = 0; j < DL; ++j) o[j] = __builtin_fmaf(pt, kv_at<KIND>(p.v, vbase + (size_t)t * D + j), o[j]);
    }
#pragma unroll
    for (int j = 0; j < DL; ++j) p.out[((size_t)b * H + h) * D + (size_t)lane * DL + j] = o[j];
}

// fp64 attention over the contiguous cache, one workgroup per (h, b): the reference's
// attention_reference (src/reference.cpp:65-100) on the GPU, for the bench's accuracy and dump
// modes. Two passes over the tokens, as there: the max score, then exp(s - max) summed with the
// weighted V rows; out = acc / sum, 0 for an empty sequence. Scores are recomputed in the second
// pass instead of stored.
__device__ double block_reduce_double(double x, bool is_max) {
    for (int o = 32; o > 0; o >>= 1) {
        const double y = __shfl_xor(x, o);
        x = is_max ? fmax(x, y) : x + y;
    }
    __shared__ double s_red[4];
    __syncthreads();  // s_red may still be read from the previous call
    if ((threadIdx.x & 63) == 0) s_red[threadIdx.x >> 6] = x;
    __syncthreads();
    double r = s_red[0];
    for (int w = 1; w < 4; ++w) r = is_max ? fmax(r, s_red[w]) : r + s_red[w];
    return r;
}

template <int KIND>
__global__ __launch_bounds__(256) void attention_fp64_kernel(NaiveParams p, int D, int G) {
    const int h = blockIdx.x, b = blockIdx.y, H = p.num_heads, len = live_len(p.seq_lens, b, p.max_len);
    const int tid = threadIdx.x;
    const size_t kv0 = ((size_t)b * p.num_kv_heads + h / G) * p.max_len * D;
    const double scale = p.scale;  // the reference's float 1/sqrt(D), widened
    __shared__ double s_q[128];
    __shared__ double s_e[256];
    __shared__ double s_acc[256];
    for (int d = tid; d < D; d += 256) s_q[d] = p.q[((size_t)b * H + h) * D + d];
    __syncthreads();
    auto score = [&](int t) {
        double s = 0.0;
        for (int d = 0; d < D; ++d) s += s_q[d] * (double)kv_at<KIND>(p.k, kv0 + (size_t)t * D + d);
        return s * scale;
    };
    double m = -HUGE_VAL;
    for (int t = tid; t < len; t += 256) m = fmax(m, score(t));
    m = block_reduce_double(m, true);
    const int d = tid % D, slices = 256 / D, sl = tid / D;
    double l = 0.0, acc = 0.0;
    for (int t0 = 0; t0 < len; t0 += 256) {
        const double e = t0 + tid < len ? exp(score(t0 + tid) - m) : 0.0;
        s_e[tid] = e;
        l += e;
        __syncthreads();
        for (int j = sl; j < 256 && t0 + j < len; j += slices)
            acc += s_e[j] * (double)kv_at<KIND>(p.v, kv0 + (size_t)(t0 + j) * D + d);
        __syncthreads();
    }
    l = block_reduce_double(l, false);
    s_acc[tid] = acc;
    __syncthreads();
    if (tid < D) {
        double o = 0.0;
        for (int k = 0; k < slices; ++k) o += s_acc[k * D + tid];
        p.out[((size_t)b * H + h) * D + tid] = len > 0 ? (float)(o / l) : 0.0f;
    }
}

// The streaming-read ceiling (the reference's read_bw, src/kernels.metal:220-233), one workgroup per
// CU: workgroup g reads the contiguous words [g * per_group, (g + 1) * per_group), kReadBwThreads at
// a time, kReadBwUnroll 16-byte loads in flight per thread (32 KB per workgroup). The words are
// XOR-accumulated; the store fires only on a sentinel that no buffer the probe reads (all words
// equal) produces. NT: non-temporal loads, the probe's (fastest); the cache flush uses ordinary
// loads, which allocate in the L2s and the MALL and so evict what was there.
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

template <bool NT>
__device__ __forceinline__ u32x4_t stream_load(const u32x4_t* p) {
    if constexpr (NT) return __builtin_nontemporal_load(p);
    else return *p;
}

template <bool NT>
__global__ __launch_bounds__(kReadBwThreads) void read_bw_kernel(const u32x4_t* __restrict__ src, size_t n16,
                                                                 size_t per_group, float* sink) {
    const size_t beg = (size_t)blockIdx.x * per_group;
    const size_t end = beg + per_group < n16 ? beg + per_group : n16;
    constexpr int T = kReadBwThreads, U = kReadBwUnroll;
    size_t i = beg + threadIdx.x;
    uint32_t acc = 0;
    for (; i + (U - 1) * T < end; i += U * T) {
        u32x4_t x[U];
#pragma unroll
        for (int u = 0; u < U; ++u) x[u] = stream_load<NT>(src + i + u * T);
        __builtin_amdgcn_sched_barrier(0);  // all U loads go out before the first wait
#pragma unroll
        for (int u = 0; u < U; ++u) acc ^= x[u].x ^ x[u].y ^ x[u].z ^ x[u].w;
    }
    for (; i < end; i += T) {
        const u32x4_t x = stream_load<NT>(src + i);
        acc ^= x.x ^ x.y ^ x.z ^ x.w;
    }
    if (acc == 0x9e3779b9u) sink[((size_t)blockIdx.x * T + threadIdx.x) % kReadBwSink] = 1.0f;
}

// Does nothing: the dispatch floor of a launch (kvb_run_empty_grid). The argument keeps the kernel
// signature of a real launch (one kernarg).
__global__ void empty_kernel(int) {}

__global__ __launch_bounds__(256) void fill_kernel(uint4* dst, size_t n16, uint32_t value) {
    const uint4 v = make_uint4(value, value, value, value);
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += (size_t)gridDim.x * 256) dst[i] = v;
}

}  // namespace

hipError_t launch_empty(int groups, int threads, hipStream_t s, const Marks& m) {
    launch_marked(empty_kernel, dim3(groups), dim3(threads), s, m, 0);
    return hipGetLastError();
}

hipError_t launch_paged_reduce(int head_dim, const ReduceParams& p, int batch, hipStream_t s, const Marks& m) {
    const dim3 grid(p.num_heads, batch);
    if (head_dim == 64) launch_marked(paged_reduce_kernel<64>, grid, dim3(64), s, m, p);
    else if (head_dim == 128) launch_marked(paged_reduce_kernel<128>, grid, dim3(128), s, m, p);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

template <int KIND, int D>
void launch_naive_passes(const NaiveParams& p, int group, int batch, hipStream_t s, const Marks& m) {
    const dim3 sgrid((unsigned)((p.max_len > 0 ? p.max_len : 1) + 15) / 16, p.num_heads, batch);
    const Marks first{m.start, nullptr}, last{nullptr, m.stop};
    launch_marked(naive_scores_kernel<KIND, D>, sgrid, dim3(64), s, first, p, group);
    hipLaunchKernelGGL(naive_softmax_kernel, dim3(p.num_heads, batch), dim3(64), 0, s, p);
    launch_marked(naive_pv_kernel<KIND, D>, dim3(p.num_heads, batch), dim3(64), s, last, p, group);
}

hipError_t launch_naive(int kind, int head_dim, int group, const NaiveParams& p, int batch, hipStream_t s,
                        const Marks& m) {
    if (head_dim == 64) {
        if (kind == KV_F16) launch_naive_passes<KV_F16, 64>(p, group, batch, s, m);
        else launch_naive_passes<KV_F32, 64>(p, group, batch, s, m);
    } else if (head_dim == 128) {
        if (kind == KV_F16) launch_naive_passes<KV_F16, 128>(p, group, batch, s, m);
        else launch_naive_passes<KV_F32, 128>(p, group, batch, s, m);
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_attention_fp64(int kind, int head_dim, int group, const NaiveParams& p, int batch, hipStream_t s,
                                 const Marks& m) {
    const dim3 grid(p.num_heads, batch);
    if (kind == KV_F16) launch_marked(attention_fp64_kernel<KV_F16>, grid, dim3(256), s, m, p, head_dim, group);
    else launch_marked(attention_fp64_kernel<KV_F32>, grid, dim3(256), s, m, p, head_dim, group);
    return hipGetLastError();
}

hipError_t launch_read_bw(const void* src, size_t n16, int groups, float* sink, hipStream_t s, const Marks& m,
                          bool nontemporal) {
    if (groups <= 0) return hipErrorInvalidValue;
    const size_t per_group = (n16 + groups - 1) / groups;
    if (nontemporal)
        launch_marked(read_bw_kernel<true>, dim3(groups), dim3(kReadBwThreads), s, m, static_cast<const u32x4_t*>(src),
                      n16, per_group, sink);
    else
        launch_marked(read_bw_kernel<false>, dim3(groups), dim3(kReadBwThreads), s, m, static_cast<const u32x4_t*>(src),
                      n16, per_group, sink);
    return hipGetLastError();
}

hipError_t launch_fill(void* dst, size_t n16, uint32_t value, hipStream_t s) {
    hipLaunchKernelGGL(fill_kernel, dim3(2048), dim3(256), 0, s, static_cast<uint4*>(dst), n16, value);
    return hipGetLastError();
}

}  // namespace kvbk
