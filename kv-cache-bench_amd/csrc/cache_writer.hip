// The cache writers on the GPU: the contiguous cache [B][Hkv][max_len][D] into the paged pool
// [blocks][Hkv][page][D] through the block table, as the reference's host-side scatter_to_paged
// (src/reference.hpp:60-68) and quantize_to_paged_i8 (src/reference.cpp:32-51) do, with the same
// bytes and scales.
//
// One workgroup per (KV head, sequence, logical block), the logical block slowest so the blocks of
// every length spread over the XCDs. A block's live rows are contiguous both in the contiguous
// cache and in its physical block, so scattering is a 16-byte copy of rows * D * esz bytes (D is 64
// or 128, so a row is a whole number of 16-byte words). Quantising reads the block twice (the
// second time from L2): its max |x| first, the int8 values after.
#include "kvb_kernels.hpp"

namespace kvbk {
namespace {

constexpr int kWriterThreads = 256;

__global__ __launch_bounds__(kWriterThreads) void scatter_kernel(CacheWriteParams p) {
    const int kvh = blockIdx.x, b = blockIdx.y, blk_i = blockIdx.z;
    const int len = live_len(p.seq_lens, b, p.len_cap), t0 = blk_i * p.page_size;
    if (t0 >= len) return;
    const int rows = min(len - t0, p.page_size);
    const size_t row_bytes = (size_t)p.head_dim * p.elem_size;
    const size_t n16 = rows * row_bytes / 16;
    const uint4* src = reinterpret_cast<const uint4*>(static_cast<const char*>(p.contig) +
                                                      (((size_t)b * p.num_kv_heads + kvh) * p.max_len + t0) * row_bytes);
    const size_t blk = (size_t)p.block_table[(size_t)b * p.max_blocks + blk_i];
    uint4* dst = reinterpret_cast<uint4*>(static_cast<char*>(p.paged) +
                                          (blk * p.num_kv_heads + kvh) * p.page_size * row_bytes);
    for (size_t w = threadIdx.x; w < n16; w += kWriterThreads) dst[w] = src[w];
}

__device__ __forceinline__ float block_max(float x) {
    for (int o = 32; o > 0; o >>= 1) x = fmaxf(x, __shfl_xor(x, o));
    __shared__ float s_max[kWriterThreads / 64];
    if ((threadIdx.x & 63) == 0) s_max[threadIdx.x >> 6] = x;
    __syncthreads();
    float m = s_max[0];
    for (int w = 1; w < kWriterThreads / 64; ++w) m = fmaxf(m, s_max[w]);
    return m;
}

// x / scale rounded half to even and clamped to +-127 (scale > 0), as the reference's
// int8(clamp(nearbyint(x / scale), -127, 127)); the division is IEEE (correctly rounded).
__device__ __forceinline__ uint32_t quantize_byte(float x, float scale) {
    const float q = fminf(fmaxf(__builtin_rintf(x / scale), -127.0f), 127.0f);
    return (uint32_t)(uint8_t)(int8_t)(int)q;
}

__device__ __forceinline__ float abs_max4(float m, const float4& v) {
    return fmaxf(fmaxf(m, fmaxf(fabsf(v.x), fabsf(v.y))), fmaxf(fabsf(v.z), fabsf(v.w)));
}

__device__ __forceinline__ uint32_t quantize4(const float4& v, float scale) {
    if (!(scale > 0.0f)) return 0u;  // an all-zero slice: every byte 0
    return quantize_byte(v.x, scale) | quantize_byte(v.y, scale) << 8 | quantize_byte(v.z, scale) << 16 |
           quantize_byte(v.w, scale) << 24;
}

// A block of up to kWriterThreads * kQuantRegs groups of 4 values (page 128 at head_dim 128) is
// read once and kept in registers between the max and the quantisation; a larger one is read twice,
// the second time from L2.
constexpr int kQuantRegs = 16;

__global__ __launch_bounds__(kWriterThreads) void quantize_kernel(CacheWriteParams p) {
    const int kvh = blockIdx.x, b = blockIdx.y, blk_i = blockIdx.z;
    const int len = live_len(p.seq_lens, b, p.len_cap), t0 = blk_i * p.page_size;
    if (t0 >= len) return;  // uniform over the workgroup, before the barrier in block_max
    const int rows = min(len - t0, p.page_size);
    const size_t n4 = (size_t)rows * p.head_dim / 4;  // groups of 4 values (head_dim % 4 == 0)
    const float4* src = reinterpret_cast<const float4*>(static_cast<const float*>(p.contig) +
                                                        (((size_t)b * p.num_kv_heads + kvh) * p.max_len + t0) * p.head_dim);
    const size_t blk = (size_t)p.block_table[(size_t)b * p.max_blocks + blk_i];
    uint32_t* dst = reinterpret_cast<uint32_t*>(static_cast<int8_t*>(p.paged) +
                                                (blk * p.num_kv_heads + kvh) * p.page_size * p.head_dim);
    float amax = 0.0f;
    if (n4 <= (size_t)kWriterThreads * kQuantRegs) {  // uniform over the workgroup
        float4 v[kQuantRegs];
#pragma unroll
        for (int r = 0; r < kQuantRegs; ++r) {
            const size_t w = threadIdx.x + (size_t)r * kWriterThreads;
            v[r] = w < n4 ? src[w] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            amax = abs_max4(amax, v[r]);
        }
        const float scale = block_max(amax) / 127.0f;
        if (threadIdx.x == 0) p.scales[blk * p.num_kv_heads + kvh] = scale;
#pragma unroll
        for (int r = 0; r < kQuantRegs; ++r) {
            const size_t w = threadIdx.x + (size_t)r * kWriterThreads;
            if (w < n4) dst[w] = quantize4(v[r], scale);
        }
        return;
    }
    for (size_t w = threadIdx.x; w < n4; w += kWriterThreads) amax = abs_max4(amax, src[w]);
    const float scale = block_max(amax) / 127.0f;
    if (threadIdx.x == 0) p.scales[blk * p.num_kv_heads + kvh] = scale;
    for (size_t w = threadIdx.x; w < n4; w += kWriterThreads) dst[w] = quantize4(src[w], scale);
}

}  // namespace

hipError_t launch_write_paged(const CacheWriteParams& p, int batch, int max_blocks_used, hipStream_t s,
                              const Marks& m) {
    const dim3 grid(p.num_kv_heads, batch, max_blocks_used);
    if (p.quantize) launch_marked(quantize_kernel, grid, dim3(kWriterThreads), s, m, p);
    else launch_marked(scatter_kernel, grid, dim3(kWriterThreads), s, m, p);
    return hipGetLastError();
}

}  // namespace kvbk
