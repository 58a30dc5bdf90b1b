// Launch parameters and launcher declarations shared by the gfx950 kernels and the runtime.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace kvbk {

enum KvKind { KV_F32 = 0, KV_F16 = 1, KV_I8 = 2 };

// Waves per paged_decode workgroup: 4 for every type, as the reference's kSimdGroups
// (src/metal_attn.hpp:41), one per SIMD. With 8 int8 waves (two per SIMD) the second wave on each
// SIMD ended its loop about 7 us after the first on c4, and the workgroup waited for it: measured on
// MI355X, int8 at 4 waves takes 47.2 us on c4 (8 waves: 48.8), 211 us on c5 (223), and c3 the same.
constexpr int decode_waves(int /*kind*/) { return 4; }
// Tokens one wave handles per step of its loop: the N of a 16x16 MFMA tile.
constexpr int kTile = 16;

// The waves of a paged_decode workgroup that serves qg query heads of one KV head: qw heads per
// wave, ts token streams (stream s walks the partition's 32-token tiles s, s + ts, ...) and hs head
// splits (the waves of split j serve heads j * qw .. j * qw + qw - 1 and walk the same tiles as the
// other splits' waves of their stream), hs * ts waves in all.
//  * Up to 16 heads (fp32: 8) one wave serves every head: four streams, one wave per SIMD, the
//    reference's kSimdGroups (16 heads: one head per MFMA column, fp16 and int8).
//  * 32 heads: two splits of four streams of 16-head waves, 8 waves, two per SIMD. int8 waves read
//    each tile themselves, the second split mostly from the CU's caches; the two fp16 waves of a
//    stream load half a tile each and share it through LDS (SHL in paged_decode_kernel).
// (MI355X, 4 x 32k tokens, 8 KV heads, page 128, before head splits: int8 with 16 query heads per KV
// head 84.0 us as two 8-head workgroups; fp16 with 32, 132.2 us as two 16-head workgroups; int8
// with 32, 122.7 us as four 8-head workgroups.)
struct DecodeShape {
    int qw, hs, ts;
};
constexpr DecodeShape decode_shape(int kind, int qg) {
    if (kind == KV_I8 && qg == 32) return DecodeShape{16, 2, 4};
    if (kind == KV_F16 && qg == 32) return DecodeShape{16, 2, 4};
    return DecodeShape{qg, 1, decode_waves(kind)};
}
constexpr int decode_wg_waves(int kind, int qg) { return decode_shape(kind, qg).hs * decode_shape(kind, qg).ts; }
// The fused merge of more than 16 partitions gives each thread one 16-byte chunk of the group's
// [qg][head_dim] output; a workgroup with more chunks than threads leaves such a merge to
// paged_reduce (fp16 workgroups of 16 heads, whose one-split build keeps that path out).
constexpr bool fused_merge_many(int kind, int qg, int head_dim) {
    return qg <= 8 || (decode_shape(kind, qg).hs > 1 && qg * head_dim / 4 <= 64 * decode_wg_waves(kind, qg));
}

// A sequence's length as a kernel uses it: seq_lens[b] (device memory) clamped to [0, cap], where
// cap is what the host sized the launch for (run_paged: min(max_blocks * page_size,
// max_parts * part_tokens); the naive kernels: max_len). The host validates its own copy of the
// lengths; if the device copy disagrees, the clamp keeps every block-table read inside the
// sequence's row, every workspace access inside its (sequence, head) slots and every contiguous-cache
// read inside its max_len rows. When the two copies agree, as they must, the clamp changes nothing.
__device__ __forceinline__ int live_len(const int32_t* seq_lens, int b, int cap) {
    return max(0, min(seq_lens[b], cap));
}

// Division by a launch-constant divisor d >= 1 without a divide: for 0 <= n < 2^31,
// n / d = mulhi(n, mul) >> shift with l = ceil(log2 d), mul = ceil(2^(31 + l) / d), shift = l - 1
// (mul < 2^32 because d > 2^(l-1)); d = 1 is mul = 0 (n itself). The error of the rounded-up mul
// adds less than n / 2^(31 + l) < 1 / d to n / d, which leaves its floor unchanged. (Checked
// exhaustively for every n on d = 1, 3, 7, 16, 48, 64, 96, 128, 4095.)
struct FastDiv {
    uint32_t mul = 0, shift = 0;
};
inline FastDiv make_fast_div(uint32_t d) {
    FastDiv f;
    if (d <= 1) return f;
    uint32_t l = 0;
    while ((1ull << l) < d) ++l;
    f.mul = (uint32_t)(((1ull << (31 + l)) + d - 1) / d);
    f.shift = l - 1;
    return f;
}
__device__ __forceinline__ int fast_div(int n, FastDiv f) {
    return f.mul ? (int)(__umulhi((uint32_t)n, f.mul) >> f.shift) : n;
}

struct DecodeParams {
    const float* q;             // [B][H][D]
    const void* k;              // [blocks][Hkv][page][D]
    const void* v;
    const int32_t* block_table; // [B][max_blocks]
    const int32_t* seq_lens;    // [B]
    const float* k_scale;       // [blocks][Hkv], i8 only
    const float* v_scale;
    float* part_out;            // [B][H][max_parts][D]: partition output o / l
    float2* part_ml;            // [B][H][max_parts]: (max score, exp-sum), natural-log units
    int num_heads;
    int num_kv_heads;
    int group;                  // H / Hkv
    int page_size;
    FastDiv page_div;           // division by page_size
    int tile_in_page;           // page_size and part_tokens are multiples of 32: a 32-token tile lies in one page
    int table_in_lanes;         // tile-aligned, and a partition touches at most kLaneBlocks blocks
    int max_blocks;
    int max_parts;
    int part_tokens;
    int len_cap;                // live_len's cap: min(max_blocks * page_size, max_parts * part_tokens)
    float qscale;               // softmax scale * log2(e): scores are kept in base-2 units
    // Fused merge (null: leave the merge to paged_reduce). The last workgroup of a (sequence,
    // head group) to finish merges its partitions into out; counters[b * (H / qg) + group] counts
    // arrivals and is reset to 0 by that workgroup (it must start at 0). Requires
    // qg * max_parts <= fused_merge_slots(kind, head_dim).
    float* out;                 // [B][H][D]
    int* counters;              // [B][H / qg]
    int batch;
    // Nonzero: a ragged batch in longest-first order. Grid y enumerates this many work items (see
    // ragged_item in paged_decode_impl.hpp) instead of grid (y, z) = (sequence, partition).
    // Requires batch <= kRaggedMaxBatch and part_tokens < 65536.
    int ragged_items;
    // Nonzero: launch the measurement variant that issues the decode's loads and computes nothing
    // (tile-aligned pages only: page_size and part_tokens multiples of kTile).
    int loads_only;
    // Nonzero: each workgroup computes two consecutive partitions (the PAIR kernels). Requires
    // tile-aligned pages, an f16 or i8 cache, the plain grid (ragged_items 0), and part_tokens a
    // multiple of 2 * kTile * decode_waves(kind) (32-token tiles, dealt round robin to the waves), so
    // that each partition keeps its tiles' waves and order; and one head split (decode_shape).
    int pair;
    // Query heads per workgroup: a divisor of group, at most the kernel's QG; read by the PART
    // kernels only (the others serve QG heads). Last, so that it leaves the other fields' offsets
    // in the kernel arguments as they were.
    int qg;
    // Nonzero (any-page path only, page_size or part_tokens not a multiple of kTile): a workgroup's
    // range touches at most kTableStage blocks, so the STAGE kernel copies their ids into LDS.
    int table_in_lds;
};

// Block ids the any-page kernel stages in LDS per workgroup (16 KB): a 4096-token partition at any
// page size, page 1 included.
constexpr int kTableStage = 4096;

// Blocks of one partition that paged_decode holds in lanes: one per lane of one VGPR (and, for int8,
// one VGPR each for the K and V scales). With more, it reads the block table per tile instead.
constexpr int kLaneBlocks = 64;

// Ragged batches up to this many sequences use the longest-first work order (one lane per
// sequence, 8 sequences per lane at most).
constexpr int kRaggedMaxBatch = 512;

// Weight of one partition in the merge, w = l exp(m - M) (m, M in natural-log units). paged_reduce
// and the fused merge both use it, then sum L += w and o = fma(w, o_i, o) in partition order, so
// the two give the same bits: w is rounded here, and the compiler may not fuse its product into
// L's sum (which it would otherwise do in one kernel and not in the other).
__device__ __forceinline__ float partition_weight(float m, float l, float M) {
#pragma clang fp contract(off)
    return l * __builtin_amdgcn_exp2f((m - M) * 1.4426950408889634f);
}

// Partition (m, l) pairs the fused merge stages in LDS (the V-tile space of one workgroup: 32
// tokens x head_dim per wave in the storage type). Past this the partitions are merged by
// paged_reduce as a second kernel.
constexpr int fused_merge_slots(int kind, int head_dim) {
    return decode_waves(kind) * 32 * head_dim * (kind == KV_F32 ? 4 : kind == KV_I8 ? 1 : 2) / 8;
}

struct ReduceParams {
    const float* part_out;
    const float2* part_ml;
    const int32_t* seq_lens;
    float* out;                 // [B][H][D]
    int num_heads;
    int max_parts;
    int part_tokens;
    int len_cap;                // as DecodeParams::len_cap
};

struct NaiveParams {
    const float* q;
    const void* k;              // [B][Hkv][max_len][D]
    const void* v;
    const int32_t* seq_lens;
    float* scores;              // [B][H][max_len]
    float* out;
    int num_heads;
    int num_kv_heads;
    int max_len;
    float scale;
};

// Timing marks of a launch: events that the kernel dispatch itself stamps with its start and end
// (hipExtLaunchKernelGGL), so a pair brackets the kernels' execution and not the launch gap before
// the first one (the reference's GPUStartTime / GPUEndTime, src/metal_attn.mm:119-130).
struct Marks {
    hipEvent_t start = nullptr;
    hipEvent_t stop = nullptr;
    // Set: the paged_decode dispatch writes the name of the kernel it would launch here (as the
    // profilers print it) and launches nothing.
    char* describe = nullptr;
    size_t describe_cap = 0;
};

template <typename... KArgs, typename... Args>
inline void launch_marked_lds(void (*kernel)(KArgs...), dim3 grid, dim3 block, size_t lds, hipStream_t s,
                              const Marks& m, Args... args) {
    if (m.start || m.stop)
        hipExtLaunchKernelGGL(kernel, grid, block, lds, s, m.start, m.stop, 0, args...);
    else
        hipLaunchKernelGGL(kernel, grid, block, lds, s, args...);
}
template <typename... KArgs, typename... Args>
inline void launch_marked(void (*kernel)(KArgs...), dim3 grid, dim3 block, hipStream_t s, const Marks& m,
                          Args... args) {
    launch_marked_lds(kernel, grid, block, 0, s, m, args...);
}

// paged_decode for one storage kind: grid (H / qg, batch, max_parts), or (H / qg, ragged_items, 1)
// for a ragged batch, decode_wg_waves(kind, qg) waves per workgroup. qg (= p.qg) picks the kernel
// built for the next of 1, 2, 4 and 8 query heads, whose columns past qg are idle, or the one built
// for 16 (fp16, int8) or 32 (fp16, int8) heads. `fast`: every 16-token tile lies inside one page
// (page_size % 16 == 0 and part_tokens % 16 == 0), so block ids and scales are read once per tile.
hipError_t launch_paged_decode_f32(int head_dim, int qg, bool fast, const DecodeParams& p, int batch, hipStream_t s,
                                   const Marks& m = {});
hipError_t launch_paged_decode_f16(int head_dim, int qg, bool fast, const DecodeParams& p, int batch, hipStream_t s,
                                   const Marks& m = {});
hipError_t launch_paged_decode_i8(int head_dim, int qg, bool fast, const DecodeParams& p, int batch, hipStream_t s,
                                  const Marks& m = {});

// paged_reduce: grid (H, batch), head_dim threads.
hipError_t launch_paged_reduce(int head_dim, const ReduceParams& p, int batch, hipStream_t s, const Marks& m = {});

// The naive three-pass baseline over a contiguous cache (f32 or f16).
hipError_t launch_naive(int kind, int head_dim, int group, const NaiveParams& p, int batch, hipStream_t s,
                        const Marks& m = {});

// The cache writers (scatter_to_paged / quantize_to_paged_i8 on the GPU).
struct CacheWriteParams {
    const void* contig;         // [B][Hkv][max_len][D]: elem_size bytes per value, fp32 if quantize
    void* paged;                // [blocks][Hkv][page][D]: elem_size bytes, int8 if quantize
    float* scales;              // [blocks][Hkv], quantize only
    const int32_t* block_table; // [B][max_blocks]
    const int32_t* seq_lens;    // [B]
    int num_kv_heads;
    int head_dim;               // 64 or 128
    int elem_size;              // 1, 2 or 4 (scatter)
    int page_size;
    int max_blocks;
    int max_len;
    int quantize;               // 1: fp32 -> int8 with per-(block, KV head) scales
    int len_cap;                // live_len's cap: min(max_len, max_blocks * page_size)
};
// grid (Hkv, batch, max_blocks_used): max_blocks_used = ceil(max_len / page)
hipError_t launch_write_paged(const CacheWriteParams& p, int batch, int max_blocks_used, hipStream_t s,
                              const Marks& m = {});

// fp64 attention over the contiguous cache (f32 or f16), grid (H, batch): the accuracy reference.
hipError_t launch_attention_fp64(int kind, int head_dim, int group, const NaiveParams& p, int batch, hipStream_t s,
                                 const Marks& m = {});

// Streaming read of n16 16-byte words, one contiguous chunk per workgroup; the guarded store into
// sink (kReadBwSink floats) never fires for real data. Measured on MI355X (cold, one launch), one
// workgroup per CU of 512 threads with 4 loads in flight each was the fastest shape of a sweep
// (grid-stride over 512..131072 workgroups, chunks over 256..8192 workgroups of 256..1024 threads,
// 1..16 loads in flight) at every size tried: 7.15 TB/s on 537 MB, 7.20 on 1 GiB, 7.25 on 4 GiB,
// against 6.56, 6.43 and 6.75-6.99 for 32768 workgroups x 256 threads x 8 grid-strided loads.
constexpr int kReadBwThreads = 512;
constexpr int kReadBwUnroll = 4;
constexpr size_t kReadBwSink = 2048 * 256;
// nontemporal: the probe's loads; false: ordinary loads, which allocate in (and so evict) the L2s and
// the MALL, for the cache flush.
hipError_t launch_read_bw(const void* src, size_t n16, int groups, float* sink, hipStream_t s, const Marks& m = {},
                          bool nontemporal = true);
// Overwrites n16 16-byte words with `value`.
hipError_t launch_fill(void* dst, size_t n16, uint32_t value, hipStream_t s);
// A kernel that does nothing, `groups` workgroups of `threads` threads (kvb_run_empty_grid).
hipError_t launch_empty(int groups, int threads, hipStream_t s, const Marks& m);

}  // namespace kvbk
