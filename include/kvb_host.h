/*
 * kvb_host.h -- C ABI of libkvb_host.so's cache writers and workload generator, for FFI callers
 * (the Python package, bench.py) that build inputs for libkvb_hip.so without the C++ API.
 * These are the host-side producers of the paged cache the decode kernels read: the layout,
 * scatter and int8 quantiser of the reference's src/reference.cpp:11-63 and the workload of
 * src/workload.hpp:26-64, with the generator of include/kvb/rng.hpp. All pointers are host memory.
 * Functions return 0, or -1 on bad arguments.
 */
#ifndef KVB_HOST_H
#define KVB_HOST_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Value distributions of kvbh_fill_workload. */
enum { KVBH_UNIFORM = 0, KVBH_NORMAL = 1 };

/* Fills q (float [B][H][D]) and the contiguous cache k, v ([B][Hkv][max_len][D]; kv_type F16:
 * IEEE binary16 bit patterns, F32 and I8: float) as kvb::Workload does (Workload::Workload,
 * src/workload.hpp:34-64). k32/v32, if not NULL, receive the fp32 values before fp16 rounding.
 * `threads` generator threads (0 = all cores). */
int kvbh_fill_workload(int batch, int num_heads, int num_kv_heads, int head_dim, const int* lens, int max_len,
                       int kv_type, uint64_t seed, float q_amp, int varied, int dist, float* q, void* k, void* v,
                       float* k32, float* v32, int threads);

/* make_paged_layout (src/reference.cpp:11-30 with an oversized pool). dims: max_blocks, live blocks,
 * pool blocks. table: int32 [batch][max_blocks]. */
int kvbh_layout_dims(const int* lens, int batch, int page_size, double pool_factor, int* max_blocks, int* live_blocks,
                     int* pool_blocks);
int kvbh_make_paged_layout(const int* lens, int batch, int page_size, double pool_factor, uint64_t seed,
                           int32_t* table);

/* scatter_to_paged (src/reference.hpp:60-68) for elem_size 4 (f32) or 2 (f16). */
int kvbh_scatter_to_paged(int batch, int num_kv_heads, int head_dim, int page_size, int max_blocks,
                          const int32_t* table, const int* lens, int max_len, size_t elem_size, const void* contig,
                          void* paged);
/* quantize_to_paged_i8 / dequantize_paged_i8 (src/reference.cpp:32-63); scales float [pool][Hkv]. */
int kvbh_quantize_to_paged_i8(int batch, int num_kv_heads, int head_dim, int page_size, int max_blocks,
                              const int32_t* table, const int* lens, int max_len, const float* contig, int8_t* paged,
                              float* scales);
int kvbh_dequantize_paged_i8(int batch, int num_kv_heads, int head_dim, int page_size, int max_blocks,
                             const int32_t* table, const int* lens, int max_len, const int8_t* paged,
                             const float* scales, float* contig);
/* poison_paged: NaN (elem 4/2) or -128 (elem 1, plus NaN scales of unused blocks; scales may be
 * NULL) in every pool element no live token owns. pool_blocks = physical blocks in the pool. */
int kvbh_poison_paged(int batch, int num_kv_heads, int head_dim, int page_size, int max_blocks, int pool_blocks,
                      const int32_t* table, const int* lens, size_t elem_size, void* paged, float* scales);

/* The MI355X partition policy (kvb::mi355x_part_tokens). */
int kvbh_mi355x_part_tokens(int batch, int num_heads, int num_kv_heads, int head_dim, int max_len, int min_groups,
                            int min_part, int max_part);
/* The same policy given the batch's lengths (lens[batch]): a ragged batch caps the partition at
 * kvb::ragged_part_cap: 2048, 3584 or 4096 by its longest sequence (3584 for c5). */
int kvbh_mi355x_part_tokens_lens(int batch, int num_heads, int num_kv_heads, int head_dim, const int* lens,
                                 int min_groups, int min_part, int max_part);

#ifdef __cplusplus
}
#endif
#endif /* KVB_HOST_H */
