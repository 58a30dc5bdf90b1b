/*
 * kvb_oracle.h -- CPU oracle for the paged-KV decode-attention path.
 *
 * TEST INFRASTRUCTURE ONLY. This is a plain-C restatement of the reference's CPU side
 * (chipontix/kv-cache-bench: src/reference.hpp, src/reference.cpp, src/workload.hpp,
 * src/metal_attn.hpp:43-51, tests/gpu_tests.cpp:13-62, src/kernels.metal:97-147). It is the
 * checker the tests, __graft_entry__.smoke() and the cpu_baseline leg of bench.py compare
 * against. Nothing in the product (the HIP library, the C++ host, the Python package) may
 * include, link, load or call it.
 *
 * Pinning (what keeps this restatement honest):
 *   - attention_f32/_f16: the reference's own exact properties (tests/cpu_tests.cpp:40-84:
 *     zero query = mean of V, dominant key = its V row exactly, huge scores finite, GQA heads
 *     identical), brute-force agreement with an independent single-pass evaluation in the
 *     tests, and agreement with the reference's attention_reference compiled from its own
 *     source into oracle/_ref (when /root/reference is mounted).
 *   - make_paged_layout: permutation/count invariants of tests/cpu_tests.cpp:85-94 and the
 *     empty-sequence table of tests/boundary_tests.cpp:106-109; the shuffle itself is this
 *     build's own library-independent Fisher-Yates (the reference's std::shuffle stream is
 *     implementation-defined), so only the invariants, not the permutation, match _ref.
 *   - quantize/dequantize: closed form (round trip <= s/2, peak 127, zero slice -> scale 0,
 *     tests/cpu_tests.cpp:115-148) and bit-exact agreement with _ref on the same layout.
 *   - auto_part_tokens: the threshold table of tests/boundary_tests.cpp:86-92 and _ref.
 *   - max_abs_diff: the NaN KAT of tests/boundary_tests.cpp:80-85.
 *   - mt19937_64: the 10000th output fixed by the C++ standard ([rand.predef]).
 *   - f16 conversion: exhaustive agreement with the hardware/compiler conversion in tests.
 *   - partition_state: the states merge back to attention_f32 (the split-K identity).
 *   - fp16/int8 storage bounds: sound on constructed cases that need each of their terms (a V
 *     tie that rounds down; two K rows that round to one stored row from either side).
 *   - split_decode (a CPU model of this build's kernel): the GPU parity battery, run on it.
 * tests/mutation/mutate.py plants mistakes in this file and checks that those pins catch each one.
 */
#ifndef KVB_ORACLE_H
#define KVB_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
    int batch;
    int num_heads;    /* query heads H */
    int num_kv_heads; /* KV heads Hkv, H % Hkv == 0 */
    int head_dim;     /* D */
} kvbo_shape;

/* ---- scalar helpers ---------------------------------------------------------------------- */

/* IEEE binary16 <-> binary32. f16 -> f32 is exact; f32 -> f16 rounds to nearest even. */
float kvbo_f16_to_f32(uint16_t h);
uint16_t kvbo_f32_to_f16(float f);

/* max |a[i] - b[i]| in fp64; +inf if any difference is NaN (src/reference.hpp:27-35). */
double kvbo_max_abs_diff(const float* a, const float* b, size_t n);

/* ---- mt19937_64 (the engine is fully specified by the C++ standard) ---------------------- */
typedef struct {
    uint64_t mt[312];
    int idx;
} kvbo_mt64;
void kvbo_mt64_seed(kvbo_mt64* g, uint64_t seed);
uint64_t kvbo_mt64_next(kvbo_mt64* g);
/* Uniform integer in [0, n) by 128-bit multiply-shift of one raw draw. */
uint64_t kvbo_mt64_below(kvbo_mt64* g, uint64_t n);

/* ---- layouts (src/reference.hpp:37-58) --------------------------------------------------- */
size_t kvbo_contig_index(const kvbo_shape* s, int max_len, int b, int kvh, int t, int d);
size_t kvbo_paged_index(const kvbo_shape* s, int page_size, int max_blocks, const int32_t* table, int b,
                        int kvh, int t, int d);

/* Sizes of the layout make_paged_layout builds (src/reference.cpp:11-30): max_blocks =
 * max_b ceil(len_b / page), live = sum_b ceil(len_b / page), pool = ceil(live * pool_factor)
 * (pool_factor >= 1; 1 reproduces the reference, whose pool is exactly the live blocks).
 * Returns 0, or -1 on bad arguments. */
int kvbo_layout_dims(const int* lens, int batch, int page_size, double pool_factor, int* max_blocks,
                     int* live_blocks, int* pool_blocks);

/* Block table [batch][max_blocks]: physical ids 0..pool-1 shuffled by Fisher-Yates driven by
 * mt19937_64(seed) (for i = pool-1 .. 1: swap(i, below(i+1))), assigned in order to sequence
 * 0's logical blocks, then sequence 1's, ...; unused entries are -1. Returns 0 / -1. */
int kvbo_make_paged_layout(const int* lens, int batch, int page_size, double pool_factor, uint64_t seed,
                           int32_t* table);

/* Copies every live token of the contiguous [B][Hkv][max_len][D] cache into the paged pool
 * [blocks][Hkv][page][D] (src/reference.hpp:60-68); elements are elem_size bytes, copied bit-exactly. */
void kvbo_scatter_to_paged(const kvbo_shape* s, int page_size, int max_blocks, const int32_t* table,
                           const int* lens, int max_len, size_t elem_size, const void* contig, void* paged);

/* int8 per-(physical block, KV head) quantiser (src/reference.cpp:32-51): amax over the live
 * tokens of the slice, scale = amax / 127 (fp32), q = clamp(nearbyint(x / scale), -127, 127), or 0
 * when the scale is 0. scales is [pool][Hkv]. */
void kvbo_quantize_to_paged_i8(const kvbo_shape* s, int page_size, int max_blocks, const int32_t* table,
                               const int* lens, int max_len, const float* contig, int8_t* paged,
                               float* scales);
/* The inverse on live tokens: contig = float(q) * scale (src/reference.cpp:53-63). */
void kvbo_dequantize_paged_i8(const kvbo_shape* s, int page_size, int max_blocks, const int32_t* table,
                              const int* lens, int max_len, const int8_t* paged, const float* scales,
                              float* contig);

/* ---- the fp64 two-pass reference (src/reference.cpp:65-100) ------------------------------ */
/* out[b][h][d] = softmax_t(scale * q.k_t) . v_t over the contiguous cache, accumulated in fp64
 * with a two-pass softmax (max, then exp-sum); an empty sequence gives exactly 0. `threads`
 * workers take rows b*H+h round robin. k/v of attention_f16 are IEEE binary16 bit patterns. */
void kvbo_attention_f32(const kvbo_shape* s, const int* lens, int max_len, const float* q, const float* k,
                        const float* v, float* out, float scale, int threads);
void kvbo_attention_f16(const kvbo_shape* s, const int* lens, int max_len, const float* q,
                        const uint16_t* k, const uint16_t* v, float* out, float scale, int threads);

/* Per-partition state the split-K decode writes to its workspace (src/kernels.metal:97-120):
 * for query head h of sequence b and partition p (tokens [p*part, min(len, (p+1)*part))),
 * m = max score (natural-log units, scale applied), l = sum exp(score - m), o[d] = sum exp(score - m)
 * v[d] / l. Computed in fp64 on the contiguous fp32 cache. Returns 0 if the partition is
 * empty (nothing written), 1 otherwise. */
int kvbo_partition_state_f32(const kvbo_shape* s, const int* lens, int max_len, const float* q, const float* k,
                             const float* v, float scale, int part_tokens, int b, int h, int p, double* m,
                             double* l, double* o);

/* Split-K partition size when part_tokens is 0 (src/metal_attn.hpp:43-51): the largest power of
 * two in [64, 512] with batch * Hkv * ceil(max_len / part) >= 512. */
int kvbo_auto_part_tokens(int batch, int num_kv_heads, int max_len);

/* A CPU model of this build's split-K decode (kv-cache-bench_amd/csrc/paged_decode_impl.hpp), in
 * fp32, reading the paged pool through the block table as the kernel does. Per (sequence, query
 * head) and partition of part_tokens tokens (src/kernels.metal:60-64): `waves` online-softmax
 * states over tiles of 16 tokens taken round robin (the tail tile masked at the sequence end), the
 * int8 K scale on the score and the V scale on p; the states merge with weights exp(m_w - M) into
 * the partition's (o / L, M, L) (src/kernels.metal:97-120). The products use the kernel's number
 * formats: q * scale scaled by a power of two, as high and low fp16 parts (fp16 caches) or three
 * signed byte digits (int8), p (int8: p * v_scale, normalised by the wave's largest V-scale power
 * of two) as high and low fp16 parts, each part with its own accumulator, summed at the end. Then, as a second phase, the partition
 * merge of paged_reduce (src/kernels.metal:124-147): out = sum w_i o_i / sum w_i with
 * w_i = l_i exp(m_i - M); an empty sequence gives 0. exp is evaluated as the GPU's exp unit
 * returns it, with results below 2^-126 zero.
 * kv_type: 0 fp32, 1 fp16 (bit patterns), 2 int8 with k_scale / v_scale [pool blocks][Hkv].
 * part_tokens 0 means kvbo_auto_part_tokens. part_out [B][H][max_parts][D] and
 * part_ml [B][H][max_parts][2] may be NULL; the slots of empty partitions are left NaN.
 * `lens` plays the kernel's device copy of the lengths and max_len the host's: as in the kernel,
 * each length is clamped to [0, min(max_blocks * page_size, max_parts * part_tokens)] and a block id
 * of -1 reads as zeros, so lengths that disagree with max_len and the table stay inside them.
 * Returns max_parts; -2 if an access left a sequence's table row or its workspace slots (the
 * model counts them); -1 on bad arguments.
 * It is the host of the mutation harness's planted kernel mistakes (tests/mutation/mutate.py), and
 * it is pinned by the same parity battery as the GPU kernels (tests/test_split_model.py). */
int kvbo_split_decode(const kvbo_shape* s, int kv_type, int page_size, int max_blocks, const int32_t* table,
                      const int* lens, int max_len, const float* q, const void* k_pool, const void* v_pool,
                      const float* k_scale, const float* v_scale, float scale, int part_tokens, int waves,
                      float* part_out, float* part_ml, float* out, int threads);

/* Derived storage-error bounds (tests/gpu_tests.cpp:16-62). q is [B][H][D] fp32; k32/v32 the
 * unrounded fp32 contiguous data; scales [pool][Hkv]. Both include the 2e-5 kernel tolerance. */
double kvbo_fp16_storage_bound(const kvbo_shape* s, const int* lens, int max_len, const float* q,
                               const float* k32, const float* v32);
double kvbo_i8_storage_bound(const kvbo_shape* s, const int* lens, int page_size, int max_blocks,
                             const int32_t* table, const float* q, const float* k_scale,
                             const float* v_scale);

#ifdef __cplusplus
}
#endif
#endif /* KVB_ORACLE_H */
