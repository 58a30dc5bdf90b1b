// paged_decode for gfx950: split-K decode attention over a paged KV cache.
//
// Semantics follow the reference's paged_decode (src/kernels.metal:35-121): a workgroup owns one
// partition of part_tokens tokens of one sequence and qg query heads of one KV head, and writes the
// partition's normalised output o / l plus (m, l) to slot (b*H + h)*max_parts + part of the
// split-K workspace. The mapping onto CDNA4 is this build's own:
//
//  * Each wave64 walks 32-token tiles of the partition (wave w takes tiles w, w+4, ...), with the
//    next tile's K and V loads in flight while it computes one, and keeps its own online-softmax
//    state; the workgroup merges the four wave states at the end, as the reference merges its
//    simdgroups.
//  * Both products run on MFMA. Scores come out transposed, S^T = K Q^T, one 16x16 tile per 16
//    tokens: the tokens are rows, the 16 columns are the qg heads split into a high and a low fp16
//    part (columns 2h, 2h+1), so K is read as stored and q keeps ~22 bits; the MFMA accumulates in
//    fp32. The kernel is built for QG = 1, 2, 4 or 8 heads and serves qg <= QG of them (DecodeParams::qg:
//    a group of 3 runs the QG = 4 build, of 5, 6 or 7 the QG = 8 build, both as their PART variants,
//    which read qg at run time); the columns past qg are zero. fp32 caches use v_mfma_f32_16x16x4_f32 on q and K as they are (columns 2h+1 are zero).
//  * In that layout a lane holds 8 tokens of one column, which is exactly its share of the P^T
//    operand of O^T = V^T P^T (v_mfma_f32_16x16x32_f16 over 32 tokens): p = exp2(s - m) never
//    leaves the lane, split into high and low fp16 parts like q. V^T comes from LDS through the
//    transposing reads (ds_read_b64_tr_b16 / _b8): the wave stores the V tile row-major, as stored
//    (int8 as bytes, widened to exact fp16 after the read), with a 16-byte-chunk XOR swizzle that
//    spreads the rows one half-wave reads over all the banks.
//  * K is loaded straight into the A-operand layout: lane l reads 16 bytes of token l%16, lanes l,
//    l+16, l+32, l+48 cover 64 contiguous bytes of that row per instruction. The contraction order
//    over d is free, so each storage type picks the d order its loads give and q matches (dslot).
//  * DPP quad swaps merge the high/low columns; lane shuffles reduce the tile max and the sums
//    across the four row groups.
//  * int8: the scores run on v_mfma_i32_16x16x64_i8 with K as stored and q split into three signed
//    byte digits (q * 2^-e = d0 + d1 / 2^7 + d2 / 2^14): exact integer dot products per digit,
//    combined in fp32. V bytes become exact fp16 (x ^ 0x80 under a 0x64 exponent, minus 1152) for the
//    P*V MFMA. The per-(block, KV head) K scale multiplies the score and the V scale multiplies p
//    (normalised by a running power of two per wave so the fp16 split of p * v_scale stays out of
//    the subnormal range).
//  * With DecodeParams::out set, the merge of the partitions (paged_reduce's job) is fused: the
//    last workgroup of a (sequence, head group) to finish, found with an agent-scope counter,
//    merges them, so a decode step is one kernel. Up to 16 partitions, each thread reads its
//    head's (m, l) with its rows in one round trip; past that, the (m, l) go through LDS.
//  * The LOADS instantiation (kvb_run_paged_loads) keeps every load and drops the arithmetic: the
//    time of the decode's memory traffic alone, for measurement.
//  * A ragged batch runs in longest-first order (ragged_item): grid y enumerates its partitions,
//    the largest first, and each wave finds its workgroup's (sequence, partition) from seq_lens.
//  * Tokens past the partition end get weight 0 and never reach the arithmetic as data. With
//    `FAST` (every 16-token half tile inside one page) the block id and scales are one scalar read
//    per half tile and K/V come through a buffer resource sized to its live rows, so rows past the
//    end read as zeros without touching memory; otherwise every lane looks up its own token's block
//    (any page size) and lanes past the end re-read the partition's first token and zero it.
#pragma once

#include <algorithm>
#include <cstdio>
#include <type_traits>

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include "kvb_kernels.hpp"

namespace kvbk {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float floatx4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef int i32x2_t __attribute__((ext_vector_type(2)));
typedef int i32x4_t __attribute__((ext_vector_type(4)));
typedef __fp16 fp16x4_t __attribute__((__vector_size__(4 * sizeof(__fp16))));
typedef __fp16 fp16x8_t __attribute__((__vector_size__(8 * sizeof(__fp16))));
typedef __attribute__((address_space(3))) fp16x4_t lds_fp16x4_t;
typedef __attribute__((address_space(3))) i32x2_t lds_i32x2_t;

// Pointers into the constant address space (4): loads through them may be scalar (s_load).
typedef __attribute__((address_space(4))) const int32_t* const_i32;
typedef __attribute__((address_space(4))) const float* const_f32;

// Buffer-instruction cache policy sc1: device (agent) scope, coherent across the XCDs' L2s.
constexpr int kScopeAgent = 16;
constexpr float kNegBig = -1e30f;  // "minus infinity" that keeps exp2(kNegBig - m) == 0 and no inf - inf
constexpr float kLn2 = 0.693147180559945309f;
constexpr float kLog2e = 1.4426950408889634f;
constexpr int kHalf = 16;          // tokens per MFMA row block
constexpr int kTok = 2 * kHalf;    // tokens per wave step (the K of a 16x16x32 MFMA)
// Cache policy of the K/V loads: non-temporal (the data is read once per step). Measured on MI355X
// streaming reads reach ~7.0 TB/s with it against ~6.3 TB/s without.
constexpr int kNonTemporal = 2;

#ifdef KVB_WG_TIMESTAMPS
// Measurement build only (make -C kv-cache-bench_amd timestamps, into build-ts/): per-workgroup
// s_memrealtime stamps (100 MHz) of the last launch, kWgStampWords per linear workgroup id:
//   0 start; 1 wave 0's loop end; 2 the slowest wave's loop end; 3 the partition stores issued (after
//   the wave states are merged); 4 those stores acknowledged; 5 the arrival count returned (0 in the
//   two-kernel form); 6 merge done (0 where the workgroup did not merge); 7 where wave 0 ran: HW_ID
//   (SIMD, CU, SH, SE) in the low 32 bits, XCC_ID above.
// The loads-only variant writes its loop end into words 1-4. Read by kvb_wg_stamps_<kind>
// (paged_decode_<kind>.hip). The stamped build waits for its partition stores before the merge test
// in the two-kernel form too.
constexpr unsigned kWgStampGroups = 65536, kWgStampWords = 8;
__device__ unsigned long long g_wg_stamps[kWgStampGroups * kWgStampWords];
__device__ __forceinline__ unsigned long long wg_where() {
    const unsigned hw = __builtin_amdgcn_s_getreg((31 << 11) | 4);    // hwreg(HW_REG_HW_ID)
    const unsigned xcc = __builtin_amdgcn_s_getreg((31 << 11) | 20);  // hwreg(HW_REG_XCC_ID)
    return ((unsigned long long)xcc << 32) | hw;
}
#endif

// x as one value the compiler must materialise (an empty asm that may rewrite it). The fp16 split
// of p into high and low parts needs the high part the P*V MFMA receives to be the one the low part
// is taken against. For 16-head waves the compiler built the high operand with v_cvt_pk_f16_f32 from
// the fp32 product while the low part was taken against f16(p * v_scale) rounded once by v_fma_mix:
// on MI355X a few rows of a partition came out about one fp16 step of p off (2.3e-6 where the
// 8-head waves of the same heads were exact).
__device__ __forceinline__ _Float16 pinned(_Float16 x) {
    asm volatile("" : "+v"(x));
    return x;
}

// ---- cross-lane helpers -------------------------------------------------------------------------

template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}
constexpr int kQuadSwap1 = 0xB1;  // quad_perm [1,0,3,2]: lane l <-> l ^ 1
// The value of lane l ^ 1 (every lane of a quad permutation is valid: no old value to keep).
__device__ __forceinline__ float quad_swap1(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), kQuadSwap1, 0xF, 0xF, true));
}

// The max / sum of a value over lanes l, l^16, l^32, l^48, on every lane. (Not v_permlane16/32_swap:
// with the same value in both operands this compiler folds the two results into one.)
__device__ __forceinline__ float max_x16_x32(float x) {
    x = fmaxf(x, __shfl_xor(x, 16));
    return fmaxf(x, __shfl_xor(x, 32));
}
__device__ __forceinline__ float sum_x16_x32(float x) {
    x += __shfl_xor(x, 16);
    return x + __shfl_xor(x, 32);
}
__device__ __forceinline__ float wave_max(float x) {
    for (int off = 32; off > 0; off >>= 1) x = fmaxf(x, __shfl_xor(x, off));
    return x;
}

// 8 int8 (two dwords) -> 8 exact fp16: 0x6400 | (x ^ 0x80) is the fp16 value 1024 + x + 128.
__device__ __forceinline__ half8_t i8x8_to_half8(uint32_t w0, uint32_t w1) {
    const uint32_t x0 = w0 ^ 0x80808080u, x1 = w1 ^ 0x80808080u;
    const uint32_t h0 = __builtin_amdgcn_perm(0x64646464u, x0, 0x04010400u);
    const uint32_t h1 = __builtin_amdgcn_perm(0x64646464u, x0, 0x04030402u);
    const uint32_t h2 = __builtin_amdgcn_perm(0x64646464u, x1, 0x04010400u);
    const uint32_t h3 = __builtin_amdgcn_perm(0x64646464u, x1, 0x04030402u);
    const half2_t bias = {(_Float16)1152.0f, (_Float16)1152.0f};
    const half2_t a = __builtin_bit_cast(half2_t, h0) - bias;
    const half2_t b = __builtin_bit_cast(half2_t, h1) - bias;
    const half2_t c = __builtin_bit_cast(half2_t, h2) - bias;
    const half2_t d = __builtin_bit_cast(half2_t, h3) - bias;
    half8_t r;
    r[0] = a[0]; r[1] = a[1]; r[2] = b[0]; r[3] = b[1];
    r[4] = c[0]; r[5] = c[1]; r[6] = d[0]; r[7] = d[1];
    return r;
}

// ---- per storage type --------------------------------------------------------------------------
// KLOADS: 16-byte K loads per lane per half tile; NJ: score MFMAs per half tile; kdoff/dslot: the d
// order of the score contraction (a K load's first element, and MFMA j slot s). V is read row-major:
// VL lanes per row (16 bytes each), 64/VL rows per load, NV loads per half tile. In LDS, V keeps its
// storage type (fp16, int8 or fp32) with row stride D elements; 16-byte chunk ch of row t sits at
// ch ^ vswz(t) (fp32: ch ^ swz(t)).
//
// fp16 and int8 V^T operands come from transposing LDS reads (ds_read_b64_tr_b16 / _tr_b8): in each
// 16-lane group, the 4 halves (8 bytes) that lane l addresses form a flat sequence F, and lane i
// receives F[i], F[i + 16], ... So for d = 16 mb + i and the lane's 8 tokens, lane l addresses
// token (l >> 2) [b16] or (l >> 1) [b8] of the 8, at d = 16 mb + 4 (l & 3) [b16] or 8 (l & 1) [b8].
// vswz spreads the rows one half-wave reads (8 rows x 32 bytes for fp16, 16 x 16 for int8) over
// all 64 banks.

template <int KIND, int D>
struct KvT;

template <int D>
struct KvT<KV_F16, D> {
    static constexpr int ESZ = 2, KLOADS = D / 32, NJ = D / 32;
    static constexpr int VL = D * 2 / 16, NV = kHalf * VL / 64;
    static constexpr int LDS_ESZ = 2;
    __device__ static int kdoff(int c, int q4) { return 32 * c + 8 * q4; }
    __device__ static int dslot(int j, int q4, int s) { return 32 * j + 8 * q4 + s; }
    // rows 0-7 (and 8-15, 16-23, 24-31): 32-byte chunk pairs at 8 distinct offsets mod 256 bytes
    __device__ static int vswz(int t) { return D == 128 ? 2 * (t & 7) : 2 * ((t >> 1) & 3); }
};
template <int D>
struct KvT<KV_I8, D> {
    static constexpr int ESZ = 1, KLOADS = D / 64, NJ = D / 32;
    static constexpr int VL = D / 16, NV = kHalf * VL / 64;
    static constexpr int LDS_ESZ = 1;
    __device__ static int kdoff(int c, int q4) { return 64 * c + 16 * q4; }
    __device__ static int dslot(int j, int q4, int s) { return 64 * (j >> 1) + 16 * q4 + 8 * (j & 1) + s; }
    // a half-wave reads rows {0-3, 4-7, 16-19, 20-23} (or the other 16): 16 chunks at distinct
    // offsets mod 256 bytes
    __device__ static int vswz(int t) {
        return D == 128 ? (((t >> 1) & 3) | ((t >> 2) & 4)) : (((t >> 2) & 1) | ((t >> 3) & 2));
    }
};
template <int D>
struct KvT<KV_F32, D> {
    static constexpr int ESZ = 4, KLOADS = D / 16, NJ = D / 4;
    static constexpr int VL = D * 4 / 16, NV = kHalf * VL / 64;
    static constexpr int LDS_ESZ = 4;
    __device__ static int kdoff(int c, int q4) { return 16 * c + 4 * q4; }
    __device__ static int dslot(int j, int q4, int /*s*/) { return 16 * (j >> 2) + 4 * q4 + (j & 3); }
    __device__ static int swz(int t) { return 4 * ((t >> 2) & 1); }
};

// Raw registers of one 32-token tile.
template <int KIND, int D>
struct TileRegs {
    using T = KvT<KIND, D>;
    uint4 k[2][T::KLOADS];
    uint4 v[2][T::NV];
    // int8: K and V scales of the tokens this lane holds in the score layout (FAST: one per half)
    float ks[KIND == KV_I8 ? 8 : 1], vs[KIND == KV_I8 ? 8 : 1];
    // FAST with the partition's blocks in lanes: each half's block, relative to the partition's first
    int rel[2];
};

// ---- the kernel ---------------------------------------------------------------------------------

// ---- longest-first work order for ragged batches ---------------------------------------------
// With DecodeParams::ragged_items set, grid y enumerates work items rather than (sequence,
// partition) pairs: first every full partition (len / part_tokens per sequence, in sequence order),
// then each sequence's partial last partition, longest first (ties: lower sequence first), then one
// item per empty sequence (whose output is written as 0). The longest pieces start first and the
// short ones fill the end; in the plain order the partial last partitions of the longest sequences
// started last, and the step ended on them (c5: 363 -> 341 us fp16, 203 -> 183 us int8 on MI355X).
// A partition is computed by the same code whatever its position, so the results are the same bits.
// Each wave finds its workgroup's item from seq_lens, one lane per sequence.
struct WorkItem {
    int b, part;  // b < 0: no such item (the host's lengths and seq_lens disagree)
};

// Inclusive prefix sum over the 64 lanes with DPP: row shifts 1, 2, 4, 8 within each 16-lane row,
// then row 0's total into row 1 and row 2's into row 3 (row_bcast:15), then rows 0-1's into rows
// 2-3 (row_bcast:31). Lanes a shift or a row mask leaves out read the `old` operand, 0.
__device__ __forceinline__ int wave_inclusive_sum(int x) {
    x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xF, 0xF, false);  // row_shr:1
    x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xF, 0xF, false);  // row_shr:2
    x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xF, 0xF, false);  // row_shr:4
    x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xF, 0xF, false);  // row_shr:8
    x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xA, 0xF, false);  // row_bcast:15, rows 1 and 3
    x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xC, 0xF, false);  // row_bcast:31, rows 2 and 3
    return x;
}

// Item i of `items` (the launch's grid y, counted by the host from its copy of the lengths). If the
// lengths in seq_lens (clamped by live_len) make a different number of items, the two copies
// disagree: every workgroup then gets no item and the launch does nothing, rather than leave some
// partitions unlaunched and their group's arrival counter short of its count for later launches.
__device__ __forceinline__ WorkItem ragged_item(const int32_t* seq_lens, int batch, int part_tokens, int len_cap,
                                                int i, int items) {
    constexpr int E = kRaggedMaxBatch / 64;
    const int lane = threadIdx.x & 63;
    const int ne = (batch + 63) >> 6;
    int len[E];
    for (int e = 0; e < E; ++e) len[e] = (e < ne && 64 * e + lane < batch) ? live_len(seq_lens, 64 * e + lane, len_cap) : 0;
    WorkItem r{-1, 0};
    // full partitions, in sequence order: an exclusive scan of len / part_tokens
    int before = 0;
    for (int e = 0; e < E && e < ne; ++e) {
        const int f = len[e] / part_tokens;
        const int s = wave_inclusive_sum(f);
        const int excl = before + s - f;
        const unsigned long long hit = __ballot(f > 0 && excl <= i && i < excl + f);
        if (hit) {
            const int l = __ffsll(hit) - 1;
            r = WorkItem{64 * e + l, i - __builtin_amdgcn_readlane(excl, l)};
        }
        before += __builtin_amdgcn_readlane(s, 63);
    }
    // partial last partitions: keys rem << 16 | (0xFFFF - b) (distinct; 0 marks a sequence without
    // one); then the empty sequences
    int npart = 0, nempty = 0;
    unsigned key[E];
    for (int e = 0; e < E; ++e) {
        const int rem = len[e] % part_tokens;
        key[e] = (e < ne && rem > 0) ? ((unsigned)rem << 16) | (0xFFFFu - (unsigned)(64 * e + lane)) : 0u;
        if (e < ne) {
            npart += __popcll(__ballot(key[e] != 0u));
            nempty += __popcll(__ballot(len[e] == 0 && 64 * e + lane < batch));
        }
    }
    if (before + npart + nempty != items) return WorkItem{-1, 0};  // uniform: the lengths disagree
    if (r.b < 0) {
        // partial last partitions, longest first: the (i - full)-th largest key, found bit by bit
        // from the top
        int j = i - before;
        if (j < npart) {
            unsigned want = 0;
            const int top = 16 + (32 - __builtin_clz((unsigned)part_tokens));  // keys < 2^top
            for (int bit = min(top, 32) - 1; bit >= 0; --bit) {
                const unsigned cand = want | (1u << bit), hi = ~0u << bit;
                int cnt = 0;
                for (int e = 0; e < E && e < ne; ++e) cnt += __popcll(__ballot((key[e] & hi) == cand));
                if (j < cnt) want = cand;
                else j -= cnt;
            }
            const int b = 0xFFFF - (int)(want & 0xFFFFu);
            int lb = 0;
            for (int e = 0; e < E && e < ne; ++e)
                if (e == (b >> 6)) lb = __builtin_amdgcn_readlane(len[e], b & 63);
            r = WorkItem{b, lb / part_tokens};
        } else {
            // empty sequences, in sequence order
            int k = j - npart;
            for (int e = 0; e < E && e < ne; ++e) {
                const unsigned long long m = __ballot(len[e] == 0 && 64 * e + lane < batch);
                const int c = __popcll(m);
                if (r.b < 0 && k < c) {
                    const int rank = __popcll(m & ((1ull << lane) - 1ull));
                    const unsigned long long hit = __ballot(((m >> lane) & 1ull) && rank == k);
                    r = WorkItem{64 * e + __ffsll(hit) - 1, 0};
                }
                k -= c;
            }
        }
    }
    return WorkItem{__builtin_amdgcn_readfirstlane(r.b), __builtin_amdgcn_readfirstlane(r.part)};
}

// (waves_per_eu: the register budget. 2 waves per SIMD (two workgroups per CU) leave 256 VGPRs per
// lane. The tile-aligned int8 kernel is held to 3 (168 VGPRs, no spills), so that three of its
// workgroups share a CU on multi-round grids; at 169 VGPRs it would drop to two. With one query head
// per workgroup it would spill there, so that case keeps 2, as do the PAIR kernels, which run one
// workgroup per CU.)
// LOADS: the measurement variant (kvb_run_paged_loads). It issues every load of the decode in the
// same order and consumes the registers with XORs, and computes and writes nothing.
// PAIR: a workgroup computes two consecutive partitions (grid z = ceil(max_parts / 2)), so that a grid
// of two or more workgroups per CU runs as one per CU (DecodeParams::pair). Its waves walk the two
// partitions' tiles in order; each partition's tiles go to the same waves, in the same order, as in
// a workgroup of its own (part_tokens is a multiple of 32 * waves), and a wave starts its second
// partition from a fresh state, so every partition gets the same bits either way.
// QG is the workgroup's query heads. Past 16 its waves split them (decode_shape: QW heads per wave,
// HS head splits of TS token streams): a wave walks its stream's tiles for its split's heads. int8:
// each tile is read by HS waves, the first from HBM and the others mostly from the CU's caches, with
// ordinary loads; fp16: the stream's two waves load half a tile each and share it through LDS (SHL).
template <int KIND, int D, int QG, bool FAST, bool LOADS = false, bool PAIR = false, bool PART = false,
          bool SHARE = false, bool STAGE = false>
__global__ __launch_bounds__(64 * decode_wg_waves(KIND, QG)) __attribute__((amdgpu_waves_per_eu(
    decode_wg_waves(KIND, QG) > 4 ? 2
    : decode_shape(KIND, QG).qw > 8 ? 1
    : KIND == KV_I8 && FAST && !LOADS && !PAIR && QG > 1 ? 3 : 2))) void paged_decode_kernel(DecodeParams p) {
    using T = KvT<KIND, D>;
    using R = TileRegs<KIND, D>;
    constexpr DecodeShape DS = decode_shape(KIND, QG);
    constexpr int QW = DS.qw, HS = DS.hs, TS = DS.ts, W = HS * TS;
    constexpr int NJ = T::NJ, VL = T::VL, NV = T::NV, NMB = D / 16;
    constexpr bool F32 = KIND == KV_F32;
    static_assert(QG == 1 || QG == 2 || QG == 4 || QG == 8 || (QG == 16 && KIND != KV_F32) || (QG == 32 && KIND != KV_F32),
                  "QG must be 1, 2, 4, 8 or (fp16, int8) 16 or 32");
    static_assert(HS == 1 || (!PART && !PAIR), "head splits serve whole groups, one partition per workgroup");
    static_assert(QW * HS == QG && (QW <= 8 || (QW == 16 && KIND != KV_F32)), "decode_shape");
    // Up to 8 heads per wave, the score MFMA's 16 columns hold each head twice (a high and a low
    // column). With 16 heads per wave (COLH) a column holds one head: its high and low parts run as
    // two MFMAs (int8: its three digits as three) and the P*V products as two, into separate high and
    // low accumulators, so every lane of the softmax serves a head of its own and a 16-head tile costs
    // the softmax instructions of an 8-head one. Same products, same sums, same order: a 16-head wave
    // gives each head the bits of an 8-head wave. (The two-block form it replaced, two 8-head blocks
    // per tile, ran fp16 at 4 x 32k tokens with 16 heads per KV head in 87.1 us, and int8 in 149.3.)
    constexpr bool COLH = QW == 16;
    constexpr int NA = COLH ? 2 : 1;      // accumulator sets: one, or (COLH) high and low
    constexpr int HQ = COLH ? 16 : 8;     // rows of a wave's state in LDS (heads, the ones past qg unread)
    // Lazy rescaling (16-head waves): the running max m is a reference that moves only when a tile's
    // max passes it by more than kLazyRescale (p <= 2^8, in range for the fp16 parts), and the true
    // max mt is kept beside it for the partition's stored state. A 16-head wave's accumulators live
    // in AGPRs, where a rescale costs a read, a multiply and a write per value, and with 16 heads some
    // head's max grows on most tiles (about 27 of a c4 wave's 32). 8-head waves rescale eagerly.
    constexpr bool LAZY = COLH;
    constexpr float kLazyRescale = 8.0f;
    // SHL (fp16, two head splits): the two waves of a stream share each tile through LDS. The first
    // split's wave loads the tile's K rows, the second's its V rows, each into a half-tile register
    // buffer (32 VGPRs at head_dim 128 where a whole tile takes 64); both write their half to the
    // stream's LDS slot (two per stream, alternating), meet at the stream's LDS counter, and compute
    // the tile from the slot. Each tile is read from HBM once, two tiles are in flight per stream,
    // and the registers left free fit four streams at two waves per SIMD. (Read by each split from
    // the CU's caches instead, four streams of fp16 tiles at head_dim 128 outgrew them and the second
    // reads went back to HBM: 165 us at 4 x 32k tokens with 32 query heads per KV head, against 108
    // for two streams.)
    constexpr bool SHL = HS == 2 && KIND == KV_F16;
    // Tile register buffers per wave: one computed while the next is loaded (see the tile walk).
    // fp32 tiles are too large for more than one. (Three for int8, whose tiles are half an fp16
    // tile, spill at head_dim 128 and measured slower.)
    constexpr int NBUF = F32 ? 1 : 2;
    // Cache policy of the K/V tile loads: non-temporal when one workgroup reads each page; ordinary
    // with SHARE, whose sibling workgroups read each page again from L2 (MI355X, c4's size with
    // groups of 16: 163.5 -> 106.9 us fp16, 88.2 -> 68.0 int8, against 133.7 / 80.9 with the sibling
    // order alone; non-temporal stays for one workgroup per KV head: 84.5 us there, 93.9 without).
    // Head splits (HS > 1) read each tile once per split: ordinary loads, as SHARE (SHL: once).
    constexpr int kKvPolicy = SHARE || (HS > 1 && !SHL) ? 0 : kNonTemporal;

    // Per wave: the V tile (32 rows of D elements, swizzled); after the loop it holds the wave's
    // final accumulators [HQ][D] fp32 for the merge (every head row is written, the ones past qg
    // unread): the larger of the two.
    // SHL: [W][one tile's K and V]: the two slots of stream s are s_v[2 s] and s_v[2 s + 1] (K rows
    // as loaded, lane-major, then the V tile), and wave w's final accumulators go to s_v[w] after the
    // walk.
    constexpr int SKB = kTok * D * T::LDS_ESZ;  // SHL: the K half of a slot
    constexpr int SVB = SHL ? (2 * SKB >= HQ * D * 4 ? 2 * SKB : HQ * D * 4)
                            : kTok * T::LDS_ESZ >= HQ * 4 ? kTok * D * T::LDS_ESZ : HQ * D * 4;
    __shared__ __attribute__((aligned(16))) unsigned char s_v[W][SVB];
    __shared__ float2 s_ml[W][QW];
    __shared__ float s_mt[LAZY ? W : 1][QW];  // LAZY: each wave's true max per head
    // PAIR: each wave's state for the first partition, [QG][D] fp32 and (m, l), as the V tile holds
    // the last partition's after the walk (room for 8 heads at least: state_to_lds writes all 8 of a
    // head block, the heads past qg unread)
    __shared__ __attribute__((aligned(16))) float s_part[PAIR ? W : 1][PAIR ? HQ * D : 4];
    __shared__ float2 s_ml2[PAIR ? W : 1][QW];
    __shared__ float s_mt2[PAIR && LAZY ? W : 1][QW];

    // Grid (H / qg, B, max_parts), head group fastest: workgroups go to the 8 XCDs round robin by
    // linear id, so consecutive ids (one partition of consecutive head groups and sequences) spread
    // every partition's work over all XCDs. With the partition fastest, the XCD followed the
    // partition index, and the partitions that short sequences leave empty left XCDs idle (c5
    // fp16: 486 -> 366 us; equal lengths under a longer max_len ran 1.7x slower).
#ifdef KVB_WG_TIMESTAMPS
    const unsigned long long ts0 = __builtin_amdgcn_s_memrealtime();
    const unsigned lin = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
#endif
    constexpr int G = PAIR ? 2 : 1;  // partitions per workgroup
    // SHARE: a KV head has S = group / qg > 1 workgroups (its query heads in S blocks), which read the
    // same pages. Their ids are remapped to lie 8 apart, so that they run on one XCD (workgroups go
    // to the XCDs round robin by linear id) at about the same time, and the later reads of a page
    // hit that XCD's L2; the loads are then ordinary (temporal) loads. In blocks of 8 * S ids: id
    // i of a block is sibling i / 8 of unit 8 * block + i % 8, units being (KV head, y, z) in the
    // plain order (KV head fastest). Only when the units fill whole blocks; otherwise the plain order.
    int bx = blockIdx.x, by = blockIdx.y, bz = blockIdx.z;
    if constexpr (SHARE) {
        const unsigned S = p.group / (PART ? p.qg : QG), X = gridDim.x, Y = gridDim.y, Z = gridDim.z;
        const unsigned XK = X / S;  // KV heads
        if (S > 1 && (XK * Y * Z) % 8 == 0) {
            const unsigned id = blockIdx.x + X * (blockIdx.y + Y * blockIdx.z);
            const unsigned blk = id / (8 * S), within = id % (8 * S);
            const unsigned unit = 8 * blk + within % 8, yz = unit / XK;
            bx = (int)((unit % XK) * S + within / 8);
            by = (int)(yz % Y);
            bz = (int)(yz / Y);
        }
    }
    int part = bz * G, b = by;  // part: the workgroup's first partition
    if (p.ragged_items) {
        const WorkItem it = ragged_item(p.seq_lens, p.batch, p.part_tokens, p.len_cap, by, gridDim.y);
        if (it.b < 0 || it.b >= p.batch || it.part >= p.max_parts) return;  // uniform, before any barrier
        b = it.b;
        part = it.part;
    }
    // Query heads of this workgroup: QG, or with PART the group's p.qg < QG (the MFMA columns past
    // them idle). A full group keeps the count a constant, so its column masks fold away.
    const int NQ = PART ? p.qg : QG;
    const int h0 = bx * NQ;
    const int len = live_len(p.seq_lens, b, p.len_cap);  // nparts <= max_parts, t1 <= max_blocks * P
    const int t0 = part * p.part_tokens;
    const int H = p.num_heads, Hkv = p.num_kv_heads, P = p.page_size;
    if (t0 >= len) {  // uniform over the workgroup, before any barrier
        // fused merge: an empty sequence attends to nothing, its output is exactly 0
        if (p.out && len == 0 && part == 0)
            for (int idx = threadIdx.x; idx < NQ * D; idx += 64 * W) p.out[((size_t)b * H + h0) * D + idx] = 0.0f;
        return;
    }
    const int t1 = min(len, t0 + G * p.part_tokens);
    const int ng = PAIR ? (t1 - t0 + p.part_tokens - 1) / p.part_tokens : 1;  // partitions holding tokens
    const int kvh = h0 / p.group;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // The wave's token stream (its tiles: stream, stream + TS, ...) and head split (its heads: hw0 ..
    // hw0 + NQW - 1). One split: the wave's stream is its index and it serves the workgroup's heads.
    const int stream = HS == 1 ? wave : wave % TS;
    const int hw0 = HS == 1 ? h0 : h0 + (wave / TS) * QW;
    const int NQW = HS == 1 ? NQ : QW;
    const int c = lane & 15, q4 = lane >> 4;  // MFMA: column (stack row of q) / token row, row quad
    // Per tile, outside the lanes case below: the block table is read through the constant address
    // space (nothing writes it during the kernel), so the wave-uniform reads are scalar loads, whose
    // counter (lgkmcnt) is separate from the K/V loads'. As vector loads, the wait for a block id
    // (vmcnt counts in order) would also wait for every tile still in flight; a block id is waited
    // for as soon as it is read. The int8 scales are the opposite case: nothing waits for them until
    // the tile's arithmetic, so they are vector (buffer) loads, counted by vmcnt in order with the
    // tile they belong to, whose own wait covers them. As scalar loads they were still outstanding
    // when the arithmetic began, and every LDS wait there (lgkmcnt is shared with scalar loads, which
    // return out of order and so can only be waited to zero) waited for them as well: with cold
    // caches an HBM round trip per tile (c3 int8 on MI355X: 48.3 us per step that way, 46.5 us with
    // the scales in lanes).
    const const_i32 bt = (const_i32)p.block_table + (size_t)b * p.max_blocks;
    // STAGE (the any-page path): each lane finds the block of its own rows, so its lookups are
    // vector reads, and a vector load of a block id would be waited for together with every tile
    // still in flight (vmcnt counts in issue order), which serialises the walk. The range's block
    // ids are copied into LDS once instead, and a lookup is an LDS read. (MI355X, c4's size with
    // 8-token pages: see the tile walk.)
    static_assert(!STAGE || !FAST, "STAGE is an any-page variant");
    __shared__ int s_tab[STAGE ? kTableStage : 1];
    const int tb0 = fast_div(t0, p.page_div);
    if constexpr (STAGE) {
        const int nbs = fast_div(t1 - 1, p.page_div) - tb0 + 1;  // <= kTableStage (host-checked)
        for (int i = threadIdx.x; i < nbs; i += 64 * W) s_tab[i] = p.block_table[(size_t)b * p.max_blocks + tb0 + i];
        __syncthreads();
    }
    auto block_of = [&](int bi) -> int {
        if constexpr (STAGE) return s_tab[bi - tb0];
        else return bt[bi];
    };
    const const_f32 ksc = (const_f32)p.k_scale, vsc = (const_f32)p.v_scale;
    const __amdgpu_buffer_rsrc_t rks = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(p.k_scale), (short)0,
                                                                         0x7fffffff, 0x00020000);
    const __amdgpu_buffer_rsrc_t rvs = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(p.v_scale), (short)0,
                                                                         0x7fffffff, 0x00020000);
    // FAST, when a partition touches at most kLaneBlocks blocks (p.table_in_lanes): lane i of every
    // wave holds the id of the partition's (bi0 + i)-th block and, for int8, its K and V scales, loaded
    // once, here. A tile then takes its block id and scales with v_readlane: no scalar load and wait per
    // tile in the load path, and no scale load in flight during the arithmetic. (One register per
    // value: an array indexed at run time would be placed in LDS, a read and a wait per lookup.)
    const bool lanes = FAST && p.table_in_lanes;
    const int bi0 = fast_div(t0, p.page_div);
    int blkv = 0;  // loaded below, after q's loads are issued
    float ksv = 0.0f, vsv = 0.0f;
    auto lane_block = [&](int rel) { return __builtin_amdgcn_readlane(blkv, rel); };
    const char* kbase = static_cast<const char*>(p.k);
    const char* vbase = static_cast<const char*>(p.v);
    unsigned char* vt = s_v[wave];

    // ---- tile loads (no branches around them, so the compiler can keep a tile in flight)
    // Tile-aligned int8 (KFIRST): the K rows of both halves go out before the V rows of either, so
    // each pool is read in runs of a whole tile (32 rows, 4 KB at head_dim 128) instead of alternating
    // between K and V every half tile. MI355X, against the interleaved order: c5 int8 182.5-182.9 us
    // against 186.0-186.7, c4's shape in int8 46.9-47.1 against 47.9, c3 even. fp16 keeps the
    // interleaved order: K first made c2 28.0-28.1 us against 27.6-27.7, and c5 fp16 339 against 335.
    constexpr bool KFIRST = FAST && KIND == KV_I8;
    auto load_tile = [&](R& r, int tt) {
        int braw = 0, off = 0;  // FAST: the block id of the half tile and its first row in the page
        __amdgpu_buffer_rsrc_t rvh[KFIRST ? 2 : 1];  // KFIRST: each half's V resource, for after both K
        for (int h = 0; h < 2; ++h) {
            const int th = tt + h * kHalf;  // first token of this half tile
            if constexpr (FAST) {
                // [th, th+16) lies in one page: one block id and a buffer resource over exactly its
                // live rows; a half at or past t1 (the prefetch after the last tile) gets an empty one.
                // With tile_in_page the whole 32-token tile lies in one page (its first token is a
                // multiple of 32), so the second half takes the first half's block, 16 rows further.
                // A block id of -1 (an unused table entry, reachable only when seq_lens disagrees with
                // the host's lengths) reads as an empty page.
                const int tc = min(th, t1 - 1);
                if (h == 0 || !p.tile_in_page) {
                    const int bi = fast_div(tc, p.page_div);
                    r.rel[h] = bi - bi0;
                    braw = lanes ? lane_block(bi - bi0) : bt[bi];
                    off = tc - bi * P;
                } else {
                    r.rel[h] = r.rel[0];
                    off += kHalf;
                }
                const int blk = max(braw, 0);
                const size_t row0 = ((size_t)blk * Hkv + kvh) * P + off;
                // (readfirstlane between the min and the max: the value is wave-uniform, and fused
                // into one v_med3 it would land in a VGPR the prefetch may be writing)
                const int rows = braw < 0 ? 0 : max(0, __builtin_amdgcn_readfirstlane(min(kHalf, t1 - th)));
                const int nbytes = rows * D * T::ESZ;
                const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
                    const_cast<char*>(kbase + row0 * D * T::ESZ), (short)0, nbytes, 0x00020000);
                const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
                    const_cast<char*>(vbase + row0 * D * T::ESZ), (short)0, nbytes, 0x00020000);
                for (int m = 0; m < T::KLOADS; ++m)
                    r.k[h][m] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                                                              rk, (c * D + T::kdoff(m, q4)) * T::ESZ, 0, kKvPolicy));
                if constexpr (KFIRST) {
                    rvh[h] = rv;
                } else {
                    for (int i = 0; i < NV; ++i)
                        r.v[h][i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                                                                  rv, (i * (64 / VL) + lane / VL) * D * T::ESZ + (lane % VL) * 16, 0, kKvPolicy));
                }
                if constexpr (KIND == KV_I8) {
                    // (with tile_in_page the second half's scales are the first half's: the arithmetic
                    // selects them; copying the register here would wait for its load, and so for
                    // every tile in flight)
                    if (!lanes && (h == 0 || !p.tile_in_page)) {
                        const int soff = (blk * Hkv + kvh) * 4;
                        r.ks[h] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rks, soff, 0, 0));
                        r.vs[h] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rvs, soff, 0, 0));
                    }
                }
            } else {
                // Any page size: each lane finds the block of its own token. Lanes past t1 read the
                // partition's first token (always live) and zero what they got; a block id of -1
                // reads as zeros too (from block 0).
                const int tk = th + c;
                const int tks = tk < t1 ? tk : t0;
                const int kbi = fast_div(tks, p.page_div);
                const int kid = block_of(kbi);
                const bool kval = tk < t1 && kid >= 0;
                const size_t krow = ((size_t)max(kid, 0) * Hkv + kvh) * P + (tks - kbi * P);
                const char* kb = kbase + krow * D * T::ESZ;
                for (int m = 0; m < T::KLOADS; ++m) {
                    const uint4 x = *reinterpret_cast<const uint4*>(kb + T::kdoff(m, q4) * T::ESZ);
                    r.k[h][m] = kval ? x : make_uint4(0, 0, 0, 0);
                }
                for (int i = 0; i < NV; ++i) {
                    const int tv = th + i * (64 / VL) + lane / VL;
                    const int tvs = tv < t1 ? tv : t0;
                    const int vbi = fast_div(tvs, p.page_div);
                    const int vid = block_of(vbi);
                    const bool vval = tv < t1 && vid >= 0;
                    const size_t vrow = ((size_t)max(vid, 0) * Hkv + kvh) * P + (tvs - vbi * P);
                    const uint4 x = *reinterpret_cast<const uint4*>(vbase + vrow * D * T::ESZ + (lane % VL) * 16);
                    r.v[h][i] = vval ? x : make_uint4(0, 0, 0, 0);
                }
                if constexpr (KIND == KV_I8) {
                    for (int i = 0; i < 4; ++i) {  // the score-layout tokens th + 4*q4 + i of this lane
                        const int ts = th + 4 * q4 + i;
                        const int tss = ts < t1 ? ts : t0;
                        const size_t slot = (size_t)max(block_of(fast_div(tss, p.page_div)), 0) * Hkv + kvh;
                        r.ks[4 * h + i] = ksc[slot];
                        r.vs[4 * h + i] = vsc[slot];
                    }
                }
            }
        }
        if constexpr (KFIRST)
            for (int h = 0; h < 2; ++h)
                for (int i = 0; i < NV; ++i)
                    r.v[h][i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                                                              rvh[h], (i * (64 / VL) + lane / VL) * D * T::ESZ + (lane % VL) * 16, 0, kKvPolicy));
    };

    // ---- SHL: this wave's half of a tile, K rows (split 0) or V rows (split 1), into x[h][m]: the
    // rows and buffer ranges of load_tile, each lane's row and byte of the one or the other (for
    // fp16 a half tile takes as many 16-byte loads of K as of V). Past t1 it reads zeros.
    constexpr int NL = T::KLOADS;
    static_assert(!SHL || T::NV == T::KLOADS, "SHL: equal K and V loads");
    const int split = HS == 1 ? 0 : wave / TS;
    const char* hbase = split ? vbase : kbase;
    auto hrow = [&](int m) { return split ? m * (64 / VL) + lane / VL : c; };              // row of the half tile
    auto hcol = [&](int m) { return split ? (lane % VL) * 16 : T::kdoff(m, q4) * T::ESZ; };  // its byte
    auto load_half = [&](uint4 (&x)[2][NL], int tt) {
        int braw = 0, off = 0;
        for (int h = 0; h < 2; ++h) {
            const int th = tt + h * kHalf;
            if constexpr (FAST) {  // (load_tile's rows and range)
                const int tc = min(th, t1 - 1);
                if (h == 0 || !p.tile_in_page) {
                    const int bi = fast_div(tc, p.page_div);
                    braw = lanes ? lane_block(bi - bi0) : bt[bi];
                    off = tc - bi * P;
                } else {
                    off += kHalf;
                }
                const size_t row0 = ((size_t)max(braw, 0) * Hkv + kvh) * P + off;
                const int rows = braw < 0 ? 0 : max(0, __builtin_amdgcn_readfirstlane(min(kHalf, t1 - th)));
                const __amdgpu_buffer_rsrc_t rh = __builtin_amdgcn_make_buffer_rsrc(
                    const_cast<char*>(hbase + row0 * D * T::ESZ), (short)0, rows * D * T::ESZ, 0x00020000);
                for (int m = 0; m < NL; ++m)
                    x[h][m] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                                                            rh, hrow(m) * D * T::ESZ + hcol(m), 0, kKvPolicy));
            } else {
                for (int m = 0; m < NL; ++m) {
                    const int tk = th + hrow(m);
                    const int tks = tk < t1 ? tk : t0;
                    const int bi = fast_div(tks, p.page_div);
                    const int id = block_of(bi);
                    const size_t row = ((size_t)max(id, 0) * Hkv + kvh) * P + (tks - bi * P);
                    const uint4 v = *reinterpret_cast<const uint4*>(hbase + row * D * T::ESZ + hcol(m));
                    x[h][m] = tk < t1 && id >= 0 ? v : make_uint4(0, 0, 0, 0);
                }
            }
        }
    };
    // the half into the slot: K lane-major (each lane reads back its own offsets), V as store_v
    // lays it out
    auto put_half = [&](unsigned char* slot, const uint4 (&x)[2][NL]) {
        if constexpr (SHL)
            for (int h = 0; h < 2; ++h)
                for (int m = 0; m < NL; ++m) {
                    int o;
                    if (split == 0) {
                        o = ((h * NL + m) * 64 + lane) * 16;
                    } else {
                        const int t = h * kHalf + m * (64 / VL) + lane / VL;
                        o = SKB + t * D * T::LDS_ESZ + 16 * ((lane % VL) ^ T::vswz(t));
                    }
                    *reinterpret_cast<u32x4_t*>(slot + o) = __builtin_bit_cast(u32x4_t, x[h][m]);
                }
    };

    // ---- q as the B operand of S^T = K Q^T: column c holds head c/2, high (c even) or low part;
    // COLH, head c, whose high and low parts (int8: digits) go to separate MFMAs.
    // Its loads go out first, then the wave's first NBUF - 1 tiles; the q split then runs under
    // the tiles' latency. (vmcnt counts loads in the order they were issued: a q load issued
    // after the tiles could only be waited for together with them.)
    const int hh = COLH ? c : c >> 1, hl = COLH ? 0 : c & 1;  // the column's head (of the wave's), its part
    const bool qcol = hh < NQW;
    float up;  // scores are MFMA results times `up` (a power of two; fp16: per 8 heads, int8: per head)
    half8_t aq16[KIND == KV_F16 ? NA : 1][KIND == KV_F16 ? NJ : 1];  // COLH: high parts, low parts
    float aq32[F32 ? NJ : 1];
    // int8: q digits of the score MFMAs (d0 + d2 and d1 + zeros; COLH: d0, d1, d2), KLOADS each
    i32x4_t aq8[KIND == KV_I8 ? (COLH ? 3 : 2) * T::KLOADS : 1];
    constexpr int QS = F32 ? 1 : 8;  // q elements per MFMA slot
    float qv[NJ][QS];                // raw loads only: any use before the barrier below would wait for them
    {
        const float* qp = p.q + ((size_t)b * H + hw0 + (qcol ? hh : 0)) * D;
        for (int j = 0; j < NJ; ++j)
            for (int s = 0; s < QS; ++s) qv[j][s] = qp[T::dslot(j, q4, s)];
    }
    // the partition's blocks (and int8 scales) into lanes: their round trip overlaps q's
    if (lanes) {
        const int nb = fast_div(t1 - 1, p.page_div) - bi0 + 1;  // <= kLaneBlocks (host-checked)
        if (lane < nb) blkv = p.block_table[(size_t)b * p.max_blocks + bi0 + lane];
        if constexpr (KIND == KV_I8) {
            const int soff = lane < nb ? (max(blkv, 0) * Hkv + kvh) * 4 : 0;
            ksv = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rks, soff, 0, 0));
            vsv = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rvs, soff, 0, 0));
        }
    }

    const int ntiles = (t1 - t0 + kTok - 1) / kTok;
    int it = stream;
    R r[SHL ? 1 : NBUF];
    uint4 x[SHL ? 2 : 1][2][NL];  // SHL: the stream's next two tiles, this wave's halves
    if constexpr (SHL) {
        for (int k = 0; k < 2; ++k) {
            load_half(x[k], t0 + (it + k * TS) * kTok);
            __builtin_amdgcn_sched_barrier(0);
        }
    } else {
        for (int k = 0; k + 1 < NBUF; ++k) {
            load_tile(r[k], t0 + (it + k * TS) * kTok);
            // (in buffer order, as the loop issues them: the loop head is entered from here and from the
            // back edge, and the wait for buffer 0 there can leave the later buffers in flight only if
            // both paths issued them in the same order)
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    // (an empty asm with a memory clobber: without it the tile loads are sunk past the q split, to
    // their first use, and the q loads past the tiles')
    asm volatile("" ::: "memory");

    up = 1.0f;
    for (int j = 0; j < NJ; ++j)
        for (int s = 0; s < QS; ++s) qv[j][s] = (qcol && (!F32 || hl == 0)) ? qv[j][s] * p.qscale : 0.0f;
    if constexpr (F32) {
        for (int j = 0; j < NJ; ++j) aq32[j] = qv[j][0];
    } else {
        float amax = 0.0f;
        bool finite = true;
        for (int j = 0; j < NJ; ++j)
            for (int s = 0; s < 8; ++s) {
                const float a = fabsf(qv[j][s]);
                amax = fmaxf(amax, a);
                finite = finite && a <= 3.402823466e38f;
            }
        // fp16: one scale for the wave's 8 heads (COLH: for each 8 of its 16, columns 0-7 and 8-15,
        // as two 8-head waves would take), floating point keeping each element's relative precision.
        // int8: one per head, over the lanes holding it (columns 2h, 2h + 1 or, COLH, column h; all
        // q4): the digits are fixed point, so a head with a small q next to a large one keeps its own
        // precision.
        if constexpr (KIND == KV_I8) {
            if (!finite) amax = __builtin_inff();  // (the max carries it to the head's other lanes)
            amax = max_x16_x32(amax);
            if constexpr (!COLH) amax = fmaxf(amax, dpp<kQuadSwap1>(amax));
        } else if constexpr (COLH) {
            for (int x = 1; x < 8; x <<= 1) amax = fmaxf(amax, __shfl_xor(amax, x));
            amax = max_x16_x32(amax);
        } else {
            amax = wave_max(amax);
        }
        int e = 0;
        if (amax > 0.0f && amax <= 3.402823466e38f) {
            frexpf(amax, &e);  // amax < 2^e
            // fp16: the scaled q stays below 2^14, far from overflow; int8: below 2^7, a digit's range
            e -= KIND == KV_I8 ? 7 : 14;
        }
        float down = ldexpf(1.0f, -e);
        up = ldexpf(1.0f, e);
        if (KIND == KV_I8 && !(amax <= 3.402823466e38f)) {
            // a NaN or infinite q element: the head's scores are NaN, as in floating point (the
            // digits alone would clamp it to a finite value)
            down = 0.0f;
            up = __builtin_nanf("");
        }
        if constexpr (KIND == KV_F16) {
            for (int j = 0; j < NJ; ++j)
                for (int s = 0; s < 8; ++s) {
                    const float x = qv[j][s] * down;
                    const _Float16 hi = (_Float16)x;
                    const _Float16 lo = (_Float16)(x - (float)hi);
                    if constexpr (COLH) {
                        aq16[0][j][s] = hi;
                        aq16[NA - 1][j][s] = lo;
                    } else {
                        aq16[0][j][s] = hl ? lo : hi;
                    }
                }
        } else {
            // int8 scores run on the integer MFMA, K as stored: x = q * down = d0 + d1 / 2^7 +
            // d2 / 2^14 + err, |err| <= 2^-15, each digit a signed byte (every step is exact in
            // fp32). Column 2h (hl == 0) carries d0 into the first MFMA and d2 into the second;
            // column 2h + 1 carries d1 and zeros. COLH: column h carries d0, d1 and d2 into three.
            // Slot t of load m is d = 64 m + 16 q4 + t, as K's.
            for (int m = 0; m < T::KLOADS; ++m) {
                uint32_t wa[4] = {0u, 0u, 0u, 0u}, wb[4] = {0u, 0u, 0u, 0u}, wc[4] = {0u, 0u, 0u, 0u};
                for (int t = 0; t < 16; ++t) {
                    const float x = qv[2 * m + (t >> 3)][t & 7] * down;
                    const float d0 = fminf(fmaxf(__builtin_rintf(x), -127.0f), 127.0f);
                    const float r1 = (x - d0) * 128.0f;
                    const float d1 = fminf(fmaxf(__builtin_rintf(r1), -127.0f), 127.0f);
                    const float d2 = fminf(fmaxf(__builtin_rintf((r1 - d1) * 128.0f), -127.0f), 127.0f);
                    auto byte = [&](float d) { return (uint32_t)(uint8_t)(int8_t)(int)d << (8 * (t & 3)); };
                    if constexpr (COLH) {
                        wa[t >> 2] |= byte(d0);
                        wb[t >> 2] |= byte(d1);
                        wc[t >> 2] |= byte(d2);
                    } else {
                        wa[t >> 2] |= byte(hl ? d1 : d0);
                        wb[t >> 2] |= hl ? 0u : byte(d2);
                    }
                }
                aq8[m] = i32x4_t{(int)wa[0], (int)wa[1], (int)wa[2], (int)wa[3]};
                aq8[T::KLOADS + m] = i32x4_t{(int)wb[0], (int)wb[1], (int)wb[2], (int)wb[3]};
                if constexpr (COLH) aq8[2 * T::KLOADS + m] = i32x4_t{(int)wc[0], (int)wc[1], (int)wc[2], (int)wc[3]};
            }
        }
    }

    // ---- int8: p * v_scale is split into fp16 high and low parts for the P*V MFMA. It is
    // normalised by 2^-ve, ve the exponent of the largest V scale the wave has met so far, so it
    // stays in fp16's normal range however small the scales are; when a tile brings a larger
    // scale the accumulators are rescaled by the (exact) power of two, as for a new running max,
    // and at the end they are scaled by 2^ve. (ve starts below every float exponent: 2^-160 is 0.)
    float vdown = 1.0f;
    int ve = -160;

    // ---- V tile -> LDS as stored (row-major, swizzled 16-byte chunks; int8 is widened to fp16 only
    // after the transposing read)
    auto store_v = [&](const R& r) {
        for (int h = 0; h < 2; ++h)
            for (int i = 0; i < NV; ++i) {
                const int t = h * kHalf + i * (64 / VL) + lane / VL;  // tile row
                const int ch = lane % VL;                             // 16-byte chunk of the loaded row
                int sch;
                if constexpr (F32) sch = ch ^ T::swz(t);
                else sch = ch ^ T::vswz(t);
                *reinterpret_cast<u32x4_t*>(vt + t * D * T::LDS_ESZ + 16 * sch) = __builtin_bit_cast(u32x4_t, r.v[h][i]);
            }
    };

    // ---- per-wave online-softmax state. Lane (c, q4) holds column c (head hh) for the tokens
    // 16h + 4*q4 + i of each tile (slot j = 4h + i of the P^T operand): m is uniform over the lanes
    // of a head, l is the lane's partial sum over its tokens. acc[a][mb]: O^T rows 16 mb.., set a
    // (COLH: the high parts' products, then the low parts'; else both, in columns 2h and 2h + 1).
    float m = kNegBig, l = 0.0f;
    float mt = kNegBig;  // LAZY: the true running max (m is then the reference the p are taken against)
    floatx4_t acc[NA][NMB];
    for (int a = 0; a < NA; ++a)
        for (int mb = 0; mb < NMB; ++mb) acc[a][mb] = floatx4_t{0.0f, 0.0f, 0.0f, 0.0f};

    uint32_t lsink = 0;  // LOADS: what the tiles' registers XOR to
    auto compute_tile = [&](const R& r, int tt) {
        if constexpr (LOADS) {
            for (int h = 0; h < 2; ++h) {
                for (int mm = 0; mm < T::KLOADS; ++mm) lsink ^= r.k[h][mm].x ^ r.k[h][mm].y ^ r.k[h][mm].z ^ r.k[h][mm].w;
                for (int i = 0; i < NV; ++i) lsink ^= r.v[h][i].x ^ r.v[h][i].y ^ r.v[h][i].z ^ r.v[h][i].w;
            }
            if constexpr (KIND == KV_I8)
                for (int j = 0; j < 2; ++j)
                    lsink ^= __builtin_bit_cast(uint32_t, r.ks[j]) ^ __builtin_bit_cast(uint32_t, r.vs[j]);
            (void)tt;
            return;
        }
        if constexpr (!SHL) store_v(r);  // (SHL: the tile is in LDS already)
        // S^T = K Q^T for both halves. S[a][h]: a = 0 the column's part (COLH: the high part,
        // int8 d0 + d2 / 2^14), a = 1 (COLH) the low part (int8 d1 / 2^7): the values columns 2h and
        // 2h + 1 hold in the two-column layout.
        floatx4_t S[NA][2];
        for (int h = 0; h < 2; ++h) {
            for (int a = 0; a < NA; ++a) S[a][h] = floatx4_t{0.0f, 0.0f, 0.0f, 0.0f};
            if constexpr (F32) {
                for (int j = 0; j < NJ; ++j) {
                    const uint4 w4 = r.k[h][j >> 2];
                    const uint32_t w = (j & 3) == 0 ? w4.x : (j & 3) == 1 ? w4.y : (j & 3) == 2 ? w4.z : w4.w;
                    S[0][h] = __builtin_amdgcn_mfma_f32_16x16x4f32(__builtin_bit_cast(float, w), aq32[j], S[0][h], 0, 0, 0);
                }
            } else if constexpr (KIND == KV_F16) {
                for (int a = 0; a < NA; ++a)
                    for (int j = 0; j < NJ; ++j)
                        S[a][h] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, r.k[h][j]), aq16[a][j], S[a][h], 0, 0, 0);
            } else {
                // exact integer dot products per digit; the scaled sums are the column's part
                i32x4_t SA = {0, 0, 0, 0}, SB = {0, 0, 0, 0}, SC = {0, 0, 0, 0};
                for (int m = 0; m < T::KLOADS; ++m) {
                    const i32x4_t kk = __builtin_bit_cast(i32x4_t, r.k[h][m]);
                    SA = __builtin_amdgcn_mfma_i32_16x16x64_i8(kk, aq8[m], SA, 0, 0, 0);
                    SB = __builtin_amdgcn_mfma_i32_16x16x64_i8(kk, aq8[T::KLOADS + m], SB, 0, 0, 0);
                    if constexpr (COLH) SC = __builtin_amdgcn_mfma_i32_16x16x64_i8(kk, aq8[2 * T::KLOADS + m], SC, 0, 0, 0);
                }
                if constexpr (COLH) {
                    for (int i = 0; i < 4; ++i) {
                        S[0][h][i] = __builtin_fmaf((float)SC[i], 1.0f / 16384.0f, (float)SA[i] * 1.0f);
                        S[NA - 1][h][i] = (float)SB[i] * (1.0f / 128.0f);  // (exact: a power of two)
                    }
                } else {
                    const float wa = hl ? 1.0f / 128.0f : 1.0f, wb = hl ? 0.0f : 1.0f / 16384.0f;
                    for (int i = 0; i < 4; ++i) S[0][h][i] = __builtin_fmaf((float)SB[i], wb, (float)SA[i] * wa);
                }
            }
        }
        // int8, FAST: the scales of the two halves (the first's for both with tile_in_page), from the
        // lanes that hold them when the partition's scales are in lanes
        float ksh[2], vsh[2];
        if (FAST && lanes) {
            for (int h = 0; h < 2; ++h) {
                ksh[h] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, ksv), r.rel[h]));
                vsh[h] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, vsv), r.rel[h]));
            }
        } else {
            ksh[0] = r.ks[0];
            vsh[0] = r.vs[0];
            ksh[1] = (FAST && p.tile_in_page) ? r.ks[0] : r.ks[KIND == KV_I8 ? 1 : 0];
            vsh[1] = (FAST && p.tile_in_page) ? r.vs[0] : r.vs[KIND == KV_I8 ? 1 : 0];
        }
        if constexpr (KIND == KV_I8) {
            float vmx = FAST ? fmaxf(vsh[0], vsh[1]) : 0.0f;
            if constexpr (!FAST) {
                for (int j = 0; j < 8; ++j) vmx = fmaxf(vmx, r.vs[j]);
                vmx = wave_max(vmx);
            }
            int e = ve;
            if (vmx > 0.0f) frexpf(vmx, &e);  // vmx < 2^e
            if (e > ve) {  // wave-uniform
                const float down = ldexpf(1.0f, ve - e);
                for (int a = 0; a < NA; ++a)
                    for (int mb = 0; mb < NMB; ++mb) acc[a][mb] *= down;
                ve = e;
                vdown = ldexpf(1.0f, -e);
            }
        }
        // scores of this lane's 8 tokens for head hh: high + low columns (COLH: parts), scaled,
        // masked. pb16[a]: the P^T operand of the P*V MFMAs (COLH: p's high parts, then low parts).
        half8_t pb16[NA];
        float pb32[F32 ? 8 : 1];
        {
            float s[8];
            for (int h = 0; h < 2; ++h)
                for (int i = 0; i < 4; ++i) {
                    const int j = 4 * h + i;
                    float f = up;
                    if constexpr (KIND == KV_I8) f *= FAST ? ksh[h] : r.ks[j];
                    if constexpr (COLH) s[j] = (S[0][h][i] + S[NA - 1][h][i]) * f;
                    else s[j] = (S[0][h][i] + dpp<kQuadSwap1>(S[0][h][i])) * f;
                }
            // Tokens past the partition end score kNegBig; only a partition's last tile has any, so the
            // compare-and-select runs under a wave-uniform branch. (p = exp2(kNegBig - m) below is then
            // exactly 0: m is finite, since a wave only walks tiles when its first holds a live token.)
            if (tt + kTok > t1)
                for (int j = 0; j < 8; ++j)
                    if (tt + kHalf * (j >> 2) + 4 * q4 + (j & 3) >= t1) s[j] = kNegBig;
            float mx = kNegBig;
            for (int j = 0; j < 8; ++j) mx = fmaxf(mx, s[j]);
            mx = max_x16_x32(mx);
            float mn;
            if constexpr (LAZY) {
                mt = fmaxf(mt, mx);
                mn = mx > m + kLazyRescale ? mt : m;  // (the first live tile always moves it)
            } else {
                mn = fmaxf(m, mx);
            }
            const float corr = __builtin_amdgcn_exp2f(m - mn);
            m = mn;
            float psum = 0.0f;
            for (int j = 0; j < 8; ++j) {
                const float pr = __builtin_amdgcn_exp2f(s[j] - mn);
                psum += pr;
                float pv = pr;
                const float xs = KIND == KV_I8 ? (FAST ? vsh[j >> 2] : r.vs[j]) * vdown : 1.0f;
                if constexpr (KIND == KV_I8) pv *= xs;
                if constexpr (F32) {
                    pb32[j] = hl ? 0.0f : pv;
                } else {
                    if constexpr (COLH) {
                        // (the low part as p * xs - hi from the exact product, the form the 8-head
                        // build takes)
                        const _Float16 hi = pinned((_Float16)pv);
                        pb16[0][j] = hi;
                        pb16[NA - 1][j] = (_Float16)__builtin_fmaf(pr, xs, -(float)hi);
                    } else {
                        const _Float16 hi = (_Float16)pv;
                        pb16[0][j] = hl ? (_Float16)(pv - (float)hi) : hi;
                    }
                }
            }
            l = l * corr + psum;
            // corr is 1 for every head whose running max did not grow: skip the no-op rescale (the
            // accumulators may live in AGPRs, where a multiply costs two moves as well)
            if (__builtin_amdgcn_ballot_w64(corr != 1.0f) != 0)
                for (int a = 0; a < NA; ++a)
                    for (int mb = 0; mb < NMB; ++mb) acc[a][mb] *= corr;
        }
        // LDS ops of one wave execute in order; the fence keeps the compiler from moving the V^T
        // reads above the stores.
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        // O^T += V^T P^T, 16 rows of d per MFMA
        for (int mb = 0; mb < NMB; ++mb) {
            const int d = 16 * mb + c;
            if constexpr (F32) {
                for (int u = 0; u < 8; ++u) {
                    const int t = 16 * (u >> 2) + 4 * q4 + (u & 3);
                    const float va = *reinterpret_cast<const float*>(vt + t * D * 4 + 16 * ((d >> 2) ^ T::swz(t)) + 4 * (d & 3));
                    acc[0][mb] = __builtin_amdgcn_mfma_f32_16x16x4f32(va, pb32[u], acc[0][mb], 0, 0, 0);
                }
            } else if constexpr (KIND == KV_F16) {
                // two reads: tokens 4 q4 + k, then 16 + 4 q4 + k (k < 4), of column d
                const int t0 = 4 * q4 + (c >> 2), t1 = 16 + t0, ch = (16 * mb + 4 * (c & 3)) >> 3, off = 8 * (c & 1);
                const fp16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4f16(
                    (lds_fp16x4_t*)(vt + t0 * D * 2 + 16 * (ch ^ T::vswz(t0)) + off));
                const fp16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4f16(
                    (lds_fp16x4_t*)(vt + t1 * D * 2 + 16 * (ch ^ T::vswz(t1)) + off));
                const half8_t va = __builtin_bit_cast(half8_t, (fp16x8_t){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]});
                for (int a = 0; a < NA; ++a)
                    acc[a][mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pb16[a], acc[a][mb], 0, 0, 0);
            } else {
                // one read: the 8 tokens of column d as bytes, widened to exact fp16
                const int k = c >> 1, t = (k < 4 ? 0 : 12) + 4 * q4 + k;
                const i32x2_t x = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
                    (lds_i32x2_t*)(vt + t * D + 16 * (mb ^ T::vswz(t)) + 8 * (c & 1)));
                const half8_t va = i8x8_to_half8(x[0], x[1]);
                for (int a = 0; a < NA; ++a)
                    acc[a][mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pb16[a], acc[a][mb], 0, 0, 0);
            }
        }
        // the next store_v overwrites the tile: keep it after these reads
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };

    // ---- walk the tiles: buffer k holds the wave's tiles k, k + NBUF, ... Each step first waits
    // until the tile it computes has arrived (the only loads outstanding), then issues the next
    // tile's loads, then computes: one tile in flight per wave at any time, its latency under the
    // computation. Issuing the next tile before that wait instead (two in flight while waiting)
    // kept more bytes in flight per CU and was slower: on MI355X boxes where c4 ran 85.4-86.7 us
    // that way it ran 83.8-84.0 us this way, and c5 fp16 330-332 against 338 us; elsewhere the two
    // were within noise. The prefetch is unconditional (past the end it reads zeros) so no branch
    // splits the load counters the compiler tracks. The loop runs whole rounds of NBUF steps and
    // has one exit. The last round may step past the wave's last tile: such a step masks every
    // score (p = 0, corr = 1 exactly), reads zeros or masked rows, and at most renormalises the
    // int8 accumulators by a power of two, so it changes nothing. (sched_barrier: the scheduler
    // would otherwise move part of the prefetch across the wait or below the computation.)
    // ---- the wave's state -> LDS: [HQ][D] fp32 and (m, l). The lanes of column pair (2 hh, 2 hh + 1)
    // hold the high and low parts of d = 16 mb + 4 q4 + i (i < 4) of head hh; their sums form one
    // 16-byte chunk per mb, of which lane hl writes values 2 hl and 2 hl + 1 (no lane idles and no
    // branch splits the swaps from the adds). COLH: lane (hh, q4) holds both parts of its head's
    // chunk and writes it whole. Chunk c of head h's row is stored at c ^ (h & 7) so that the 8
    // heads' rows do not all start in the same LDS banks. Heads past qg (PART, or QG 4 and less) are
    // written too and never read. `live`: false writes an empty state (a wave with no tile in that
    // partition).
    auto state_to_lds = [&](float* dst, float2* dml, float* dmt, bool live) {
        const float vupf = KIND == KV_I8 ? ldexpf(1.0f, ve) : 1.0f;
        const float lsum = sum_x16_x32(l);
        for (int mb = 0; mb < NMB; ++mb) {
            float* chunk = dst + hh * D + 4 * ((4 * mb + q4) ^ (hh & 7));
            if constexpr (COLH) {
                const floatx4_t a = acc[0][mb], z = acc[NA - 1][mb];
                float4 v = make_float4(a[0] + z[0], a[1] + z[1], a[2] + z[2], a[3] + z[3]);
                v = live ? make_float4(v.x * vupf, v.y * vupf, v.z * vupf, v.w * vupf) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                *reinterpret_cast<float4*>(chunk) = v;
            } else {
                // lane hl keeps values 2 hl, 2 hl + 1 and sends the other two, which its partner
                // (lane l ^ 1, the other part) keeps
                const floatx4_t a = acc[0][mb];
                const float k0 = hl ? a[2] : a[0], k1 = hl ? a[3] : a[1];
                const float x0 = hl ? a[0] : a[2], x1 = hl ? a[1] : a[3];
                float2 v = make_float2(k0 + quad_swap1(x0), k1 + quad_swap1(x1));
                v = live ? make_float2(v.x * vupf, v.y * vupf) : make_float2(0.0f, 0.0f);
                *reinterpret_cast<float2*>(chunk + 2 * hl) = v;
            }
        }
        if (hl == 0 && qcol && q4 == 0) {
            dml[hh] = live ? make_float2(m, lsum) : make_float2(kNegBig, 0.0f);
            if constexpr (LAZY) dmt[hh] = live ? mt : kNegBig;
        }
    };

    // PAIR: `cur` is the partition of the range (0 or 1) the wave's state belongs to. At its first
    // tile of the second partition the wave moves its state to s_part and starts afresh.
    int cur = 0;
    const int tpp = p.part_tokens / kTok;  // tiles per partition
    if constexpr (SHL) {
        // Step j: the wave's half of tile j (two steps old) goes to slot j % 2, the half of tile j + 2
        // is issued into its registers, and once both waves of the stream have written their halves
        // both compute tile j from the slot. The two meet at the stream's counter in LDS: each adds
        // its arrival (a release: its slot writes complete first) and waits until the count holds
        // both arrivals of this step (an acquire: its slot reads follow). Slot j % 2 was last read at
        // step j - 2, before the wave's arrival at step j - 1, which the other wave waited for before
        // writing the slot again. Both waves take the same steps (their stream's tiles, in whole
        // pairs; the last pair may step past the last tile, reading zeros, and computes nothing
        // there), and each adds before it waits, so every wait ends. Only the two waves of a stream
        // wait for each other: with a workgroup barrier at every step instead, each step waited for
        // the slowest of the four streams (98.1-101.6 us against 92.3-94.3 at 4 x 32k tokens with 32
        // query heads per KV head).
        __shared__ unsigned s_pair[SHL ? TS : 1];
        if (threadIdx.x < TS) s_pair[threadIdx.x] = 0u;
        __syncthreads();
        const int wt = it < ntiles ? (ntiles - it + TS - 1) / TS : 0;
        unsigned want = 0;
        for (int rd = 0; rd < (wt + 1) / 2; ++rd) {
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                if constexpr (LOADS) {  // the same loads, consumed by XORs; nothing shared or computed
                    for (int h = 0; h < 2; ++h)
                        for (int m = 0; m < NL; ++m) lsink ^= x[k][h][m].x ^ x[k][h][m].y ^ x[k][h][m].z ^ x[k][h][m].w;
                    load_half(x[k], t0 + (it + 2 * TS) * kTok);
                    __builtin_amdgcn_sched_barrier(0);
                    it += TS;
                    continue;
                }
                unsigned char* slot = s_v[2 * stream + k];
                put_half(slot, x[k]);
                load_half(x[k], t0 + (it + 2 * TS) * kTok);
                __builtin_amdgcn_sched_barrier(0);
                __hip_atomic_fetch_add(&s_pair[stream], 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
                want += 128;  // (each of the two waves' 64 lanes adds 1)
                while (__hip_atomic_load(&s_pair[stream], __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) < want)
                    __builtin_amdgcn_s_sleep(1);
                if (it < ntiles) {  // uniform over the stream's two waves
                    R rr{};  // (K only: fp16 has no scales, and rel is read only for them)
                    for (int h = 0; h < 2; ++h)
                        for (int m = 0; m < NL; ++m)
                            rr.k[h][m] = *reinterpret_cast<const uint4*>(slot + ((h * NL + m) * 64 + lane) * 16);
                    vt = slot + SKB;
                    compute_tile(rr, t0 + it * kTok);
                }
                it += TS;
            }
        }
        vt = s_v[wave];
        __syncthreads();  // every slot is read before the waves' states overwrite them
    } else {
    const int wtiles = it < ntiles ? (ntiles - it + TS - 1) / TS : 0;
    const int rounds = (wtiles + NBUF - 1) / NBUF;
    for (int rd = 0; rd < rounds; ++rd) {
#pragma unroll
        for (int k = 0; k < NBUF; ++k) {
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // tile `it` (buffer k) has arrived
            load_tile(r[(k + NBUF - 1) % NBUF], t0 + (it + (NBUF - 1) * TS) * kTok);
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (PAIR && !LOADS) {
                if (cur == 0 && it >= tpp && it < ntiles) {  // wave-uniform
                    state_to_lds(s_part[wave], s_ml2[wave], s_mt2[LAZY ? wave : 0], true);
                    m = kNegBig;
                    mt = kNegBig;
                    l = 0.0f;
                    for (int a = 0; a < NA; ++a)
                        for (int mb = 0; mb < NMB; ++mb) acc[a][mb] = floatx4_t{0.0f, 0.0f, 0.0f, 0.0f};
                    ve = -160;
                    vdown = 1.0f;
                    cur = 1;
                }
            }
            compute_tile(r[k], t0 + it * kTok);
            it += TS;
        }
    }
    }

#ifdef KVB_WG_TIMESTAMPS
    const unsigned long long ts1 = __builtin_amdgcn_s_memrealtime();
    __shared__ unsigned long long s_loop_end[W];
    if (lane == 0) s_loop_end[wave] = ts1;
    if (LOADS && threadIdx.x == 0 && lin < kWgStampGroups) {
        unsigned long long* st = g_wg_stamps + kWgStampWords * lin;
        st[0] = ts0;
        st[1] = st[2] = st[3] = st[4] = ts1;
        st[5] = st[6] = 0;
        st[7] = wg_where();
    }
#endif
    if constexpr (LOADS) {  // (never true for real data; keeps the loads live)
        if (lsink == 0x9e3779b9u) p.part_out[threadIdx.x % D] = 1.0f;
        return;
    }

    // ---- merge: lanes -> wave state -> workgroup. The wave's last state goes to its V tile (the
    // range's last partition); PAIR, a wave that never reached the second partition: its state is
    // the first's, and the second gets an empty one.
    float* sacc = reinterpret_cast<float*>(vt);
    bool last_live = true;
    if constexpr (PAIR) {
        if (ng == 2 && cur == 0) {  // wave-uniform
            state_to_lds(s_part[wave], s_ml2[wave], s_mt2[LAZY ? wave : 0], true);
            last_live = false;
        }
    }
    state_to_lds(sacc, s_ml[wave], s_mt[LAZY ? wave : 0], last_live);
    __syncthreads();
#ifdef KVB_WG_TIMESTAMPS
    unsigned long long ts_slowest = 0;
    for (int w = 0; w < W; ++w) ts_slowest = s_loop_end[w] > ts_slowest ? s_loop_end[w] : ts_slowest;
#endif

    // The partition's result: thread e owns the 16-byte chunk ed of head eh. It weighs the waves'
    // states once, sums them in wave order, and writes the chunk with one agent-scope (sc1) store,
    // which writes through this XCD's L2 to the device coherence point, where the merging workgroup,
    // on whichever XCD, reads it.
    // PAIR: the same for each of the range's partitions (the first's states in s_part), both at
    // once: item i is chunk i % CH of partition i / CH, so at QG 4 (128 chunks) the two partitions
    // take the two halves of the workgroup instead of two rounds of half of it.
    // (one item per thread up to QG 8 with one partition; QG 16 at head_dim 128: two)
    // Head splits: head eh is head eh % QW of the waves of split eh / QW, whose TS streams are merged
    // in stream order, as the TS waves of a one-split workgroup.
    const int CH = NQ * D / 4;  // chunks per partition
    for (int item = threadIdx.x; item < ng * CH; item += 64 * W) {
        const int gp = PAIR && item >= CH ? 1 : 0;  // (ng <= 2)
        const bool lastp = gp == ng - 1;
        const int ec = item - gp * CH;
        const int eh = ec / (D / 4), ed = ec % (D / 4);
        const int w0 = HS == 1 ? 0 : (eh / QW) * TS, lh = HS == 1 ? eh : eh % QW;  // first wave, its head
        auto wml = [&](int w) { return lastp ? s_ml[w0 + w][lh] : s_ml2[PAIR ? w : 0][lh]; };
        auto wacc = [&](int w) {
            return lastp ? reinterpret_cast<const float*>(s_v[w0 + w]) : &s_part[PAIR ? w : 0][0];
        };
        float M = kNegBig;
        for (int w = 0; w < TS; ++w) M = fmaxf(M, wml(w).x);
        // LAZY: the waves' states are taken against their reference maxes; the partition's stored
        // (m, l) against the true one, Mt >= M (its o, a ratio, is the same either way)
        float Mt = M;
        if constexpr (LAZY) {
            Mt = kNegBig;
            for (int w = 0; w < TS; ++w) Mt = fmaxf(Mt, lastp ? s_mt[w0 + w][lh] : s_mt2[PAIR ? w : 0][lh]);
        }
        float L = 0.0f;
        float4 o = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        for (int w = 0; w < TS; ++w) {
            const float wt = __builtin_amdgcn_exp2f(wml(w).x - M);
            L += wml(w).y * wt;
            const float4 v = *reinterpret_cast<const float4*>(wacc(w) + lh * D + 4 * (ed ^ (lh & 7)));
            o.x = __builtin_fmaf(v.x, wt, o.x);
            o.y = __builtin_fmaf(v.y, wt, o.y);
            o.z = __builtin_fmaf(v.z, wt, o.z);
            o.w = __builtin_fmaf(v.w, wt, o.w);
        }
        const float inv = 1.0f / L;  // (one division; L >= 1: the partition holds a live token)
        const float4 r = make_float4(o.x * inv, o.y * inv, o.z * inv, o.w * inv);
        const size_t slot0 = ((size_t)b * H + h0) * p.max_parts + part + gp;  // head h0's slot
        const __amdgpu_buffer_rsrc_t rpo = __builtin_amdgcn_make_buffer_rsrc(
            p.part_out + slot0 * D, (short)0, NQ * p.max_parts * D * 4, 0x00020000);
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, r), rpo,
                                               (eh * p.max_parts * D + 4 * ed) * 4, 0, kScopeAgent);
        if (ed == 0) {  // (m, l) as one 8-byte agent-scope store
            const __amdgpu_buffer_rsrc_t rml = __builtin_amdgcn_make_buffer_rsrc(
                p.part_ml + slot0, (short)0, NQ * p.max_parts * 8, 0x00020000);
            const float Ls = LAZY ? L * __builtin_amdgcn_exp2f(M - Mt) : L;
            const u32x2_t ml = {__builtin_bit_cast(uint32_t, Mt * kLn2), __builtin_bit_cast(uint32_t, Ls)};
            __builtin_amdgcn_raw_buffer_store_b64(ml, rml, eh * p.max_parts * 8, 0, kScopeAgent);
        }
        if (p.out && len <= p.part_tokens)  // one partition: this is the output
            *reinterpret_cast<float4*>(p.out + ((size_t)b * H + h0 + eh) * D + 4 * ed) = r;
    }
#ifdef KVB_WG_TIMESTAMPS
    const unsigned long long ts_issued = __builtin_amdgcn_s_memrealtime();
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if (threadIdx.x == 0 && lin < kWgStampGroups) {
        unsigned long long* st = g_wg_stamps + kWgStampWords * lin;
        st[0] = ts0;
        st[1] = ts1;
        st[2] = ts_slowest;
        st[3] = ts_issued;
        st[4] = __builtin_amdgcn_s_memrealtime();
        st[5] = st[6] = 0;
        st[7] = wg_where();
    }
#endif
    if (!p.out || len <= p.part_tokens) return;

    // ---- fused merge (src/kernels.metal:123-147): the last workgroup of this (sequence, head
    // group) to arrive (the counter counts partitions: each workgroup adds the ng it wrote) weighs
    // the partitions by w_i = l_i exp(m_i - M), in paged_reduce's order
    // (the two give identical bits). Message passing without whole-cache fences: each wave waits
    // until its write-through partition stores are acknowledged (s_waitcnt vmcnt(0); __syncthreads
    // alone does not wait for stores), the barrier orders that before thread 0's count (an
    // agent-scope atomic), and the last workgroup issues its agent-scope (sc1) loads only after the
    // count came back. An agent-scope release/acquire pair would instead write back and invalidate
    // the whole L2 of the XCD in every workgroup (buffer_wbl2 / buffer_inv): 140 us per c4 step.
    __shared__ int s_last;
    const int nparts = (len + p.part_tokens - 1) / p.part_tokens;
    int* counter = p.counters + (size_t)b * gridDim.x + bx;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0)
        s_last = __hip_atomic_fetch_add(counter, ng, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == nparts - ng;
    __syncthreads();
#ifdef KVB_WG_TIMESTAMPS
    if (threadIdx.x == 0 && lin < kWgStampGroups) g_wg_stamps[kWgStampWords * lin + 5] = __builtin_amdgcn_s_memrealtime();
#endif
    if (!s_last) return;

    // The merge is on the step's critical path (it starts when the last partition ends), so its
    // latency, not its few bytes, is what costs: one round trip for everything where possible.
    // Thread e owns the 16-byte column chunk e of the group's [QG][D] output. With more than kPre
    // partitions, it issues its rows of the first kPre partitions at once, together with the
    // (m_i, l_i) of all partitions into LDS (the V tiles are free again); then w_i replaces l_i;
    // then the sums, in partition order, with the partitions past kPre in batches of kBatch.
    static_assert(sizeof(s_v) / sizeof(float2) >= fused_merge_slots(KIND, D), "merge staging size");
    constexpr int kPre = 16, kBatch = 8;
    float2* s_pml = reinterpret_cast<float2*>(&s_v[0][0]);  // [QG][nparts]
    const size_t gbase = ((size_t)b * H + h0) * p.max_parts;  // first slot of head h0
    const __amdgpu_buffer_rsrc_t rpo = __builtin_amdgcn_make_buffer_rsrc(
        p.part_out + gbase * D, (short)0, NQ * p.max_parts * D * 4, 0x00020000);
    // Chunk ec of the group's output is head ec / (D / 4), columns 4 (ec % (D / 4)) + 0..3. A thread
    // owns chunks threadIdx.x + k * 64 W: one up to QG 8, two at QG 16 (head_dim 128).
    auto row = [&](int ec, int i) {  // partition i's part of chunk ec (zeros past the group's slots)
        const int eh = ec / (D / 4), ed = ec % (D / 4);
        return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(
                                              rpo, ((eh * p.max_parts + i) * D + 4 * ed) * 4, 0, kScopeAgent));
    };
    const __amdgpu_buffer_rsrc_t rml = __builtin_amdgcn_make_buffer_rsrc(p.part_ml + gbase, (short)0,
                                                                         NQ * p.max_parts * 8, 0x00020000);
    // (m_i, l_i) of the group's head eh, one 8-byte agent-scope load. (The vector is cast whole: this
    // compiler's __builtin_bit_cast of an ext_vector element, v[1], gives the bits of v[0].)
    auto ml_at = [&](int eh, int i) {
        return __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(rml, (eh * p.max_parts + i) * 8, 0, kScopeAgent));
    };
    auto add = [](float4& o, float& L, float wt, const float4& v) {
        L += wt;
        o.x = __builtin_fmaf(wt, v.x, o.x);
        o.y = __builtin_fmaf(wt, v.y, o.y);
        o.z = __builtin_fmaf(wt, v.z, o.z);
        o.w = __builtin_fmaf(wt, v.w, o.w);
    };
    auto write_out = [&](int ec, const float4& o, float L) {  // (paged_reduce's normalisation)
        const int eh = ec / (D / 4), ed = ec % (D / 4);
        const float inv = 1.0f / L;
        *reinterpret_cast<float4*>(p.out + ((size_t)b * H + h0 + eh) * D + 4 * ed) =
            make_float4(o.x * inv, o.y * inv, o.z * inv, o.w * inv);
    };
    // Up to kPre partitions (every BASELINE configuration): each owner reads its head's (m_i, l_i)
    // straight from the workspace together with its rows, so the merge is one round trip with no
    // barrier. Same weights, same order as below. N: a bound on nparts known at compile time (8 covers
    // the BASELINE configurations and halves the code the merge walks through).
    auto merge_few = [&](auto bound) {
        constexpr int N = decltype(bound)::value;
        for (int ec = threadIdx.x; ec < NQ * D / 4; ec += 64 * W) {
            float4 pre[N];
            float2 ml[N];
            for (int j = 0; j < N; ++j)
                if (j < nparts) {
                    pre[j] = row(ec, j);
                    ml[j] = ml_at(ec / (D / 4), j);
                }
            float M = kNegBig;
            for (int j = 0; j < N; ++j)
                if (j < nparts) M = fmaxf(M, ml[j].x);
            float4 o = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            float L = 0.0f;
            for (int j = 0; j < N; ++j)
                if (j < nparts) add(o, L, partition_weight(ml[j].x, ml[j].y, M), pre[j]);
            write_out(ec, o, L);
        }
    };
    if (nparts <= kPre) {  // uniform
        if (nparts <= 8) merge_few(std::integral_constant<int, 8>{});
        else merge_few(std::integral_constant<int, kPre>{});
        if (threadIdx.x == 0) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#ifdef KVB_WG_TIMESTAMPS
        if (threadIdx.x == 0 && lin < kWgStampGroups) g_wg_stamps[kWgStampWords * lin + 6] = __builtin_amdgcn_s_memrealtime();
#endif
        return;
    }
    // More than kPre partitions: one chunk per thread (fused_merge_many; the host leaves a group with
    // more chunks than threads and more than kPre partitions to paged_reduce).
    if constexpr (fused_merge_many(KIND, QG, D)) {
        const int ec = threadIdx.x;
        const bool owner = ec < NQ * D / 4;
        float4 pre[kPre];
        for (int j = 0; j < kPre; ++j) pre[j] = row(ec, j);
        for (int x = threadIdx.x; x < NQ * nparts; x += 64 * W) s_pml[x] = ml_at(x / nparts, x % nparts);
        __syncthreads();
        for (int x = threadIdx.x; x < NQ * nparts; x += 64 * W) {
            const float2* mrow = s_pml + (x / nparts) * nparts;
            float M = kNegBig;
            for (int i = 0; i < nparts; ++i) M = fmaxf(M, mrow[i].x);
            s_pml[x].y = partition_weight(s_pml[x].x, s_pml[x].y, M);
        }
        __syncthreads();
        if (owner) {
            const float2* wrow = s_pml + (ec / (D / 4)) * nparts;
            float4 o = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            float L = 0.0f;
            for (int j = 0; j < kPre; ++j) add(o, L, wrow[j].y, pre[j]);
            for (int i0 = kPre; i0 < nparts; i0 += kBatch) {
                float4 v[kBatch];
                for (int j = 0; j < kBatch; ++j) v[j] = row(ec, i0 + j);
                for (int j = 0; j < kBatch; ++j)
                    if (i0 + j < nparts) add(o, L, wrow[i0 + j].y, v[j]);
            }
            write_out(ec, o, L);
        }
    }
    if (threadIdx.x == 0) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#ifdef KVB_WG_TIMESTAMPS
    if (threadIdx.x == 0 && lin < kWgStampGroups) g_wg_stamps[kWgStampWords * lin + 6] = __builtin_amdgcn_s_memrealtime();
#endif
}

// Dynamic LDS for the loads-only variant so that a CU holds as many of its workgroups as of the
// decode kernel's: the variant needs fewer registers and would otherwise run more workgroups per CU
// whenever the grid has more than one per CU. The largest size at which the occupancy calculator
// gives the variant the decode's count (at most what one workgroup may allocate); computed once per
// instantiation.
template <int KIND, int D, int QG, bool PAIR, bool PART, bool SHARE>
hipError_t loads_only_lds(size_t* lds) {
    static size_t cached = SIZE_MAX;
    if (cached == SIZE_MAX) {
        const auto loads = paged_decode_kernel<KIND, D, QG, true, true, PAIR, PART, SHARE>;
        const int threads = 64 * decode_wg_waves(KIND, QG);
        int occ = 0, dev = 0, lds_cu = 0, lds_wg = 0;
        hipFuncAttributes fa{};
        hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &occ, paged_decode_kernel<KIND, D, QG, true, false, PAIR, PART, SHARE>, threads, 0);
        if (e == hipSuccess) e = hipGetDevice(&dev);
        if (e == hipSuccess) e = hipDeviceGetAttribute(&lds_cu, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor, dev);
        if (e == hipSuccess) e = hipDeviceGetAttribute(&lds_wg, hipDeviceAttributeMaxSharedMemoryPerBlock, dev);
        if (e == hipSuccess) e = hipFuncGetAttributes(&fa, reinterpret_cast<const void*>(loads));
        if (e != hipSuccess) return e;
        size_t dyn = 0;
        if (occ > 0) {
            size_t per_group = std::min<size_t>((size_t)lds_cu / occ, (size_t)lds_wg) & ~size_t(255);
            for (; per_group > fa.sharedSizeBytes; per_group -= 256) {
                int got = 0;
                e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&got, loads, threads, per_group - fa.sharedSizeBytes);
                if (e != hipSuccess) return e;
                if (got >= occ) {
                    dyn = per_group - fa.sharedSizeBytes;
                    break;
                }
            }
        }
        cached = dyn;
    }
    *lds = cached;
    return hipSuccess;
}

template <int KIND, int D, int QG, bool FAST, bool PAIR, bool PART, bool SHARE, bool STAGE = false>
hipError_t launch_one(const DecodeParams& p, int batch, hipStream_t s, const Marks& m) {
    if (m.describe) {  // the demangled name of the instantiation below, as rocprofv3 prints it
        auto tf = [](bool x) { return x ? "true" : "false"; };
        const bool loads = FAST && p.loads_only;
        std::snprintf(m.describe, m.describe_cap,
                      "void kvbk::paged_decode_kernel<%d, %d, %d, %s, %s, %s, %s, %s, %s>(kvbk::DecodeParams)", KIND, D,
                      QG, tf(FAST), tf(loads), tf(PAIR), tf(PART), tf(SHARE), tf(!loads && STAGE));
        return hipSuccess;
    }
    const int gz = PAIR ? (p.max_parts + 1) / 2 : p.max_parts;
    const dim3 grid(p.num_heads / p.qg, p.ragged_items ? p.ragged_items : batch, p.ragged_items ? 1 : gz);
    if (p.loads_only) {  // tile-aligned pages only
        if constexpr (!FAST) {
            return hipErrorInvalidValue;
        } else {
            size_t lds = 0;
            if (const hipError_t e = loads_only_lds<KIND, D, QG, PAIR, PART, SHARE>(&lds); e != hipSuccess) return e;
            launch_marked_lds(paged_decode_kernel<KIND, D, QG, true, true, PAIR, PART, SHARE>, grid, dim3(64 * decode_wg_waves(KIND, QG)),
                              lds, s, m, p);
        }
    } else {
        launch_marked(paged_decode_kernel<KIND, D, QG, FAST, false, PAIR, PART, SHARE, STAGE>, grid, dim3(64 * decode_wg_waves(KIND, QG)), s, m, p);
    }
    return hipGetLastError();
}

// Two partitions per workgroup (DecodeParams::pair): tile-aligned f16 and i8 caches, plain grid only.
template <int KIND, int D, int QG, bool PART, bool SHARE = false>
hipError_t launch_qg(bool fast, const DecodeParams& p, int batch, hipStream_t s, const Marks& m) {
    if (!fast) {
        if (p.pair) return hipErrorInvalidValue;
        return p.table_in_lds ? launch_one<KIND, D, QG, false, false, PART, SHARE, true>(p, batch, s, m)
                              : launch_one<KIND, D, QG, false, false, PART, SHARE>(p, batch, s, m);
    }
    if constexpr (KIND != KV_F32 && decode_shape(KIND, QG).hs == 1) {
        if (p.pair) return p.ragged_items ? hipErrorInvalidValue : launch_one<KIND, D, QG, true, true, PART, SHARE>(p, batch, s, m);
    } else {
        if (p.pair) return hipErrorInvalidValue;
    }
    return launch_one<KIND, D, QG, true, false, PART, SHARE>(p, batch, s, m);
}

template <int KIND, int D>
hipError_t launch_for_dim(int qg, bool fast, const DecodeParams& p, int batch, hipStream_t s, const Marks& m) {
    const bool sib = p.group > qg;  // more than one workgroup per KV head
    switch (qg) {
        // SHARE builds where a KV head has more than one workgroup and one workgroup serves 3 or 5-8
        // heads (groups 9, 10, 12, 14, 16, 24, 32, ...); groups whose workgroups serve 1, 2 or 4
        // heads each (11, 13, 22, 44, ...) keep the plain order and non-temporal loads.
        case 1: return launch_qg<KIND, D, 1, false>(fast, p, batch, s, m);
        case 2: return launch_qg<KIND, D, 2, false>(fast, p, batch, s, m);
        case 3: return sib ? launch_qg<KIND, D, 4, true, true>(fast, p, batch, s, m)
                           : launch_qg<KIND, D, 4, true>(fast, p, batch, s, m);
        case 4: return launch_qg<KIND, D, 4, false>(fast, p, batch, s, m);
        case 5:
        case 6:
        case 7: return sib ? launch_qg<KIND, D, 8, true, true>(fast, p, batch, s, m)
                           : launch_qg<KIND, D, 8, true>(fast, p, batch, s, m);
        case 8: return sib ? launch_qg<KIND, D, 8, false, true>(fast, p, batch, s, m)
                           : launch_qg<KIND, D, 8, false>(fast, p, batch, s, m);
        case 16:
            if constexpr (KIND != KV_F32)
                return sib ? launch_qg<KIND, D, 16, false, true>(fast, p, batch, s, m)
                           : launch_qg<KIND, D, 16, false>(fast, p, batch, s, m);
            return hipErrorInvalidValue;
        case 32:
            if constexpr (KIND != KV_F32)
                return sib ? launch_qg<KIND, D, 32, false, true>(fast, p, batch, s, m)
                           : launch_qg<KIND, D, 32, false>(fast, p, batch, s, m);
            return hipErrorInvalidValue;
        default: return hipErrorInvalidValue;
    }
}

template <int KIND>
hipError_t launch_for_kind(int head_dim, int qg, bool fast, const DecodeParams& p, int batch, hipStream_t s,
                           const Marks& m) {
    if (head_dim == 64) return launch_for_dim<KIND, 64>(qg, fast, p, batch, s, m);
    if (head_dim == 128) return launch_for_dim<KIND, 128>(qg, fast, p, batch, s, m);
    return hipErrorInvalidValue;
}

}  // namespace kvbk
