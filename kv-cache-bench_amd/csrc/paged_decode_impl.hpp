// paged_decode for gfx950: split-K decode attention over a paged KV cache.
//
// Semantics follow the reference's paged_decode (src/kernels.metal:35-121): a workgroup owns one
// partition of part_tokens tokens of one sequence and QG query heads of one KV head, and writes the
// partition's normalised output o / l plus (m, l) to slot (b*H + h)*max_parts + part of the
// split-K workspace. The mapping onto CDNA4 is this build's own:
//
//  * Each wave64 walks 16-token tiles of the partition (wave w takes tiles w, w+4, ...) and keeps
//    its own online-softmax state (m, l, acc) for the QG heads; the workgroup merges the four
//    wave states at the end, as the reference merges its simdgroups.
//  * Scores S = Q K^T of a tile come from MFMA: one 16x16 tile with the 16 tokens as columns and
//    the QG heads as rows. fp16/int8 caches use v_mfma_f32_16x16x32_f16 with q split into a high
//    and a low fp16 part (rows 2h and 2h+1), so the product keeps ~22 bits of q and the fp32
//    accumulation of the MFMA: K is read as stored, q is never rounded to fp16 as a whole. fp32
//    caches use v_mfma_f32_16x16x4_f32 on q and K as they are (rows 2h+1 are zero).
//  * K is loaded straight into the MFMA B-operand layout: lane l reads 16 bytes of token l%16,
//    lanes l, l+16, l+32, l+48 cover 64 contiguous bytes of that row per instruction. The
//    contraction order over d is free, so each storage type picks the d order its loads give and
//    q is laid out to match (dslot_*).
//  * The tile max is a 16-lane DPP row reduction; p = exp2(s - m) with q pre-scaled by
//    scale*log2(e); p and the rescale factors go through LDS to the lanes that hold V.
//  * V is read row-major (16 lanes x 16 bytes per fp16 row) and P*V runs on the VALU in fp32
//    (a decode step has one query per head, so P*V is QG dot products per V element).
//  * int8: bytes become exact fp16 (x ^ 0x80 under a 0x64 exponent, minus 1152) for the MFMA; the
//    per-(block, KV head) K scale multiplies the score and the V scale multiplies p before P*V.
//  * Tokens past the partition end get weight 0 and never reach the arithmetic as data. With
//    `FAST` (every tile inside one page) the block id and scales are one scalar read per tile and
//    K/V come through a buffer resource sized to the tile's live rows, so rows past the end read as
//    zeros without touching memory; otherwise every lane looks up its own token's block (any page
//    size) and lanes past the end re-read the partition's first token and zero it.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include "kvb_kernels.hpp"

namespace kvbk {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float floatx4_t __attribute__((ext_vector_type(4)));

constexpr float kNegBig = -1e30f;  // "minus infinity" that keeps exp2(kNegBig - m) == 0 and no inf - inf
constexpr float kLn2 = 0.693147180559945309f;

// ---- cross-lane helpers -------------------------------------------------------------------------

template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}
constexpr int kQuadSwap1 = 0xB1;     // quad_perm [1,0,3,2]
constexpr int kQuadSwap2 = 0x4E;     // quad_perm [2,3,0,1]
constexpr int kRowHalfMirror = 0x141;
constexpr int kRowMirror = 0x140;

// Max / sum over the 16 lanes of a DPP row; every lane of the row gets the result.
__device__ __forceinline__ float row_max16(float x) {
    x = fmaxf(x, dpp<kQuadSwap1>(x));
    x = fmaxf(x, dpp<kQuadSwap2>(x));
    x = fmaxf(x, dpp<kRowHalfMirror>(x));
    x = fmaxf(x, dpp<kRowMirror>(x));
    return x;
}
__device__ __forceinline__ float row_sum16(float x) {
    x += dpp<kQuadSwap1>(x);
    x += dpp<kQuadSwap2>(x);
    x += dpp<kRowHalfMirror>(x);
    x += dpp<kRowMirror>(x);
    return x;
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

// ---- per storage type: load widths and the d order of the MFMA contraction -------------------

template <int KIND, int D>
struct KvT;

template <int D>
struct KvT<KV_F16, D> {
    static constexpr int ESZ = 2;
    static constexpr int KLOADS = D / 32;  // 16-byte loads per lane per tile for K
    static constexpr int NJ = D / 32;      // 16x16x32 f16 MFMAs per tile
    static constexpr int VDW = 4;          // dwords per lane per V row (8 elements)
    // d of K byte-load c for row quad q4, and d of MFMA j slot s
    __device__ static int kdoff(int c, int q4) { return 32 * c + 8 * q4; }
    __device__ static int dslot(int j, int q4, int s) { return 32 * j + 8 * q4 + s; }
};
template <int D>
struct KvT<KV_I8, D> {
    static constexpr int ESZ = 1;
    static constexpr int KLOADS = D / 64;
    static constexpr int NJ = D / 32;
    static constexpr int VDW = 2;
    __device__ static int kdoff(int c, int q4) { return 64 * c + 16 * q4; }
    __device__ static int dslot(int j, int q4, int s) { return 64 * (j >> 1) + 16 * q4 + 8 * (j & 1) + s; }
};
template <int D>
struct KvT<KV_F32, D> {
    static constexpr int ESZ = 4;
    static constexpr int KLOADS = D / 16;
    static constexpr int NJ = D / 4;       // 16x16x4 f32 MFMAs per tile
    static constexpr int VDW = 8;
    __device__ static int kdoff(int c, int q4) { return 16 * c + 4 * q4; }
    __device__ static int dslot(int j, int q4, int /*s*/) { return 16 * (j >> 2) + 4 * q4 + (j & 3); }
};

// Raw registers of one tile.
template <int KIND, int D>
struct TileRegs {
    using T = KvT<KIND, D>;
    static constexpr int LPR = D / 8, RPL = 64 / LPR, NV = kTile / RPL;
    uint4 k[T::KLOADS];
    uint32_t v[NV][T::VDW];
    float kscale, vscale;  // int8: scales of this lane's K-layout token (p folds in the V scale)
};

// ---- the kernel ---------------------------------------------------------------------------------

template <int KIND, int D, int QG, bool FAST>
__global__ __launch_bounds__(64 * kDecodeWaves) void paged_decode_kernel(DecodeParams p) {
    using T = KvT<KIND, D>;
    using R = TileRegs<KIND, D>;
    constexpr int W = kDecodeWaves;
    constexpr int LPR = R::LPR, RPL = R::RPL, NV = R::NV, NJ = T::NJ;
    static_assert(QG == 1 || QG == 2 || QG == 4 || QG == 8, "QG must be 1, 2, 4 or 8");

    __shared__ float s_p[W][kTile][QG];   // p of the current tile, [token][head]
    __shared__ float s_corr[W][QG];       // rescale factor of the current tile
    __shared__ float s_acc[W][QG][D];     // final per-wave accumulators
    __shared__ float2 s_ml[W][QG];        // final per-wave (m, l)

    const int part = blockIdx.x, b = blockIdx.z;
    const int h0 = blockIdx.y * QG;
    const int len = p.seq_lens[b];
    const int t0 = part * p.part_tokens;
    if (t0 >= len) return;  // uniform over the workgroup, before any barrier
    const int t1 = min(len, t0 + p.part_tokens);
    const int H = p.num_heads, Hkv = p.num_kv_heads, P = p.page_size;
    const int kvh = h0 / p.group;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n = lane & 15, q4 = lane >> 4;              // MFMA: token column / stack row, row quad
    const int vr = lane / LPR, vc = lane % LPR;            // V: row within a load, 8-element chunk
    const int32_t* bt = p.block_table + (size_t)b * p.max_blocks;
    const char* kbase = static_cast<const char*>(p.k);
    const char* vbase = static_cast<const char*>(p.v);

    // ---- q as MFMA A operand: stack row m = lane % 16 holds head m/2, high (m even) or low part.
    const int hh = n >> 1, hl = n & 1;
    const bool qrow = hh < QG;
    const float* qp = p.q + ((size_t)b * H + h0 + (qrow ? hh : 0)) * D;
    float up = 1.0f;  // scores are MFMA results times `up` (a power of two)
    half8_t aq16[KIND == KV_F32 ? 1 : NJ];
    float aq32[KIND == KV_F32 ? NJ : 1];
    if constexpr (KIND == KV_F32) {
        for (int j = 0; j < NJ; ++j) aq32[j] = (qrow && hl == 0) ? qp[T::dslot(j, q4, 0)] * p.qscale : 0.0f;
    } else {
        float qv[NJ][8];
        float amax = 0.0f;
        for (int j = 0; j < NJ; ++j)
            for (int s = 0; s < 8; ++s) {
                qv[j][s] = qrow ? qp[T::dslot(j, q4, s)] * p.qscale : 0.0f;
                amax = fmaxf(amax, fabsf(qv[j][s]));
            }
        amax = wave_max(amax);
        int e = 0;
        if (amax > 0.0f) {
            frexpf(amax, &e);  // amax < 2^e
            e -= 14;           // the scaled q stays below 2^14, far from fp16 overflow
        }
        const float down = ldexpf(1.0f, -e);
        up = ldexpf(1.0f, e);
        for (int j = 0; j < NJ; ++j)
            for (int s = 0; s < 8; ++s) {
                const float x = qv[j][s] * down;
                const _Float16 hi = (_Float16)x;
                const _Float16 lo = (_Float16)(x - (float)hi);
                aq16[j][s] = hl ? lo : hi;
            }
    }

    // ---- tile loads (no branches around them, so the compiler can keep a tile in flight)
    auto load_v_row = [&](uint32_t* dst, auto&& load16, auto&& load8, int off) {
        if constexpr (T::VDW == 8) {
            const uint4 a = load16(off), c = load16(off + 16);
            dst[0] = a.x; dst[1] = a.y; dst[2] = a.z; dst[3] = a.w;
            dst[4] = c.x; dst[5] = c.y; dst[6] = c.z; dst[7] = c.w;
        } else if constexpr (T::VDW == 4) {
            const uint4 a = load16(off);
            dst[0] = a.x; dst[1] = a.y; dst[2] = a.z; dst[3] = a.w;
        } else {
            const uint2 a = load8(off);
            dst[0] = a.x; dst[1] = a.y;
        }
    };
    auto load_tile = [&](R& r, int tt) {
        if constexpr (FAST) {
            // The tile [tt, tt+16) lies in one page: one block id, and a buffer resource that
            // covers exactly the tile's live rows, so rows at or past t1 read as zeros.
            // A tile at or past t1 (the prefetch after the last one) gets an empty range.
            const int tc = min(tt, t1 - 1);
            const int blk = bt[tc / P];
            const size_t row0 = ((size_t)blk * Hkv + kvh) * P + (tc % P);
            // (readfirstlane: the value is wave-uniform, and a descriptor must live in SGPRs)
            const int nbytes = __builtin_amdgcn_readfirstlane(max(0, min(kTile, t1 - tt)) * D * T::ESZ);
            const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<char*>(kbase + row0 * D * T::ESZ), (short)0, nbytes, 0x00020000);
            const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<char*>(vbase + row0 * D * T::ESZ), (short)0, nbytes, 0x00020000);
            for (int c = 0; c < T::KLOADS; ++c)
                r.k[c] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                                                       rk, (n * D + T::kdoff(c, q4)) * T::ESZ, 0, 0));
            auto v16 = [&](int off) { return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rv, off, 0, 0)); };
            auto v8 = [&](int off) { return __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rv, off, 0, 0)); };
            for (int i = 0; i < NV; ++i) load_v_row(r.v[i], v16, v8, ((i * RPL + vr) * D + 8 * vc) * T::ESZ);
            if constexpr (KIND == KV_I8) {
                r.kscale = p.k_scale[(size_t)blk * Hkv + kvh];
                r.vscale = p.v_scale[(size_t)blk * Hkv + kvh];
            }
        } else {
            // Any page size: each lane finds the block of its own token. Lanes past t1 read the
            // partition's first token (always live) and zero what they got.
            const int tk = tt + n;
            const bool kval = tk < t1;
            const int tks = kval ? tk : t0;
            const int kblk = bt[tks / P];
            const size_t krow = ((size_t)kblk * Hkv + kvh) * P + (tks % P);
            const char* kb = kbase + krow * D * T::ESZ;
            for (int c = 0; c < T::KLOADS; ++c) {
                const uint4 x = *reinterpret_cast<const uint4*>(kb + T::kdoff(c, q4) * T::ESZ);
                r.k[c] = kval ? x : make_uint4(0, 0, 0, 0);
            }
            if constexpr (KIND == KV_I8) {
                r.kscale = p.k_scale[(size_t)kblk * Hkv + kvh];
                r.vscale = p.v_scale[(size_t)kblk * Hkv + kvh];
            }
            for (int i = 0; i < NV; ++i) {
                const int tv = tt + i * RPL + vr;
                const bool vval = tv < t1;
                const int tvs = vval ? tv : t0;
                const size_t vrow = ((size_t)bt[tvs / P] * Hkv + kvh) * P + (tvs % P);
                const char* src = vbase + vrow * D * T::ESZ;
                auto v16 = [&](int off) {
                    const uint4 x = *reinterpret_cast<const uint4*>(src + off);
                    return vval ? x : make_uint4(0, 0, 0, 0);
                };
                auto v8 = [&](int off) {
                    const uint2 x = *reinterpret_cast<const uint2*>(src + off);
                    return vval ? x : make_uint2(0, 0);
                };
                load_v_row(r.v[i], v16, v8, 8 * vc * T::ESZ);
            }
        }
    };

    // ---- per-wave online-softmax state
    // Lanes of row quad q4 own heads 2*q4 (a) and 2*q4+1 (b); m is uniform over the 16 lanes,
    // l is a per-lane partial sum over that lane's tokens.
    const int ha = 2 * q4, hb = 2 * q4 + 1;
    float ma = kNegBig, mb = kNegBig, la = 0.0f, lb = 0.0f;
    float acc[QG][8];
    for (int h = 0; h < QG; ++h)
        for (int e = 0; e < 8; ++e) acc[h][e] = 0.0f;

    auto compute_tile = [&](const R& r, int tt) {
        // S = Q K^T for the 16 tokens of the tile
        floatx4_t S = {0.0f, 0.0f, 0.0f, 0.0f};
        if constexpr (KIND == KV_F32) {
            for (int j = 0; j < NJ; ++j) {
                const uint4 w4 = r.k[j >> 2];
                const uint32_t w = (j & 3) == 0 ? w4.x : (j & 3) == 1 ? w4.y : (j & 3) == 2 ? w4.z : w4.w;
                S = __builtin_amdgcn_mfma_f32_16x16x4f32(aq32[j], __builtin_bit_cast(float, w), S, 0, 0, 0);
            }
        } else if constexpr (KIND == KV_F16) {
            for (int j = 0; j < NJ; ++j)
                S = __builtin_amdgcn_mfma_f32_16x16x32_f16(aq16[j], __builtin_bit_cast(half8_t, r.k[j]), S, 0, 0, 0);
        } else {
            for (int j = 0; j < NJ; ++j) {
                const uint4 w4 = r.k[j >> 1];
                const half8_t kb = (j & 1) ? i8x8_to_half8(w4.z, w4.w) : i8x8_to_half8(w4.x, w4.y);
                S = __builtin_amdgcn_mfma_f32_16x16x32_f16(aq16[j], kb, S, 0, 0, 0);
            }
        }
        float f = up;
        if constexpr (KIND == KV_I8) f *= r.kscale;
        const bool valid = tt + n < t1;
        const float sa = valid ? (S[0] + S[1]) * f : kNegBig;
        const float sb = valid ? (S[2] + S[3]) * f : kNegBig;
        const float mna = fmaxf(ma, row_max16(sa));
        const float mnb = fmaxf(mb, row_max16(sb));
        const float ca = __builtin_amdgcn_exp2f(ma - mna);
        const float cb = __builtin_amdgcn_exp2f(mb - mnb);
        const float pa = valid ? __builtin_amdgcn_exp2f(sa - mna) : 0.0f;
        const float pb = valid ? __builtin_amdgcn_exp2f(sb - mnb) : 0.0f;
        la = la * ca + pa;
        lb = lb * cb + pb;
        ma = mna;
        mb = mnb;
        float pv_scale = 1.0f;
        if constexpr (KIND == KV_I8) pv_scale = r.vscale;
        if (ha < QG) {
            s_p[wave][n][ha] = pa * pv_scale;
            if (n == 0) s_corr[wave][ha] = ca;
        }
        if (hb < QG) {
            s_p[wave][n][hb] = pb * pv_scale;
            if (n == 0) s_corr[wave][hb] = cb;
        }
        // LDS ops of one wave execute in order; the fence keeps the compiler from moving the
        // reads above the writes.
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

        float corr[QG];
        for (int h = 0; h < QG; ++h) corr[h] = s_corr[wave][h];
        for (int h = 0; h < QG; ++h)
            for (int e = 0; e < 8; ++e) acc[h][e] *= corr[h];
        for (int i = 0; i < NV; ++i) {
            float pr[QG];
            for (int h = 0; h < QG; ++h) pr[h] = s_p[wave][i * RPL + vr][h];
            float x[8];
            if constexpr (KIND == KV_F32) {
                for (int e = 0; e < 8; ++e) x[e] = __builtin_bit_cast(float, r.v[i][e]);
            } else if constexpr (KIND == KV_F16) {
                for (int e = 0; e < 4; ++e) {
                    const half2_t h2 = __builtin_bit_cast(half2_t, r.v[i][e]);
                    x[2 * e] = (float)h2[0];
                    x[2 * e + 1] = (float)h2[1];
                }
            } else {
                for (int e = 0; e < 8; ++e) x[e] = (float)(int8_t)(r.v[i][e >> 2] >> (8 * (e & 3)));
            }
            for (int h = 0; h < QG; ++h)
                for (int e = 0; e < 8; ++e) acc[h][e] = __builtin_fmaf(pr[h], x[e], acc[h][e]);
        }
    };

    // ---- walk the tiles: two register sets, the next tile's loads in flight while one computes.
    // The prefetch is unconditional (past the end it reads zeros) so no branch splits the load
    // counters the compiler tracks.
    const int ntiles = (t1 - t0 + kTile - 1) / kTile;
    R ra, rb;
    int it = wave;
    load_tile(ra, t0 + it * kTile);
    while (it < ntiles) {
        load_tile(rb, t0 + (it + W) * kTile);
        compute_tile(ra, t0 + it * kTile);
        it += W;
        if (it >= ntiles) break;
        load_tile(ra, t0 + (it + W) * kTile);
        compute_tile(rb, t0 + it * kTile);
        it += W;
    }

    // ---- merge: lanes -> wave state -> workgroup
    la = row_sum16(la);
    lb = row_sum16(lb);
    for (int h = 0; h < QG; ++h)
        for (int e = 0; e < 8; ++e)
            for (int off = LPR; off < 64; off <<= 1) acc[h][e] += __shfl_xor(acc[h][e], off);
    if (n == 0) {
        if (ha < QG) s_ml[wave][ha] = make_float2(ma, la);
        if (hb < QG) s_ml[wave][hb] = make_float2(mb, lb);
    }
    if (vr == 0)
        for (int h = 0; h < QG; ++h)
            for (int e = 0; e < 8; ++e) s_acc[wave][h][8 * vc + e] = acc[h][e];
    __syncthreads();

    for (int idx = threadIdx.x; idx < QG * D; idx += 64 * W) {
        const int h = idx / D, d = idx % D;
        float M = kNegBig;
        for (int w = 0; w < W; ++w) M = fmaxf(M, s_ml[w][h].x);
        float L = 0.0f, o = 0.0f;
        for (int w = 0; w < W; ++w) {
            const float wt = __builtin_amdgcn_exp2f(s_ml[w][h].x - M);
            L += s_ml[w][h].y * wt;
            o += s_acc[w][h][d] * wt;
        }
        const size_t slot = ((size_t)b * H + h0 + h) * p.max_parts + part;
        p.part_out[slot * D + d] = o / L;
        if (d == 0) p.part_ml[slot] = make_float2(M * kLn2, L);
    }
}

template <int KIND, int D, int QG, bool FAST>
hipError_t launch_one(const DecodeParams& p, int batch, hipStream_t s) {
    const dim3 grid(p.max_parts, p.num_heads / QG, batch);
    hipLaunchKernelGGL((paged_decode_kernel<KIND, D, QG, FAST>), grid, dim3(64 * kDecodeWaves), 0, s, p);
    return hipGetLastError();
}

template <int KIND, int D>
hipError_t launch_for_dim(int qg, bool fast, const DecodeParams& p, int batch, hipStream_t s) {
    switch (qg) {
        case 1: return fast ? launch_one<KIND, D, 1, true>(p, batch, s) : launch_one<KIND, D, 1, false>(p, batch, s);
        case 2: return fast ? launch_one<KIND, D, 2, true>(p, batch, s) : launch_one<KIND, D, 2, false>(p, batch, s);
        case 4: return fast ? launch_one<KIND, D, 4, true>(p, batch, s) : launch_one<KIND, D, 4, false>(p, batch, s);
        case 8: return fast ? launch_one<KIND, D, 8, true>(p, batch, s) : launch_one<KIND, D, 8, false>(p, batch, s);
        default: return hipErrorInvalidValue;
    }
}

template <int KIND>
hipError_t launch_for_kind(int head_dim, int qg, bool fast, const DecodeParams& p, int batch, hipStream_t s) {
    if (head_dim == 64) return launch_for_dim<KIND, 64>(qg, fast, p, batch, s);
    if (head_dim == 128) return launch_for_dim<KIND, 128>(qg, fast, p, batch, s);
    return hipErrorInvalidValue;
}

}  // namespace kvbk
