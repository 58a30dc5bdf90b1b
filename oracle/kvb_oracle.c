/*
 * kvb_oracle.c -- TEST INFRASTRUCTURE ONLY: plain-C restatement of the reference's CPU path
 * (chipontix/kv-cache-bench src/reference.cpp, src/reference.hpp, src/metal_attn.hpp:43-51,
 * tests/gpu_tests.cpp:13-62). Used by tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg as the checker; never by the product. See kvb_oracle.h for how each
 * function is pinned.
 */
#include "kvb_oracle.h"

#include <float.h>
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ---- f16 ---------------------------------------------------------------------------------- */

float kvbo_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    uint32_t bits;
    if (exp == 0x1f) {
        bits = sign | 0x7f800000u | (man << 13); /* inf / nan */
    } else if (exp != 0) {
        bits = sign | ((exp + 112u) << 23) | (man << 13);
    } else if (man == 0) {
        bits = sign;
    } else { /* subnormal: value = man * 2^-24 */
        int e = -1;
        do {
            man <<= 1;
            ++e;
        } while (!(man & 0x400u));
        man &= 0x3ffu;
        bits = sign | ((uint32_t)(112 - e) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

uint16_t kvbo_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    const uint32_t absx = x & 0x7fffffffu;
    if (absx >= 0x7f800000u) /* inf or nan: keep a quiet nan payload bit */
        return (uint16_t)(sign | 0x7c00u | (absx > 0x7f800000u ? 0x200u | ((absx >> 13) & 0x3ffu) : 0u));
    if (absx >= 0x477ff000u) /* rounds to >= 65520: overflow to inf */
        return (uint16_t)(sign | 0x7c00u);
    if (absx >= 0x38800000u) { /* normal f16 range, |f| >= 2^-14 */
        const uint32_t mant = absx & 0x7fffffu;
        uint32_t h = ((absx >> 23) - 112u) << 10 | (mant >> 13);
        const uint32_t rest = mant & 0x1fffu;
        if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) ++h; /* carries into the exponent correctly */
        return (uint16_t)(sign | h);
    }
    if (absx < 0x33000000u) /* |f| < 2^-25: rounds to zero (2^-25 itself is a tie to even 0) */
        return sign;
    /* subnormal f16: value = round(|f| / 2^-24) */
    const uint32_t e = absx >> 23;               /* 102..112 */
    const uint32_t mant = (absx & 0x7fffffu) | 0x800000u;
    const uint32_t shift = 126u - e;             /* 14..24: mant * 2^(e-150) / 2^-24 = mant >> (126-e) */
    uint32_t h = mant >> shift;
    const uint32_t rest = mant & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1u);
    if (rest > half || (rest == half && (h & 1u))) ++h;
    return (uint16_t)(sign | h);
}

double kvbo_max_abs_diff(const float* a, const float* b, size_t n) {
    double m = 0;
    for (size_t i = 0; i < n; ++i) {
        const double e = fabs((double)a[i] - (double)b[i]);
        if (isnan(e)) return INFINITY;
        if (e > m) m = e;
    }
    return m;
}

/* ---- mt19937_64 --------------------------------------------------------------------------- */

void kvbo_mt64_seed(kvbo_mt64* g, uint64_t seed) {
    g->mt[0] = seed;
    for (int i = 1; i < 312; ++i)
        g->mt[i] = 6364136223846793005ull * (g->mt[i - 1] ^ (g->mt[i - 1] >> 62)) + (uint64_t)i;
    g->idx = 312;
}

uint64_t kvbo_mt64_next(kvbo_mt64* g) {
    if (g->idx >= 312) {
        const uint64_t upper = 0xFFFFFFFF80000000ull, lower = 0x7FFFFFFFull;
        for (int i = 0; i < 312; ++i) {
            const uint64_t y = (g->mt[i] & upper) | (g->mt[(i + 1) % 312] & lower);
            g->mt[i] = g->mt[(i + 156) % 312] ^ (y >> 1) ^ ((y & 1u) ? 0xB5026F5AA96619E9ull : 0ull);
        }
        g->idx = 0;
    }
    uint64_t x = g->mt[g->idx++];
    x ^= (x >> 29) & 0x5555555555555555ull;
    x ^= (x << 17) & 0x71D67FFFEDA60000ull;
    x ^= (x << 37) & 0xFFF7EEE000000000ull;
    x ^= x >> 43;
    return x;
}

uint64_t kvbo_mt64_below(kvbo_mt64* g, uint64_t n) {
    return (uint64_t)(((unsigned __int128)kvbo_mt64_next(g) * n) >> 64);
}

/* ---- layouts -------------------------------------------------------------------------------- */

size_t kvbo_contig_index(const kvbo_shape* s, int max_len, int b, int kvh, int t, int d) {
    return (((size_t)b * s->num_kv_heads + kvh) * (size_t)max_len + t) * s->head_dim + d;
}

size_t kvbo_paged_index(const kvbo_shape* s, int page_size, int max_blocks, const int32_t* table, int b,
                        int kvh, int t, int d) {
    const size_t blk = (size_t)table[(size_t)b * max_blocks + t / page_size];
    return ((blk * s->num_kv_heads + kvh) * page_size + t % page_size) * s->head_dim + d;
}

int kvbo_layout_dims(const int* lens, int batch, int page_size, double pool_factor, int* max_blocks,
                     int* live_blocks, int* pool_blocks) {
    if (page_size <= 0 || batch < 0 || !(pool_factor >= 1.0)) return -1;
    long long mx = 0, live = 0;
    for (int b = 0; b < batch; ++b) {
        if (lens[b] < 0) return -1;
        const long long blocks = ((long long)lens[b] + page_size - 1) / page_size;
        if (blocks > mx) mx = blocks;
        live += blocks;
    }
    const long long pool = (long long)ceil((double)live * pool_factor);
    if (pool > 0x7fffffffLL) return -1;
    *max_blocks = (int)mx;
    *live_blocks = (int)live;
    *pool_blocks = (int)(pool < live ? live : pool);
    return 0;
}

int kvbo_make_paged_layout(const int* lens, int batch, int page_size, double pool_factor, uint64_t seed,
                           int32_t* table) {
    int max_blocks, live, pool;
    if (kvbo_layout_dims(lens, batch, page_size, pool_factor, &max_blocks, &live, &pool)) return -1;
    int32_t* phys = (int32_t*)malloc(sizeof(int32_t) * (size_t)(pool ? pool : 1));
    if (!phys) return -1;
    for (int i = 0; i < pool; ++i) phys[i] = i;
    kvbo_mt64 g;
    kvbo_mt64_seed(&g, seed);
    for (int i = pool - 1; i > 0; --i) {
        const int j = (int)kvbo_mt64_below(&g, (uint64_t)i + 1);
        const int32_t tmp = phys[i];
        phys[i] = phys[j];
        phys[j] = tmp;
    }
    for (size_t i = 0; i < (size_t)batch * max_blocks; ++i) table[i] = -1;
    int next = 0;
    for (int b = 0; b < batch; ++b) {
        const int blocks = (lens[b] + page_size - 1) / page_size;
        for (int i = 0; i < blocks; ++i) table[(size_t)b * max_blocks + i] = phys[next++];
    }
    free(phys);
    return 0;
}

void kvbo_scatter_to_paged(const kvbo_shape* s, int page_size, int max_blocks, const int32_t* table,
                           const int* lens, int max_len, size_t elem_size, const void* contig, void* paged) {
    const unsigned char* src = (const unsigned char*)contig;
    unsigned char* dst = (unsigned char*)paged;
    for (int b = 0; b < s->batch; ++b)
        for (int kvh = 0; kvh < s->num_kv_heads; ++kvh)
            for (int t = 0; t < lens[b]; ++t)
                for (int d = 0; d < s->head_dim; ++d)
                    memcpy(dst + elem_size * kvbo_paged_index(s, page_size, max_blocks, table, b, kvh, t, d),
                           src + elem_size * kvbo_contig_index(s, max_len, b, kvh, t, d), elem_size);
}

void kvbo_quantize_to_paged_i8(const kvbo_shape* s, int page_size, int max_blocks, const int32_t* table,
                               const int* lens, int max_len, const float* contig, int8_t* paged,
                               float* scales) {
    const int P = page_size, D = s->head_dim;
    for (int b = 0; b < s->batch; ++b)
        for (int i = 0; i * P < lens[b]; ++i)
            for (int kvh = 0; kvh < s->num_kv_heads; ++kvh) {
                const int t0 = i * P, t1 = lens[b] < t0 + P ? lens[b] : t0 + P;
                float amax = 0.0f;
                for (int t = t0; t < t1; ++t)
                    for (int d = 0; d < D; ++d) {
                        const float a = fabsf(contig[kvbo_contig_index(s, max_len, b, kvh, t, d)]);
                        if (a > amax) amax = a; /* std::max(amax, a): keeps amax when a is NaN */
                    }
                const float scale = amax / 127.0f;
                scales[(size_t)table[(size_t)b * max_blocks + i] * s->num_kv_heads + kvh] = scale;
                for (int t = t0; t < t1; ++t)
                    for (int d = 0; d < D; ++d) {
                        const float x = contig[kvbo_contig_index(s, max_len, b, kvh, t, d)];
                        int8_t qv = 0;
                        if (scale > 0) {
                            float r = nearbyintf(x / scale);
                            if (r < -127.0f) r = -127.0f;
                            if (r > 127.0f) r = 127.0f;
                            qv = (int8_t)r;
                        }
                        paged[kvbo_paged_index(s, page_size, max_blocks, table, b, kvh, t, d)] = qv;
                    }
            }
}

void kvbo_dequantize_paged_i8(const kvbo_shape* s, int page_size, int max_blocks, const int32_t* table,
                              const int* lens, int max_len, const int8_t* paged, const float* scales,
                              float* contig) {
    for (int b = 0; b < s->batch; ++b)
        for (int kvh = 0; kvh < s->num_kv_heads; ++kvh)
            for (int t = 0; t < lens[b]; ++t) {
                const float scale =
                    scales[(size_t)table[(size_t)b * max_blocks + t / page_size] * s->num_kv_heads + kvh];
                for (int d = 0; d < s->head_dim; ++d)
                    contig[kvbo_contig_index(s, max_len, b, kvh, t, d)] =
                        (float)paged[kvbo_paged_index(s, page_size, max_blocks, table, b, kvh, t, d)] * scale;
            }
}

/* ---- fp64 two-pass attention ----------------------------------------------------------------- */

typedef struct {
    const kvbo_shape* s;
    const int* lens;
    int max_len;
    const float* q;
    const void* k;
    const void* v;
    int f16;
    float* out;
    float scale;
    int worker, threads;
} attn_job;

static inline double load_elem(const void* p, size_t i, int f16) {
    return f16 ? (double)kvbo_f16_to_f32(((const uint16_t*)p)[i]) : (double)((const float*)p)[i];
}

static void* attn_worker(void* arg) {
    const attn_job* j = (const attn_job*)arg;
    const kvbo_shape* s = j->s;
    const int D = s->head_dim, H = s->num_heads, G = s->num_heads / s->num_kv_heads;
    const int rows = s->batch * H;
    double* p = (double*)malloc(sizeof(double) * (size_t)(j->max_len > 0 ? j->max_len : 1));
    double* acc = (double*)malloc(sizeof(double) * (size_t)D);
    for (int row = j->worker; row < rows; row += j->threads) {
        const int b = row / H, h = row % H, kvh = h / G, len = j->lens[b];
        const float* qr = j->q + (size_t)row * D;
        double mx = -INFINITY;
        for (int t = 0; t < len; ++t) {
            const size_t base = kvbo_contig_index(s, j->max_len, b, kvh, t, 0);
            double dot = 0;
            for (int d = 0; d < D; ++d) dot += (double)qr[d] * load_elem(j->k, base + d, j->f16);
            p[t] = dot * j->scale;
            if (p[t] > mx) mx = p[t];
        }
        double sum = 0;
        for (int t = 0; t < len; ++t) sum += (p[t] = exp(p[t] - mx));
        for (int d = 0; d < D; ++d) acc[d] = 0.0;
        for (int t = 0; t < len; ++t) {
            const size_t base = kvbo_contig_index(s, j->max_len, b, kvh, t, 0);
            for (int d = 0; d < D; ++d) acc[d] += p[t] * load_elem(j->v, base + d, j->f16);
        }
        for (int d = 0; d < D; ++d) j->out[(size_t)row * D + d] = len ? (float)(acc[d] / sum) : 0.0f;
    }
    free(p);
    free(acc);
    return NULL;
}

static void attention_any(const kvbo_shape* s, const int* lens, int max_len, const float* q, const void* k,
                          const void* v, int f16, float* out, float scale, int threads) {
    const int rows = s->batch * s->num_heads;
    if (rows <= 0) return;
    if (threads < 1) threads = 1;
    if (threads > rows) threads = rows;
    attn_job* jobs = (attn_job*)malloc(sizeof(attn_job) * (size_t)threads);
    pthread_t* tids = (pthread_t*)malloc(sizeof(pthread_t) * (size_t)threads);
    for (int w = 0; w < threads; ++w) {
        attn_job j = {s, lens, max_len, q, k, v, f16, out, scale, w, threads};
        jobs[w] = j;
    }
    int started = 0;
    for (int w = 1; w < threads; ++w)
        if (pthread_create(&tids[w], NULL, attn_worker, &jobs[w]) == 0) started = w;
        else break;
    if (started < threads - 1) { /* could not start every worker: run the rest here */
        for (int w = started + 1; w < threads; ++w) attn_worker(&jobs[w]);
    }
    attn_worker(&jobs[0]);
    for (int w = 1; w <= started; ++w) pthread_join(tids[w], NULL);
    free(jobs);
    free(tids);
}

void kvbo_attention_f32(const kvbo_shape* s, const int* lens, int max_len, const float* q, const float* k,
                        const float* v, float* out, float scale, int threads) {
    attention_any(s, lens, max_len, q, k, v, 0, out, scale, threads);
}

void kvbo_attention_f16(const kvbo_shape* s, const int* lens, int max_len, const float* q,
                        const uint16_t* k, const uint16_t* v, float* out, float scale, int threads) {
    attention_any(s, lens, max_len, q, k, v, 1, out, scale, threads);
}

int kvbo_partition_state_f32(const kvbo_shape* s, const int* lens, int max_len, const float* q, const float* k,
                             const float* v, float scale, int part_tokens, int b, int h, int p, double* m,
                             double* l, double* o) {
    const int D = s->head_dim, G = s->num_heads / s->num_kv_heads, kvh = h / G, len = lens[b];
    const int t0 = p * part_tokens;
    if (t0 >= len) return 0;
    const int t1 = len < t0 + part_tokens ? len : t0 + part_tokens;
    const float* qr = q + ((size_t)b * s->num_heads + h) * D;
    double mx = -INFINITY;
    for (int t = t0; t < t1; ++t) {
        const size_t base = kvbo_contig_index(s, max_len, b, kvh, t, 0);
        double dot = 0;
        for (int d = 0; d < D; ++d) dot += (double)qr[d] * (double)k[base + d];
        if (dot * scale > mx) mx = dot * scale;
    }
    double sum = 0;
    for (int d = 0; d < D; ++d) o[d] = 0;
    for (int t = t0; t < t1; ++t) {
        const size_t base = kvbo_contig_index(s, max_len, b, kvh, t, 0);
        double dot = 0;
        for (int d = 0; d < D; ++d) dot += (double)qr[d] * (double)k[base + d];
        const double w = exp(dot * scale - mx);
        sum += w;
        for (int d = 0; d < D; ++d) o[d] += w * (double)v[base + d];
    }
    for (int d = 0; d < D; ++d) o[d] /= sum;
    *m = mx;
    *l = sum;
    return 1;
}

int kvbo_auto_part_tokens(int batch, int num_kv_heads, int max_len) {
    int part = 512;
    while (part > 64 && (size_t)batch * num_kv_heads * (size_t)((max_len + part - 1) / part) < 512) part /= 2;
    return part;
}

double kvbo_fp16_storage_bound(const kvbo_shape* s, const int* lens, int max_len, const float* q,
                               const float* k32, const float* v32) {
    const double u = 1.0 / 2048, scale = 1.0 / sqrt((double)s->head_dim);
    const int G = s->num_heads / s->num_kv_heads;
    double E = 0, vmax = 0;
    for (int b = 0; b < s->batch; ++b)
        for (int h = 0; h < s->num_heads; ++h)
            for (int t = 0; t < lens[b]; ++t) {
                double acc = 0;
                for (int d = 0; d < s->head_dim; ++d) {
                    const size_t i = kvbo_contig_index(s, max_len, b, h / G, t, d);
                    acc += fabs((double)q[((size_t)b * s->num_heads + h) * s->head_dim + d]) * fabs((double)k32[i]);
                    if (fabs((double)v32[i]) > vmax) vmax = fabs((double)v32[i]);
                }
                if (u * scale * acc > E) E = u * scale * acc;
            }
    return vmax * (u + expm1(2 * E)) + 2e-5;
}

double kvbo_i8_storage_bound(const kvbo_shape* s, const int* lens, int page_size, int max_blocks,
                             const int32_t* table, const float* q, const float* k_scale,
                             const float* v_scale) {
    const double scale = 1.0 / sqrt((double)s->head_dim);
    const int G = s->num_heads / s->num_kv_heads;
    double E = 0, vq = 0, vmax = 0;
    for (int b = 0; b < s->batch; ++b)
        for (int h = 0; h < s->num_heads; ++h) {
            double q1 = 0;
            for (int d = 0; d < s->head_dim; ++d) q1 += fabs((double)q[((size_t)b * s->num_heads + h) * s->head_dim + d]);
            for (int i = 0; i * page_size < lens[b]; ++i) {
                const size_t slot = (size_t)table[(size_t)b * max_blocks + i] * s->num_kv_heads + h / G;
                if (scale * q1 * k_scale[slot] / 2 > E) E = scale * q1 * k_scale[slot] / 2;
                if ((double)v_scale[slot] / 2 > vq) vq = (double)v_scale[slot] / 2;
                if (127.0 * v_scale[slot] > vmax) vmax = 127.0 * v_scale[slot];
            }
        }
    return vmax * expm1(2 * E) + vq + 2e-5;
}

/* ---- CPU model of the split-K decode kernel -------------------------------------------------- */

enum { kModelTile = 16, kModelMaxWaves = 8, kModelMaxD = 128 };

/* The GPU's exp unit returns 0 where the result would be subnormal; the kernel's one-hot and
 * dominant-key results depend on it. */
static inline float exp_ftz(float x) {
    const float e = expf(x);
    return e < FLT_MIN ? 0.0f : e;
}

typedef struct {
    const kvbo_shape* s;
    int kv_type, page_size, max_blocks;
    const int32_t* table;
    const int* lens;
    const float *q, *k_scale, *v_scale;
    const void *k, *v;
    float scale;
    int part_tokens, max_parts, waves;
    float *ws_out, *ws_ml, *out; /* workspace [B*H*max_parts + 1 spare][D] and [..][2], NaN-filled */
    int phase, worker, threads;
    int len_cap;     /* the kernel's live_len cap: min(max_blocks * page_size, max_parts * part_tokens) */
    int* violations; /* accesses that would leave the sequence's table row or its workspace slots */
} split_job;

/* The kernel's live_len: a length from `lens` (the device copy) clamped to [0, len_cap]. */
static int model_len(const split_job* j, int b) {
    const int len = j->lens[b];
    return len < 0 ? 0 : len > j->len_cap ? j->len_cap : len;
}

static void model_violation(const split_job* j) { __atomic_fetch_add(j->violations, 1, __ATOMIC_RELAXED); }

static void load_row(const void* pool, int kv_type, size_t at, int D, float* dst) {
    for (int d = 0; d < D; ++d) {
        if (kv_type == 0) dst[d] = ((const float*)pool)[at + d];
        else if (kv_type == 1) dst[d] = kvbo_f16_to_f32(((const uint16_t*)pool)[at + d]);
        else dst[d] = (float)((const int8_t*)pool)[at + d];
    }
}

/* One partition of one (sequence, query head): the decode kernel's workgroup, one head of its group. */
/* x rounded to fp16 and back (round to nearest even). */
static inline float round_f16(float x) { return kvbo_f16_to_f32(kvbo_f32_to_f16(x)); }

/* A signed byte digit of the int8 q split: rint(x) clamped to [-127, 127]. */
static inline float digit_i8(float x) {
    const float r = rintf(x);
    return r < -127.0f ? -127.0f : r > 127.0f ? 127.0f : r;
}

static void model_partition(const split_job* j, int b, int h, int part) {
    const kvbo_shape* s = j->s;
    const int D = s->head_dim, P = j->page_size, Hkv = s->num_kv_heads;
    const int kvh = h / (s->num_heads / Hkv);
    const int len = model_len(j, b);
    const int t0 = part * j->part_tokens;
    if (t0 >= len) return; /* an empty partition writes nothing */
    const int t1 = len < t0 + j->part_tokens ? len : t0 + j->part_tokens;
    const float* qr = j->q + ((size_t)b * s->num_heads + h) * D;
    const int32_t* bt = j->table + (size_t)b * j->max_blocks;
    float wm[kModelMaxWaves], wl[kModelMaxWaves], wacc[kModelMaxWaves][kModelMaxD];
    float krow[kModelMaxD], vrow[kModelTile][kModelMaxD], sc[kModelTile], vs[kModelTile];
    /* q in the kernel's number formats (paged_decode_impl.hpp: the q split). q * scale is brought
       below 2^14 (fp16) or 2^7 (int8) by a power of two `down`; the scores are multiplied back by
       up = 1 / down. fp16: each element as a high and a low fp16 part (the MFMA's two columns of
       the head). int8: three signed byte digits, x = d0 + d1 / 2^7 + d2 / 2^14 (the integer MFMA's
       operands). fp32: q * scale as it is. */
    float qhi[kModelMaxD], qlo[kModelMaxD], qd0[kModelMaxD], qd1[kModelMaxD], qd2[kModelMaxD];
    float up = 1.0f, amax = 0.0f;
    for (int d = 0; d < D; ++d) {
        const float a = fabsf(qr[d] * j->scale);
        amax = a > amax ? a : amax;
    }
    int e = 0;
    if (j->kv_type != 0 && amax > 0.0f && amax <= FLT_MAX) {
        frexpf(amax, &e); /* amax < 2^e */
        e -= j->kv_type == 2 ? 7 : 14;
    }
    up = ldexpf(1.0f, e);
    const float down = ldexpf(1.0f, -e);
    for (int d = 0; d < D; ++d) {
        const float x = qr[d] * j->scale * (j->kv_type == 0 ? 1.0f : down);
        qhi[d] = j->kv_type == 1 ? round_f16(x) : x;
        qlo[d] = j->kv_type == 1 ? round_f16(x - qhi[d]) : 0.0f;
        qd0[d] = digit_i8(x);
        const float r1 = (x - qd0[d]) * 128.0f;
        qd1[d] = digit_i8(r1);
        qd2[d] = digit_i8((r1 - qd1[d]) * 128.0f);
    }
    if (j->kv_type == 2 && !(amax <= FLT_MAX)) up = NAN; /* a non-finite q: its scores are NaN */
    for (int w = 0; w < j->waves; ++w) {
        float m = -INFINITY, l = 0.0f;
        float* acc = wacc[w];
        /* p enters the P*V product as a high and a low fp16 part (fp16 and int8 caches), each with
           its own accumulator column; int8: p * v_scale * 2^-ve, ve the exponent of the largest V
           scale the wave has met, the accumulators rescaled when it grows and scaled by 2^ve at
           the end. */
        float acc_lo[kModelMaxD];
        int ve = -160;
        float vdown = 1.0f;
        for (int d = 0; d < D; ++d) acc[d] = acc_lo[d] = 0.0f;
        for (int tt = t0 + w * kModelTile; tt < t1; tt += j->waves * kModelTile) {
            const int n = t1 - tt < kModelTile ? t1 - tt : kModelTile; /* tokens past t1 are masked */
            float mt = -INFINITY;
            for (int i = 0; i < n; ++i) {
                const int t = tt + i;
                if (t / P >= j->max_blocks) model_violation(j); /* the clamp keeps t < max_blocks * P */
                const int32_t id = t / P < j->max_blocks ? bt[t / P] : 0;
                /* a block id of -1 (an unused entry: seq_lens disagrees with the host) reads as
                   zeros, with block 0's scales, as in the kernel */
                const size_t blk = id < 0 ? 0 : (size_t)id;
                const size_t row = ((blk * Hkv + kvh) * P + t % P) * D;
                load_row(j->k, j->kv_type, row, D, krow);
                load_row(j->v, j->kv_type, row, D, vrow[i]);
                if (id < 0)
                    for (int d = 0; d < D; ++d) krow[d] = vrow[i][d] = 0.0f;
                if (j->kv_type == 2) { /* exact integer dot products per digit, combined in fp32 */
                    float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f;
                    for (int d = 0; d < D; ++d) {
                        s0 += krow[d] * qd0[d];
                        s1 += krow[d] * qd1[d];
                        s2 += krow[d] * qd2[d];
                    }
                    sc[i] = (fmaf(s2, 1.0f / 16384.0f, s0) + s1 * (1.0f / 128.0f)) * up;
                    sc[i] *= j->k_scale[blk * Hkv + kvh];
                    vs[i] = j->v_scale[blk * Hkv + kvh];
                } else { /* the high and the low column, summed */
                    float shi = 0.0f, slo = 0.0f;
                    for (int d = 0; d < D; ++d) {
                        shi += krow[d] * qhi[d];
                        slo += krow[d] * qlo[d];
                    }
                    sc[i] = (shi + slo) * up;
                    vs[i] = 1.0f;
                }
                if (sc[i] > mt) mt = sc[i];
            }
            if (j->kv_type == 2) { /* the wave's V-scale exponent */
                float vmx = 0.0f;
                for (int i = 0; i < n; ++i) vmx = vs[i] > vmx ? vs[i] : vmx;
                int ev = ve;
                if (vmx > 0.0f) frexpf(vmx, &ev); /* vmx < 2^ev */
                if (ev > ve) {
                    const float nd = ldexpf(1.0f, -ev);
                    const float resc = nd / vdown; /* a power of two: exact */
                    for (int d = 0; d < D; ++d) {
                        acc[d] *= resc;
                        acc_lo[d] *= resc;
                    }
                    ve = ev;
                    vdown = nd;
                }
            }
            const float m_new = m > mt ? m : mt;
            const float corr = exp_ftz(m - m_new); /* rescales the tile-old state to the new max */
            l *= corr;
            for (int d = 0; d < D; ++d) {
                acc[d] *= corr;
                acc_lo[d] *= corr;
            }
            for (int i = 0; i < n; ++i) {
                const float p = exp_ftz(sc[i] - m_new);
                l += p;
                const float pv = p * vs[i] * vdown;
                const float phi = j->kv_type == 0 ? pv : round_f16(pv);
                const float plo = j->kv_type == 0 ? 0.0f : round_f16(pv - phi);
                for (int d = 0; d < D; ++d) {
                    acc[d] += phi * vrow[i][d];
                    acc_lo[d] += plo * vrow[i][d];
                }
            }
            m = m_new;
        }
        const float vupf = 1.0f / vdown; /* 2^ve (1 for fp32 and fp16) */
        for (int d = 0; d < D; ++d) acc[d] = (acc[d] + acc_lo[d]) * vupf;
        wm[w] = m;
        wl[w] = l;
    }
    /* the workgroup's merge of its wave states */
    float M = -INFINITY, L = 0.0f, wt[kModelMaxWaves];
    for (int w = 0; w < j->waves; ++w)
        if (wm[w] > M) M = wm[w];
    for (int w = 0; w < j->waves; ++w) {
        wt[w] = exp_ftz(wm[w] - M);
        L += wl[w] * wt[w];
    }
    const size_t slot = ((size_t)b * s->num_heads + h) * j->max_parts + part;
    for (int d = 0; d < D; ++d) {
        float o = 0.0f;
        for (int w = 0; w < j->waves; ++w) o += wacc[w][d] * wt[w];
        j->ws_out[slot * D + d] = o * (1.0f / L); /* the kernel multiplies by one reciprocal */
    }
    j->ws_ml[2 * slot] = M;
    j->ws_ml[2 * slot + 1] = L;
}

/* paged_reduce for one (sequence, query head). */
static void model_reduce(const split_job* j, int b, int h) {
    const int D = j->s->head_dim;
    const size_t row = (size_t)b * j->s->num_heads + h;
    float* out = j->out + row * D;
    int parts = (model_len(j, b) + j->part_tokens - 1) / j->part_tokens;
    if (parts > j->max_parts) { /* the clamp keeps parts <= max_parts */
        model_violation(j);
        parts = j->max_parts;
    }
    if (parts == 0) { /* an empty sequence attends to nothing */
        for (int d = 0; d < D; ++d) out[d] = 0.0f;
        return;
    }
    const float* ml = j->ws_ml + 2 * row * j->max_parts;
    const float* po = j->ws_out + row * j->max_parts * D;
    if (parts == 1) { /* one partition: its normalised output is the output */
        for (int d = 0; d < D; ++d) out[d] = po[d];
        return;
    }
    float M = -INFINITY;
    for (int i = 0; i < parts; ++i)
        if (ml[2 * i] > M) M = ml[2 * i];
    for (int d = 0; d < D; ++d) {
        float L = 0.0f, o = 0.0f;
        for (int i = 0; i < parts; ++i) {
            const float w = ml[2 * i + 1] * exp_ftz(ml[2 * i] - M); /* l_i exp(m_i - M) */
            L += w;
            o += w * po[(size_t)i * D + d];
        }
        out[d] = o * (1.0f / L);
    }
}

static void* split_worker(void* arg) {
    const split_job* j = (const split_job*)arg;
    const int H = j->s->num_heads, rows = j->s->batch * H;
    for (int r = j->worker; r < rows; r += j->threads) {
        if (j->phase == 0)
            for (int p = 0; p < j->max_parts; ++p) model_partition(j, r / H, r % H, p);
        else
            model_reduce(j, r / H, r % H);
    }
    return NULL;
}

int kvbo_split_decode(const kvbo_shape* s, int kv_type, int page_size, int max_blocks, const int32_t* table,
                      const int* lens, int max_len, const float* q, const void* k_pool, const void* v_pool,
                      const float* k_scale, const float* v_scale, float scale, int part_tokens, int waves,
                      float* part_out, float* part_ml, float* out, int threads) {
    if (!s || s->batch < 0 || s->num_kv_heads <= 0 || s->num_heads % s->num_kv_heads || s->head_dim <= 0 ||
        s->head_dim > kModelMaxD || kv_type < 0 || kv_type > 2 || page_size <= 0 || max_len < 0 ||
        part_tokens < 0 || waves < 1 || waves > kModelMaxWaves || (kv_type == 2 && (!k_scale || !v_scale)))
        return -1;
    if (part_tokens == 0) part_tokens = kvbo_auto_part_tokens(s->batch, s->num_kv_heads, max_len);
    const int max_parts = max_len > 0 ? (max_len + part_tokens - 1) / part_tokens : 1;
    const int D = s->head_dim, rows = s->batch * s->num_heads;
    const size_t slots = (size_t)rows * max_parts + 1; /* one spare, NaN, past the last row */
    float* ws_out = (float*)malloc(sizeof(float) * slots * D);
    float* ws_ml = (float*)malloc(sizeof(float) * slots * 2);
    if (!ws_out || !ws_ml) {
        free(ws_out);
        free(ws_ml);
        return -1;
    }
    for (size_t i = 0; i < slots * D; ++i) ws_out[i] = NAN;
    for (size_t i = 0; i < slots * 2; ++i) ws_ml[i] = NAN;
    if (threads < 1) threads = 1;
    if (rows > 0 && threads > rows) threads = rows;
    split_job* jobs = (split_job*)malloc(sizeof(split_job) * (size_t)threads);
    const long long cap_table = (long long)max_blocks * page_size, cap_ws = (long long)max_parts * part_tokens;
    const int len_cap = (int)(cap_table < cap_ws ? cap_table : cap_ws);
    int violations = 0;
    pthread_t* tids = (pthread_t*)malloc(sizeof(pthread_t) * (size_t)threads);
    for (int phase = 0; phase < 2 && rows > 0; ++phase) { /* decode, then merge: two kernels */
        for (int w = 0; w < threads; ++w) {
            split_job j = {s, kv_type, page_size, max_blocks, table, lens, q, k_scale, v_scale, k_pool, v_pool,
                           scale, part_tokens, max_parts, waves, ws_out, ws_ml, out, phase, w, threads,
                           len_cap, &violations};
            jobs[w] = j;
        }
        int started = 0;
        for (int w = 1; w < threads; ++w)
            if (pthread_create(&tids[w], NULL, split_worker, &jobs[w]) == 0) started = w;
            else break;
        for (int w = started + 1; w < threads; ++w) split_worker(&jobs[w]);
        split_worker(&jobs[0]);
        for (int w = 1; w <= started; ++w) pthread_join(tids[w], NULL);
    }
    if (part_out) memcpy(part_out, ws_out, sizeof(float) * (slots - 1) * D);
    if (part_ml) memcpy(part_ml, ws_ml, sizeof(float) * (slots - 1) * 2);
    free(jobs);
    free(tids);
    free(ws_out);
    free(ws_ml);
    return violations ? -2 : max_parts;
}
