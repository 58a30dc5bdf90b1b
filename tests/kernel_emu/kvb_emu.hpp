// A CPU emulation of the gfx950 execution model, for testing this repository's HIP sources on a
// machine without a GPU. Test infrastructure only: it is never linked into libkvb_hip.so, and no
// product path can reach it.
//
// The package's HIP sources (kv-cache-bench_amd/csrc/*.hip, including paged_decode_impl.hpp) are
// compiled unchanged as C++ for x86-64 against this header, which stands in for <hip/hip_runtime.h>.
// The only edit is mechanical and made by tests/kernel_emu/Makefile on a copy: the inline-asm
// `s_waitcnt vmcnt(0)` becomes kvbemu_wait_vmem() (loads complete at once here).
//
// Execution model:
//  * A launch runs its workgroups one after another. Each thread of a workgroup is a fiber (its own
//    stack, switched by kvbemu's context switch); a fiber runs until it reaches a cross-lane
//    operation or a barrier, then yields.
//  * A cross-lane operation (DPP, lane shuffles, readlane, ballot, the MFMAs, the transposing LDS
//    reads, the wave barrier) completes when all lanes of the wave have reached it: the last lane
//    to arrive computes every lane's result from every lane's operands. Lanes of one wave that reach
//    different operations, or a wave whose lanes exit while others wait, stop the launch with an
//    error: the kernels must keep their cross-lane operations in wave-uniform control flow.
//  * __syncthreads waits for every thread of the workgroup that has not exited.
//  * Memory is one flat space: LDS (__shared__) is a static array per kernel instantiation, shared by
//    the fibers of the running workgroup. Buffer loads and stores apply the buffer resource's range
//    check (num_records), and every access they make must lie inside a hipMalloc allocation or a
//    registered __device__ symbol; anything else stops the launch with an error (the launch then
//    returns hipErrorLaunchFailure).
//  * MFMA operand layouts are CDNA's: for 16x16xK, lane l holds row (A) or column (B) l % 16 and
//    the K slice 8 (l / 16) .. (f16, 8 per lane), 16 (l / 16) .. (i8) or l / 16 (f32); the result
//    lane l holds rows 4 (l / 16) + i (i < 4) of column l % 16. Products are summed in double and
//    rounded once (the hardware's internal order is not specified; results agree to rounding).
//  * v_exp_f32 (__builtin_amdgcn_exp2f) returns 0 below 2^-126, as the GPU's does.
#pragma once

#include <algorithm>
#include <cmath>
#include <cstddef>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <type_traits>
#include <utility>

// ---- HIP's language vocabulary ----------------------------------------------------------------
#define __global__
#define __device__
#define __host__
#define __shared__ static
#define __forceinline__ inline
#define __launch_bounds__(...)
#define __align__(n) __attribute__((aligned(n)))
// The register-budget attribute and the LDS / constant address-space qualifiers have no CPU
// meaning: one flat memory here.
#define amdgpu_waves_per_eu(...) unused
#define address_space(n) unused

#define __HIP_MEMORY_SCOPE_SINGLETHREAD 1
#define __HIP_MEMORY_SCOPE_WAVEFRONT 2
#define __HIP_MEMORY_SCOPE_WORKGROUP 3
#define __HIP_MEMORY_SCOPE_AGENT 4
#define __HIP_MEMORY_SCOPE_SYSTEM 5

struct dim3 {
    uint32_t x, y, z;
    constexpr dim3(uint32_t x_ = 1, uint32_t y_ = 1, uint32_t z_ = 1) : x(x_), y(y_), z(z_) {}
};
struct __attribute__((aligned(16))) uint4 {
    uint32_t x, y, z, w;
};
struct __attribute__((aligned(16))) float4 {
    float x, y, z, w;
};
struct __attribute__((aligned(8))) float2 {
    float x, y;
};
inline uint4 make_uint4(uint32_t x, uint32_t y, uint32_t z, uint32_t w) { return uint4{x, y, z, w}; }
inline float4 make_float4(float x, float y, float z, float w) { return float4{x, y, z, w}; }
inline float2 make_float2(float x, float y) { return float2{x, y}; }

// HIP's integer and float min / max overloads
inline int min(int a, int b) { return a < b ? a : b; }
inline int max(int a, int b) { return a > b ? a : b; }
inline unsigned min(unsigned a, unsigned b) { return a < b ? a : b; }
inline unsigned max(unsigned a, unsigned b) { return a > b ? a : b; }
inline long long min(long long a, long long b) { return a < b ? a : b; }
inline long long max(long long a, long long b) { return a > b ? a : b; }
inline unsigned long long min(unsigned long long a, unsigned long long b) { return a < b ? a : b; }
inline unsigned long long max(unsigned long long a, unsigned long long b) { return a > b ? a : b; }
inline long min(long a, long b) { return a < b ? a : b; }
inline long max(long a, long b) { return a > b ? a : b; }
inline unsigned long min(unsigned long a, unsigned long b) { return a < b ? a : b; }
inline unsigned long max(unsigned long a, unsigned long b) { return a > b ? a : b; }
inline float min(float a, float b) { return fminf(a, b); }
inline float max(float a, float b) { return fmaxf(a, b); }
inline double min(double a, double b) { return fmin(a, b); }
inline double max(double a, double b) { return fmax(a, b); }

inline int __popcll(unsigned long long x) { return __builtin_popcountll(x); }
inline int __popc(unsigned x) { return __builtin_popcount(x); }
inline int __ffsll(unsigned long long x) { return __builtin_ffsll((long long)x); }
inline int __ffsll(long long x) { return __builtin_ffsll(x); }
inline unsigned __umulhi(unsigned a, unsigned b) { return (unsigned)(((unsigned long long)a * b) >> 32); }
inline float __expf(float x) { return expf(x); }

namespace kvbemu {

// ---- execution state -----------------------------------------------------------------------------
struct Fiber;
struct Group;
extern Fiber* g_cur;  // the running thread
extern Group* g_grp;  // its workgroup

struct Idx {
    uint32_t x, y, z;
};
struct Fiber {
    void* sp = nullptr;  // saved stack pointer while switched out
    char* stack = nullptr;
    Idx tid{0, 0, 0};
    int linear = 0, lane = 0, wave = 0;
    bool done = false;
};

// The running workgroup: indices, the wave exchange areas and the barrier.
constexpr int kSlotBytes = 64;  // per-lane operand / result bytes of one cross-lane operation
struct WaveSync {
    uint64_t gen = 0;
    int arrived = 0, lanes = 64, exited = 0;
    uint64_t key = 0;
    const char* what = nullptr;
    alignas(16) unsigned char in[64][kSlotBytes];
    alignas(16) unsigned char out[64][kSlotBytes];
};
struct Group {
    Idx bid{0, 0, 0}, grid{1, 1, 1}, block{1, 1, 1};
    int threads = 0, live = 0;
    uint64_t bar_gen = 0;
    int bar_arrived = 0;
    uint64_t progress = 0;
    WaveSync* waves = nullptr;
    const std::function<void()>* body = nullptr;
};

// Stops the running launch with an error (the launch returns hipErrorLaunchFailure and
// hipGetLastError reports it; the message goes to stderr and to kvbemu_last_error()).
[[noreturn]] void fail(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
void yield();  // back to the workgroup's scheduler

// One cross-lane operation: every lane deposits `in`; when all lanes of the wave have, the last
// computes outs[l] = f(ins)[l] for all lanes. `key` identifies the operation and its uniform
// operands; lanes that disagree on it stop the launch.
template <class In, class Out, class F>
Out wave_op(uint64_t key, const char* what, const In& in, F&& f) {
    static_assert(sizeof(In) <= kSlotBytes && sizeof(Out) <= kSlotBytes, "operand too large");
    static_assert(std::is_trivially_copyable_v<In> && std::is_trivially_copyable_v<Out>, "operand type");
    Fiber* me = g_cur;
    WaveSync& w = g_grp->waves[me->wave];
    if (w.exited) fail("%s in wave %d after %d of its lanes exited", what, me->wave, w.exited);
    if (w.arrived == 0) {
        w.key = key;
        w.what = what;
    } else if (w.key != key) {
        fail("lanes of wave %d reached different cross-lane operations (%s / %s)", me->wave, w.what, what);
    }
    std::memcpy(w.in[me->lane], &in, sizeof(In));
    const uint64_t my = w.gen;
    ++g_grp->progress;
    if (++w.arrived == w.lanes) {
        In ins[64];
        Out outs[64];
        std::memset(static_cast<void*>(ins), 0, sizeof(ins));
        std::memset(static_cast<void*>(outs), 0, sizeof(outs));
        for (int l = 0; l < w.lanes; ++l) std::memcpy(&ins[l], w.in[l], sizeof(In));
        f(ins, outs, w.lanes);
        for (int l = 0; l < 64; ++l) std::memcpy(w.out[l], &outs[l], sizeof(Out));
        w.arrived = 0;
        ++w.gen;
    } else {
        while (w.gen == my) yield();
    }
    Out r;
    std::memcpy(&r, w.out[me->lane], sizeof(Out));
    return r;
}

void syncthreads();
void wait_vmem();  // s_waitcnt vmcnt(0): loads and stores complete at once here

// ---- memory: allocations that buffer accesses may touch ---------------------------------------
void track(const void* p, size_t bytes);
void untrack(const void* p);
void check_access(const void* p, size_t bytes, const char* what);
template <class T>
T* symbol(T* p) {  // HIP_SYMBOL: a __device__ variable, registered once
    track(p, sizeof(T));
    return p;
}

// ---- per-lane operations -------------------------------------------------------------------------
inline float exp2_hw(float x) {
    const float r = exp2f(x);
    return r < 0x1p-126f ? 0.0f : r;  // (NaN compares false and stays NaN)
}
// v_perm_b32: byte i of the result is byte sel_i of the 64-bit value s0:s1 (s1 low); selectors
// 8-11 give the sign of bytes 1, 3, 5, 7 repeated, 12 gives 0x00, 13 and above 0xFF.
inline uint32_t perm(uint32_t s0, uint32_t s1, uint32_t sel) {
    const uint64_t v = ((uint64_t)s0 << 32) | s1;
    uint32_t r = 0;
    for (int i = 0; i < 4; ++i) {
        const uint32_t b = (sel >> (8 * i)) & 0xFFu;
        uint32_t o;
        if (b < 8) o = (uint32_t)(v >> (8 * b)) & 0xFFu;
        else if (b < 12) o = ((v >> (8 * (2 * (b - 8) + 1) + 7)) & 1u) ? 0xFFu : 0u;
        else if (b == 12) o = 0u;
        else o = 0xFFu;
        r |= o << (8 * i);
    }
    return r;
}

struct BufferRsrc {
    const char* base;
    uint32_t num_records;
    int32_t flags;
    int32_t stride;
};
inline BufferRsrc make_buffer_rsrc(const void* p, short stride, int num_records, int flags) {
    if (stride != 0) fail("buffer resource with a stride (%d): only raw buffers are emulated", (int)stride);
    return BufferRsrc{static_cast<const char*>(p), (uint32_t)num_records, flags, stride};
}
// Raw buffer access of `dwords` dwords at voffset + soffset: each dword lies inside num_records or
// reads as 0 (a store skips it); the dwords in range must lie inside an allocation.
inline void buffer_read(const BufferRsrc& r, int voffset, int soffset, uint32_t* dst, int dwords) {
    const uint64_t off = (uint64_t)(uint32_t)voffset + (uint64_t)(uint32_t)soffset;
    for (int i = 0; i < dwords; ++i) {
        const uint64_t o = off + 4u * (uint64_t)i;
        if (o + 4 <= r.num_records) {
            check_access(r.base + o, 4, "buffer load");
            std::memcpy(&dst[i], r.base + o, 4);
        } else {
            dst[i] = 0;
        }
    }
}
inline void buffer_write(const BufferRsrc& r, int voffset, int soffset, const uint32_t* src, int dwords) {
    const uint64_t off = (uint64_t)(uint32_t)voffset + (uint64_t)(uint32_t)soffset;
    for (int i = 0; i < dwords; ++i) {
        const uint64_t o = off + 4u * (uint64_t)i;
        if (o + 4 <= r.num_records) {
            check_access(r.base + o, 4, "buffer store");
            std::memcpy(const_cast<char*>(r.base) + o, &src[i], 4);
        }
    }
}

typedef uint32_t u32x4_emu __attribute__((ext_vector_type(4)));
inline u32x4_emu raw_buffer_load_b128(BufferRsrc r, int voffset, int soffset, int /*aux*/) {
    uint32_t d[4];
    buffer_read(r, voffset, soffset, d, 4);
    return u32x4_emu{d[0], d[1], d[2], d[3]};
}
inline uint32_t raw_buffer_load_b32(BufferRsrc r, int voffset, int soffset, int /*aux*/) {
    uint32_t d;
    buffer_read(r, voffset, soffset, &d, 1);
    return d;
}
inline void raw_buffer_store_b128(u32x4_emu v, BufferRsrc r, int voffset, int soffset, int /*aux*/) {
    const uint32_t d[4] = {v[0], v[1], v[2], v[3]};
    buffer_write(r, voffset, soffset, d, 4);
}
typedef uint32_t u32x2_emu __attribute__((ext_vector_type(2)));
inline u32x2_emu raw_buffer_load_b64(BufferRsrc r, int voffset, int soffset, int /*aux*/) {
    uint32_t d[2];
    buffer_read(r, voffset, soffset, d, 2);
    return u32x2_emu{d[0], d[1]};
}
inline void raw_buffer_store_b64(u32x2_emu v, BufferRsrc r, int voffset, int soffset, int /*aux*/) {
    const uint32_t d[2] = {v[0], v[1]};
    buffer_write(r, voffset, soffset, d, 2);
}

// ---- cross-lane operations --------------------------------------------------------------------------
constexpr uint64_t op_key(uint64_t op, uint64_t a = 0, uint64_t b = 0) { return (op << 56) ^ (a << 24) ^ b; }

// DPP source lane of lane l, or -1 when the control names no lane for it.
inline int dpp_source(int ctrl, int l) {
    const int row = l >> 4, r = l & 15;
    if (ctrl >= 0 && ctrl <= 0xFF) return (l & ~3) | ((ctrl >> (2 * (l & 3))) & 3);  // quad_perm
    if (ctrl >= 0x101 && ctrl <= 0x10F) return r + (ctrl & 15) < 16 ? l + (ctrl & 15) : -1;  // row_shl
    if (ctrl >= 0x111 && ctrl <= 0x11F) return r >= (ctrl & 15) ? l - (ctrl & 15) : -1;     // row_shr
    if (ctrl >= 0x121 && ctrl <= 0x12F) return (l & ~15) | ((r - (ctrl & 15)) & 15);          // row_ror
    if (ctrl == 0x140) return (l & ~15) | (15 - r);                                           // row_mirror
    if (ctrl == 0x141) return (l & ~7) | (7 - (l & 7));                                       // row_half_mirror
    if (ctrl == 0x142) return row > 0 ? 16 * row - 1 : -1;                                    // row_bcast:15
    if (ctrl == 0x143) return row >= 2 ? 31 : -1;                                             // row_bcast:31
    fail("DPP control 0x%x is not emulated", ctrl);
}
template <class T>
T update_dpp(T old, T src, int ctrl, int row_mask, int bank_mask, bool bound_ctrl) {
    static_assert(sizeof(T) == 4, "32-bit DPP only");
    struct In {
        T old, src;
    };
    return wave_op<In, T>(op_key(1, (uint64_t)ctrl, (uint64_t)(row_mask << 8 | bank_mask << 1 | bound_ctrl)), "DPP",
                          In{old, src}, [&](const In* ins, T* outs, int n) {
                              for (int l = 0; l < n; ++l) {
                                  if (!((row_mask >> (l >> 4)) & 1) || !((bank_mask >> ((l & 15) >> 2)) & 1)) {
                                      outs[l] = ins[l].old;  // a disabled row or bank keeps its old value
                                      continue;
                                  }
                                  const int s = dpp_source(ctrl, l);
                                  if (s < 0 || s >= n) outs[l] = bound_ctrl ? T{} : ins[l].old;
                                  else outs[l] = ins[s].src;
                              }
                          });
}
// mov_dpp: update_dpp with no old value (the kernels use it with every row and bank enabled, where the
// old value is never taken; elsewhere it stands in as 0).
template <class T>
T mov_dpp(T src, int ctrl, int row_mask, int bank_mask, bool bound_ctrl) {
    return update_dpp(T{}, src, ctrl, row_mask, bank_mask, bound_ctrl);
}
template <class T>
T shfl_xor(T v, int mask, int width) {
    static_assert(sizeof(T) <= 8, "shuffle of a 4- or 8-byte value");
    return wave_op<T, T>(op_key(2, (uint64_t)mask, (uint64_t)width), "__shfl_xor", v, [&](const T* ins, T* outs, int n) {
        for (int l = 0; l < n; ++l) {
            int s = l ^ mask;
            if (s >= ((l + width) & ~(width - 1))) s = l;
            outs[l] = s < n ? ins[s] : ins[l];
        }
    });
}
inline int readlane(int v, int i) {
    struct In {
        int v, i;
    };
    return wave_op<In, int>(op_key(3), "readlane", In{v, i}, [&](const In* ins, int* outs, int n) {
        const int idx = ins[0].i;
        for (int l = 0; l < n; ++l)
            if (ins[l].i != idx) fail("readlane with a lane index that differs between lanes");
        if (idx < 0 || idx >= 64) fail("readlane of lane %d", idx);
        for (int l = 0; l < n; ++l) outs[l] = idx < n ? ins[idx].v : 0;
    });
}
inline int readfirstlane(int v) {
    return wave_op<int, int>(op_key(4), "readfirstlane", v, [](const int* ins, int* outs, int n) {
        for (int l = 0; l < n; ++l) outs[l] = ins[0];
    });
}
inline unsigned long long ballot(bool pred) {
    return wave_op<int, unsigned long long>(op_key(5), "ballot", pred ? 1 : 0, [](const int* ins, unsigned long long* outs, int n) {
        unsigned long long m = 0;
        for (int l = 0; l < n; ++l) m |= (unsigned long long)(ins[l] != 0) << l;
        for (int l = 0; l < n; ++l) outs[l] = m;
    });
}
inline void wave_barrier() {
    (void)wave_op<int, int>(op_key(6), "wave barrier", 0, [](const int*, int*, int) {});
}

typedef _Float16 half8_emu __attribute__((ext_vector_type(8)));
typedef float floatx4_emu __attribute__((ext_vector_type(4)));
typedef int i32x4_emu __attribute__((ext_vector_type(4)));
typedef int i32x2_emu __attribute__((ext_vector_type(2)));
typedef __fp16 fp16x4_emu __attribute__((__vector_size__(4 * sizeof(__fp16))));

// D = C + A B for a 16x16 tile; A16[row][k], B16[k][col] gathered from the lanes as CDNA lays them
// out (see the header comment), K = kk.
template <class E, int PER>
void mfma_16x16(const E* a, const E* b, const float* c, float* d, int n) {
    constexpr int KK = 4 * PER;
    double A[16][KK] = {}, B[KK][16] = {};
    for (int l = 0; l < n; ++l)
        for (int e = 0; e < PER; ++e) {
            A[l & 15][PER * (l >> 4) + e] = (double)a[l * PER + e];
            B[PER * (l >> 4) + e][l & 15] = (double)b[l * PER + e];
        }
    for (int l = 0; l < 64; ++l)
        for (int i = 0; i < 4; ++i) {
            const int row = 4 * (l >> 4) + i, col = l & 15;
            double s = 0.0;
            for (int k = 0; k < KK; ++k) s += A[row][k] * B[k][col];
            d[l * 4 + i] = l < n ? (float)((double)c[l * 4 + i] + s) : 0.0f;
        }
}
inline floatx4_emu mfma_f32_16x16x32_f16(half8_emu a, half8_emu b, floatx4_emu c, int cbsz, int abid, int blgp) {
    if (cbsz || abid || blgp) fail("MFMA broadcast controls are not emulated");
    struct In {
        half8_emu a, b;
        floatx4_emu c;
    };
    return wave_op<In, floatx4_emu>(op_key(7), "v_mfma_f32_16x16x32_f16", In{a, b, c}, [](const In* ins, floatx4_emu* outs, int n) {
        float A[64 * 8], B[64 * 8], C[64 * 4], D[64 * 4];
        for (int l = 0; l < 64; ++l) {
            for (int e = 0; e < 8; ++e) {
                A[l * 8 + e] = (float)ins[l].a[e];
                B[l * 8 + e] = (float)ins[l].b[e];
            }
            for (int i = 0; i < 4; ++i) C[l * 4 + i] = ins[l].c[i];
        }
        mfma_16x16<float, 8>(A, B, C, D, n);
        for (int l = 0; l < 64; ++l) outs[l] = floatx4_emu{D[l * 4], D[l * 4 + 1], D[l * 4 + 2], D[l * 4 + 3]};
    });
}
inline floatx4_emu mfma_f32_16x16x4f32(float a, float b, floatx4_emu c, int cbsz, int abid, int blgp) {
    if (cbsz || abid || blgp) fail("MFMA broadcast controls are not emulated");
    struct In {
        float a, b;
        floatx4_emu c;
    };
    return wave_op<In, floatx4_emu>(op_key(8), "v_mfma_f32_16x16x4_f32", In{a, b, c}, [](const In* ins, floatx4_emu* outs, int n) {
        float A[64], B[64], C[64 * 4], D[64 * 4];
        for (int l = 0; l < 64; ++l) {
            A[l] = ins[l].a;
            B[l] = ins[l].b;
            for (int i = 0; i < 4; ++i) C[l * 4 + i] = ins[l].c[i];
        }
        mfma_16x16<float, 1>(A, B, C, D, n);
        for (int l = 0; l < 64; ++l) outs[l] = floatx4_emu{D[l * 4], D[l * 4 + 1], D[l * 4 + 2], D[l * 4 + 3]};
    });
}
inline i32x4_emu mfma_i32_16x16x64_i8(i32x4_emu a, i32x4_emu b, i32x4_emu c, int cbsz, int abid, int blgp) {
    if (cbsz || abid || blgp) fail("MFMA broadcast controls are not emulated");
    struct In {
        i32x4_emu a, b, c;
    };
    return wave_op<In, i32x4_emu>(op_key(9), "v_mfma_i32_16x16x64_i8", In{a, b, c}, [](const In* ins, i32x4_emu* outs, int n) {
        int8_t A[16][64] = {}, B[64][16] = {};
        for (int l = 0; l < n; ++l) {
            int8_t ab[16], bb[16];
            std::memcpy(ab, &ins[l].a, 16);
            std::memcpy(bb, &ins[l].b, 16);
            for (int e = 0; e < 16; ++e) {
                A[l & 15][16 * (l >> 4) + e] = ab[e];
                B[16 * (l >> 4) + e][l & 15] = bb[e];
            }
        }
        for (int l = 0; l < 64; ++l)
            for (int i = 0; i < 4; ++i) {
                const int row = 4 * (l >> 4) + i, col = l & 15;
                uint32_t s = 0;  // (int32 arithmetic wraps, as the hardware's)
                for (int k = 0; k < 64; ++k) s += (uint32_t)((int)A[row][k] * (int)B[k][col]);
                outs[l][i] = l < n ? (int)((uint32_t)ins[l].c[i] + s) : 0;
            }
    });
}

// ds_read_b64_tr_b16 / _b8: in each group of 16 lanes, the 8 bytes that lane i addresses form part
// i of a flat sequence F (4 halves or 8 bytes per lane); lane i receives F[i], F[i + 16], ...
inline fp16x4_emu ds_read_tr16_b64(const void* p) {
    return wave_op<const void*, fp16x4_emu>(op_key(10), "ds_read_b64_tr_b16", p, [](const void* const* ins, fp16x4_emu* outs, int n) {
        for (int g = 0; g < 4; ++g) {
            uint16_t F[64];
            for (int i = 0; i < 16; ++i) {
                const int l = 16 * g + i;
                if (l < n) std::memcpy(&F[4 * i], ins[l], 8);
                else std::memset(&F[4 * i], 0, 8);
            }
            for (int i = 0; i < 16; ++i) {
                uint16_t r[4] = {F[i], F[i + 16], F[i + 32], F[i + 48]};
                std::memcpy(&outs[16 * g + i], r, 8);
            }
        }
    });
}
inline i32x2_emu ds_read_tr8_b64(const void* p) {
    return wave_op<const void*, i32x2_emu>(op_key(11), "ds_read_b64_tr_b8", p, [](const void* const* ins, i32x2_emu* outs, int n) {
        for (int g = 0; g < 4; ++g) {
            uint8_t F[128];
            for (int i = 0; i < 16; ++i) {
                const int l = 16 * g + i;
                if (l < n) std::memcpy(&F[8 * i], ins[l], 8);
                else std::memset(&F[8 * i], 0, 8);
            }
            for (int i = 0; i < 16; ++i) {
                uint8_t r[8];
                for (int j = 0; j < 8; ++j) r[j] = F[i + 16 * j];
                std::memcpy(&outs[16 * g + i], r, 8);
            }
        }
    });
}

// ---- atomics: one thread runs at a time, so plain accesses are atomic here -------------------------
template <class T, class U>
T atomic_fetch_add(T* p, U v) {
    const T o = *p;
    *p = (T)(o + (T)v);
    if (g_grp) ++g_grp->progress;  // (another fiber may be waiting for it)
    return o;
}

}  // namespace kvbemu

// ---- the names the kernels use ----------------------------------------------------------------------
#define threadIdx (::kvbemu::g_cur->tid)
#define blockIdx (::kvbemu::g_grp->bid)
#define gridDim (::kvbemu::g_grp->grid)
#define blockDim (::kvbemu::g_grp->block)

inline void __syncthreads() { ::kvbemu::syncthreads(); }
inline unsigned long long __ballot(int pred) { return ::kvbemu::ballot(pred != 0); }
template <class T>
T __shfl_xor(T v, int mask, int width = 64) {
    return ::kvbemu::shfl_xor(v, mask, width);
}
inline void kvbemu_wait_vmem() { ::kvbemu::wait_vmem(); }

typedef ::kvbemu::BufferRsrc __amdgpu_buffer_rsrc_t;
#define __builtin_amdgcn_make_buffer_rsrc(p, stride, num, flags) ::kvbemu::make_buffer_rsrc((p), (stride), (num), (flags))
#define __builtin_amdgcn_raw_buffer_load_b128 ::kvbemu::raw_buffer_load_b128
#define __builtin_amdgcn_raw_buffer_load_b32 ::kvbemu::raw_buffer_load_b32
#define __builtin_amdgcn_raw_buffer_store_b128 ::kvbemu::raw_buffer_store_b128
#define __builtin_amdgcn_raw_buffer_load_b64 ::kvbemu::raw_buffer_load_b64
#define __builtin_amdgcn_raw_buffer_store_b64 ::kvbemu::raw_buffer_store_b64
#define __builtin_amdgcn_update_dpp ::kvbemu::update_dpp
#define __builtin_amdgcn_mov_dpp ::kvbemu::mov_dpp
#define __builtin_amdgcn_readlane ::kvbemu::readlane
#define __builtin_amdgcn_readfirstlane ::kvbemu::readfirstlane
#define __builtin_amdgcn_ballot_w64 ::kvbemu::ballot
#define __builtin_amdgcn_wave_barrier ::kvbemu::wave_barrier
#define __builtin_amdgcn_mfma_f32_16x16x32_f16 ::kvbemu::mfma_f32_16x16x32_f16
#define __builtin_amdgcn_mfma_f32_16x16x4f32 ::kvbemu::mfma_f32_16x16x4f32
#define __builtin_amdgcn_mfma_i32_16x16x64_i8 ::kvbemu::mfma_i32_16x16x64_i8
#define __builtin_amdgcn_ds_read_tr16_b64_v4f16(p) ::kvbemu::ds_read_tr16_b64((const void*)(p))
#define __builtin_amdgcn_ds_read_tr8_b64_v2i32(p) ::kvbemu::ds_read_tr8_b64((const void*)(p))
#define __builtin_amdgcn_exp2f ::kvbemu::exp2_hw
#define __builtin_amdgcn_perm ::kvbemu::perm
// ordering hints with no CPU meaning: a fiber's own memory operations complete in program order
#define __builtin_amdgcn_fence(...) ((void)0)
#define __builtin_amdgcn_sched_barrier(...) ((void)0)
// s_sleep in a wait loop: the other fibers of the workgroup run meanwhile
#define __builtin_amdgcn_s_sleep(n) ::kvbemu::yield()
#define __hip_atomic_fetch_add(p, v, order, scope) ::kvbemu::atomic_fetch_add((p), (v))
// (volatile: a wait loop reads the value again after other fibers ran)
#define __hip_atomic_load(p, order, scope) (*(volatile std::remove_reference_t<decltype(*(p))>*)(p))
#define __hip_atomic_store(p, v, order, scope) ((void)(*(p) = (v)))
#define HIP_SYMBOL(x) (::kvbemu::symbol(&(x)))

// ---- the HIP runtime API the sources use ---------------------------------------------------------------
enum hipError_t {
    hipSuccess = 0,
    hipErrorInvalidValue = 1,
    hipErrorOutOfMemory = 2,
    hipErrorNoDevice = 100,
    hipErrorInvalidDevice = 101,
    hipErrorLaunchFailure = 719,
    hipErrorNotSupported = 801,
};
enum hipMemcpyKind { hipMemcpyHostToHost = 0, hipMemcpyHostToDevice, hipMemcpyDeviceToHost, hipMemcpyDeviceToDevice, hipMemcpyDefault };
enum hipDeviceAttribute_t {
    hipDeviceAttributeMultiprocessorCount = 1,
    hipDeviceAttributeMaxSharedMemoryPerMultiprocessor,
    hipDeviceAttributeMaxSharedMemoryPerBlock,
    hipDeviceAttributeClockRate,
    hipDeviceAttributeMemoryClockRate,
    hipDeviceAttributeMemoryBusWidth,
    hipDeviceAttributeL2CacheSize,
};
enum hipStreamCaptureMode { hipStreamCaptureModeGlobal = 0, hipStreamCaptureModeThreadLocal, hipStreamCaptureModeRelaxed };
constexpr unsigned hipStreamNonBlocking = 1;
constexpr unsigned hipEventDisableTiming = 2;

struct kvbemu_stream;
struct kvbemu_event;
struct kvbemu_graph;
typedef kvbemu_stream* hipStream_t;
typedef kvbemu_event* hipEvent_t;
typedef kvbemu_graph* hipGraph_t;
typedef kvbemu_graph* hipGraphExec_t;
typedef struct kvbemu_graph_node* hipGraphNode_t;

struct hipDeviceProp_t {
    char name[256];
    char gcnArchName[256];
    int multiProcessorCount;
    size_t totalGlobalMem;
    size_t sharedMemPerBlock;
};
struct hipFuncAttributes {
    size_t sharedSizeBytes;
    int numRegs;
    int maxThreadsPerBlock;
};

const char* hipGetErrorString(hipError_t e);
hipError_t hipGetLastError();
hipError_t hipGetDeviceCount(int* n);
hipError_t hipGetDevice(int* d);
hipError_t hipSetDevice(int d);
hipError_t hipGetDeviceProperties(hipDeviceProp_t* p, int d);
hipError_t hipDeviceGetAttribute(int* v, hipDeviceAttribute_t a, int d);
hipError_t hipRuntimeGetVersion(int* v);
hipError_t hipDriverGetVersion(int* v);
hipError_t hipDeviceGetPCIBusId(char* buf, int len, int d);
hipError_t hipMemGetInfo(size_t* free_bytes, size_t* total_bytes);
hipError_t hipDeviceSynchronize();
hipError_t hipMalloc(void** p, size_t bytes);
template <class T>
hipError_t hipMalloc(T** p, size_t bytes) {
    return hipMalloc(reinterpret_cast<void**>(p), bytes);
}
hipError_t hipFree(void* p);
hipError_t hipMemcpy(void* dst, const void* src, size_t bytes, hipMemcpyKind kind);
hipError_t hipMemcpyAsync(void* dst, const void* src, size_t bytes, hipMemcpyKind kind, hipStream_t s = nullptr);
hipError_t hipMemsetAsync(void* dst, int value, size_t bytes, hipStream_t s = nullptr);
hipError_t hipMemcpyFromSymbol(void* dst, const void* sym, size_t bytes, size_t offset = 0, hipMemcpyKind kind = hipMemcpyDeviceToHost);
hipError_t hipGetSymbolAddress(void** p, const void* sym);
hipError_t hipStreamCreateWithFlags(hipStream_t* s, unsigned flags);
hipError_t hipStreamCreate(hipStream_t* s);
hipError_t hipStreamDestroy(hipStream_t s);
hipError_t hipStreamSynchronize(hipStream_t s);
hipError_t hipStreamWaitEvent(hipStream_t s, hipEvent_t e, unsigned flags);
hipError_t hipEventCreate(hipEvent_t* e);
hipError_t hipEventCreateWithFlags(hipEvent_t* e, unsigned flags);
hipError_t hipEventDestroy(hipEvent_t e);
hipError_t hipEventRecord(hipEvent_t e, hipStream_t s = nullptr);
hipError_t hipEventSynchronize(hipEvent_t e);
hipError_t hipEventElapsedTime(float* ms, hipEvent_t a, hipEvent_t b);
hipError_t hipStreamBeginCapture(hipStream_t s, hipStreamCaptureMode mode);
hipError_t hipStreamEndCapture(hipStream_t s, hipGraph_t* g);
hipError_t hipGraphCreate(hipGraph_t* g, unsigned flags);
hipError_t hipGraphInstantiate(hipGraphExec_t* e, hipGraph_t g, hipGraphNode_t* err_node, char* log, size_t log_size);
hipError_t hipGraphLaunch(hipGraphExec_t e, hipStream_t s);
hipError_t hipGraphDestroy(hipGraph_t g);
hipError_t hipGraphExecDestroy(hipGraphExec_t e);
hipError_t hipFuncGetAttributes(hipFuncAttributes* a, const void* f);
hipError_t hipOccupancyMaxActiveBlocksPerMultiprocessor(int* n, const void* f, int threads, size_t dyn_lds);
template <class F>
hipError_t hipOccupancyMaxActiveBlocksPerMultiprocessor(int* n, F* f, int threads, size_t dyn_lds) {
    return hipOccupancyMaxActiveBlocksPerMultiprocessor(n, reinterpret_cast<const void*>(f), threads, dyn_lds);
}

namespace kvbemu {
// Runs grid x block threads of `body` (the kernel call with its arguments), workgroup by workgroup.
hipError_t launch(dim3 grid, dim3 block, const std::function<void()>& body);
void record(hipEvent_t e);
// Stream capture: while `s` captures, its work is appended to the graph being captured instead of
// running (`op` returns what the work would have returned); otherwise op runs now.
hipError_t enqueue(hipStream_t s, std::function<hipError_t()> op);
}  // namespace kvbemu

template <typename... KArgs, typename... Args>
void hipLaunchKernelGGL(void (*kernel)(KArgs...), dim3 grid, dim3 block, size_t /*lds*/, hipStream_t s,
                        Args... args) {
    (void)::kvbemu::enqueue(s, [=]() {  // (the arguments by value: a captured launch runs later)
        const std::function<void()> body = [&]() { kernel(args...); };
        return ::kvbemu::launch(grid, block, body);
    });
}
template <typename... KArgs, typename... Args>
void hipExtLaunchKernelGGL(void (*kernel)(KArgs...), dim3 grid, dim3 block, size_t /*lds*/, hipStream_t s,
                           hipEvent_t start, hipEvent_t stop, unsigned /*flags*/, Args... args) {
    (void)::kvbemu::enqueue(s, [=]() {
        if (start) ::kvbemu::record(start);
        const std::function<void()> body = [&]() { kernel(args...); };
        const hipError_t e = ::kvbemu::launch(grid, block, body);
        if (stop) ::kvbemu::record(stop);
        return e;
    });
}

extern "C" const char* kvbemu_last_error(void);
