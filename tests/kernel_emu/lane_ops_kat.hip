// Known answers for the cross-lane operations the kernels use: the MFMA operand layouts, the
// transposing LDS reads, DPP, lane shuffles, readlane and ballot, each checked against the
// operation's documented definition computed on the host. The same source builds two ways:
// with hipcc for gfx950 (tests/test_lane_ops_gpu.py runs it on the MI355X), and against the CPU
// emulation (tests/kernel_emu/kvb_emu.hpp, run by tests/test_kernel_emu.py). Passing on both pins
// the emulation's semantics of these operations to the hardware's. Every access is in bounds.
// Prints one line per check and exits 0 when all pass.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <vector>

namespace {

int g_failures = 0;
void check(bool ok, const char* what) {
    std::printf("%s: %s\n", ok ? "ok" : "FAIL", what);
    if (!ok) ++g_failures;
}

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x2 __attribute__((ext_vector_type(2)));
typedef __fp16 fp16x4 __attribute__((__vector_size__(8)));
// the transposing reads take LDS (address space 3) pointers
typedef __attribute__((address_space(3))) fp16x4 lds_fp16x4;
typedef __attribute__((address_space(3))) i32x2 lds_i32x2;

// ---- v_mfma_f32_16x16x32_f16: A (16 x 32) and B (32 x 16) given as matrices, placed into the lanes
// as CDNA lays them out; the result gathered back from the lanes' accumulators.
__global__ void mfma_f16_kernel(const float* A, const float* B, float* D) {
    const int l = threadIdx.x;
    half8 a, b;
    for (int e = 0; e < 8; ++e) {
        a[e] = (_Float16)A[(l % 16) * 32 + 8 * (l / 16) + e];
        b[e] = (_Float16)B[(8 * (l / 16) + e) * 16 + l % 16];
    }
    f32x4 c = {1.0f, 1.0f, 1.0f, 1.0f};
    const f32x4 d = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
    for (int i = 0; i < 4; ++i) D[(4 * (l / 16) + i) * 16 + l % 16] = d[i];
}

__global__ void mfma_i8_kernel(const int8_t* A, const int8_t* B, int* D) {
    const int l = threadIdx.x;
    int8_t a[16], b[16];
    for (int e = 0; e < 16; ++e) {
        a[e] = A[(l % 16) * 64 + 16 * (l / 16) + e];
        b[e] = B[(16 * (l / 16) + e) * 16 + l % 16];
    }
    i32x4 av, bv;
    __builtin_memcpy(&av, a, 16);
    __builtin_memcpy(&bv, b, 16);
    const i32x4 d = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, bv, (i32x4){0, 0, 0, 0}, 0, 0, 0);
    for (int i = 0; i < 4; ++i) D[(4 * (l / 16) + i) * 16 + l % 16] = d[i];
}

__global__ void mfma_f32_kernel(const float* A, const float* B, float* D) {
    const int l = threadIdx.x;
    const f32x4 d = __builtin_amdgcn_mfma_f32_16x16x4f32(A[(l % 16) * 4 + l / 16], B[(l / 16) * 16 + l % 16],
                                                          (f32x4){0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
    for (int i = 0; i < 4; ++i) D[(4 * (l / 16) + i) * 16 + l % 16] = d[i];
}

// ---- ds_read_b64_tr_b16: a 16 x 64 matrix of halves in LDS, row r at r * 64; lane l of each
// 16-lane group addresses row l / 4 (+ 4 group), columns 4 (l % 4)..; lane i must receive column
// i of the group's 4 rows.
__global__ void tr16_kernel(uint16_t* out) {
    __shared__ uint16_t lds[16 * 64];
    const int l = threadIdx.x;
    for (int i = l; i < 16 * 64; i += 64) lds[i] = (uint16_t)i;
    __syncthreads();
    const int g = l / 16, i = l % 16;
    const fp16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4f16((lds_fp16x4*)&lds[(4 * g + i / 4) * 64 + 4 * (i % 4)]);
    __builtin_memcpy(&out[4 * l], &v, 8);
}
__global__ void tr8_kernel(uint8_t* out) {
    __shared__ uint8_t lds[32 * 16];
    const int l = threadIdx.x;
    for (int i = l; i < 32 * 16; i += 64) lds[i] = (uint8_t)(i * 7 + 3);
    __syncthreads();
    const int g = l / 16, i = l % 16;
    // lane i of group g addresses row 8 g + i / 2, columns 8 (i % 2)..
    const i32x2 v = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_i32x2*)&lds[(8 * g + i / 2) * 16 + 8 * (i % 2)]);
    __builtin_memcpy(&out[8 * l], &v, 8);
}

// ---- DPP: quad_perm [1,0,3,2], row_shr:1 (bound_ctrl off: lane 0 of a row keeps old), the
// row_bcast:15 / row_bcast:31 steps of a wave prefix sum, and quad_perm [2,3,0,1], row_half_mirror
// and row_mirror (the steps of a max over 16 lanes)
__global__ void dpp_kernel(int* out) {
    const int l = threadIdx.x;
    out[l] = __builtin_amdgcn_update_dpp(-1, l, 0xB1, 0xF, 0xF, false);
    out[64 + l] = __builtin_amdgcn_update_dpp(-1, l, 0x111, 0xF, 0xF, false);
    int x = 1;
    x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xF, 0xF, false);
    x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xF, 0xF, false);
    x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xF, 0xF, false);
    x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xF, 0xF, false);
    x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xA, 0xF, false);
    x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xC, 0xF, false);
    out[128 + l] = x;
    out[192 + l] = __shfl_xor(l, 5);
    out[256 + l] = __builtin_amdgcn_readlane(l * 3, 17);
    out[320 + l] = (int)(__ballot(l % 3 == 0) >> (l % 32) & 1);
    out[384 + l] = __builtin_amdgcn_mov_dpp(7 * l + 1, 0xB1, 0xF, 0xF, true);  // no old value
    out[448 + l] = __builtin_amdgcn_update_dpp(-1, l, 0x4E, 0xF, 0xF, false);
    out[512 + l] = __builtin_amdgcn_update_dpp(-1, l, 0x141, 0xF, 0xF, false);
    out[576 + l] = __builtin_amdgcn_update_dpp(-1, l, 0x140, 0xF, 0xF, false);
}

template <class T>
struct Dev {  // a device buffer with a host copy
    std::vector<T> h;
    T* d = nullptr;
    explicit Dev(size_t n) : h(n) {
        if (hipMalloc(reinterpret_cast<void**>(&d), n * sizeof(T)) != hipSuccess) std::abort();
        (void)hipMemcpy(d, h.data(), n * sizeof(T), hipMemcpyHostToDevice);
    }
    ~Dev() { (void)hipFree(d); }
    void up() { (void)hipMemcpy(d, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice); }
    void down() { (void)hipMemcpy(h.data(), d, h.size() * sizeof(T), hipMemcpyDeviceToHost); }
};

bool launched() { return hipDeviceSynchronize() == hipSuccess && hipGetLastError() == hipSuccess; }

}  // namespace

int main() {
    {  // small integers: exact in fp16 and in the fp32 sums
        Dev<float> A(16 * 32), B(32 * 16), D(256);
        for (int i = 0; i < 16 * 32; ++i) A.h[i] = (float)((i * 7) % 11 - 5);
        for (int i = 0; i < 32 * 16; ++i) B.h[i] = (float)((i * 5) % 13 - 6);
        A.up();
        B.up();
        hipLaunchKernelGGL(mfma_f16_kernel, dim3(1), dim3(64), 0, 0, A.d, B.d, D.d);
        bool ok = launched();
        D.down();
        for (int r = 0; r < 16; ++r)
            for (int c = 0; c < 16; ++c) {
                float s = 1.0f;
                for (int k = 0; k < 32; ++k) s += A.h[r * 32 + k] * B.h[k * 16 + c];
                ok = ok && D.h[r * 16 + c] == s;
            }
        check(ok, "v_mfma_f32_16x16x32_f16 = 1 + A B with CDNA's operand layout");
    }
    {
        Dev<int8_t> A(16 * 64), B(64 * 16);
        Dev<int> D(256);
        for (int i = 0; i < 16 * 64; ++i) A.h[i] = (int8_t)((i * 37) % 255 - 127);
        for (int i = 0; i < 64 * 16; ++i) B.h[i] = (int8_t)((i * 91) % 255 - 127);
        A.up();
        B.up();
        hipLaunchKernelGGL(mfma_i8_kernel, dim3(1), dim3(64), 0, 0, A.d, B.d, D.d);
        bool ok = launched();
        D.down();
        for (int r = 0; r < 16; ++r)
            for (int c = 0; c < 16; ++c) {
                int s = 0;
                for (int k = 0; k < 64; ++k) s += (int)A.h[r * 64 + k] * (int)B.h[k * 16 + c];
                ok = ok && D.h[r * 16 + c] == s;
            }
        check(ok, "v_mfma_i32_16x16x64_i8 = A B, exact, with CDNA's operand layout");
    }
    {
        Dev<float> A(64), B(64), D(256);
        for (int i = 0; i < 64; ++i) {
            A.h[i] = (float)(i % 9 - 4);
            B.h[i] = (float)(i % 7 - 3);
        }
        A.up();
        B.up();
        hipLaunchKernelGGL(mfma_f32_kernel, dim3(1), dim3(64), 0, 0, A.d, B.d, D.d);
        bool ok = launched();
        D.down();
        for (int r = 0; r < 16; ++r)
            for (int c = 0; c < 16; ++c) {
                float s = 0.0f;
                for (int k = 0; k < 4; ++k) s += A.h[r * 4 + k] * B.h[k * 16 + c];
                ok = ok && D.h[r * 16 + c] == s;
            }
        check(ok, "v_mfma_f32_16x16x4_f32 = A B with CDNA's operand layout");
    }
    {
        Dev<uint16_t> out(256);
        hipLaunchKernelGGL(tr16_kernel, dim3(1), dim3(64), 0, 0, out.d);
        bool ok = launched();
        out.down();
        for (int l = 0; l < 64; ++l)
            for (int j = 0; j < 4; ++j) ok = ok && out.h[4 * l + j] == (uint16_t)((4 * (l / 16) + j) * 64 + l % 16);
        check(ok, "ds_read_b64_tr_b16: lane i of a 16-lane group gets column i of the 4 rows its group addresses");
    }
    {
        Dev<uint8_t> out(512);
        hipLaunchKernelGGL(tr8_kernel, dim3(1), dim3(64), 0, 0, out.d);
        bool ok = launched();
        out.down();
        for (int l = 0; l < 64; ++l)
            for (int j = 0; j < 8; ++j) ok = ok && out.h[8 * l + j] == (uint8_t)(((8 * (l / 16) + j) * 16 + l % 16) * 7 + 3);
        check(ok, "ds_read_b64_tr_b8: lane i of a 16-lane group gets column i of the 8 rows its group addresses");
    }
    {
        Dev<int> out(640);
        hipLaunchKernelGGL(dpp_kernel, dim3(1), dim3(64), 0, 0, out.d);
        bool ok = launched();
        out.down();
        bool shr = ok, scan = ok, xr = ok, rl = ok, bal = ok, mov = ok, q2 = ok, hm = ok, rm = ok;
        for (int l = 0; l < 64; ++l) {
            ok = ok && out.h[l] == (l ^ 1);
            shr = shr && out.h[64 + l] == (l % 16 == 0 ? -1 : l - 1);
            scan = scan && out.h[128 + l] == l + 1;
            xr = xr && out.h[192 + l] == (l ^ 5);
            rl = rl && out.h[256 + l] == 51;
            bal = bal && out.h[320 + l] == (int)(((l % 32) % 3 == 0));
            mov = mov && out.h[384 + l] == 7 * (l ^ 1) + 1;
            q2 = q2 && out.h[448 + l] == (l ^ 2);
            hm = hm && out.h[512 + l] == ((l & ~7) | (7 - (l & 7)));
            rm = rm && out.h[576 + l] == ((l & ~15) | (15 - (l & 15)));
        }
        check(ok, "DPP quad_perm [1,0,3,2]");
        check(shr, "DPP row_shr:1 keeps the old value in each row's first lane");
        check(scan, "DPP row_shr 1/2/4/8 + row_bcast:15/31 give the wave's inclusive prefix sum");
        check(xr, "__shfl_xor");
        check(rl, "v_readlane");
        check(bal, "ballot");
        check(mov, "mov_dpp quad_perm [1,0,3,2] (bound_ctrl, no old value)");
        check(q2, "DPP quad_perm [2,3,0,1]");
        check(hm, "DPP row_half_mirror");
        check(rm, "DPP row_mirror");
    }
    std::printf("%s: %d failure(s)\n", g_failures ? "FAILED" : "PASSED", g_failures);
    return g_failures ? 1 : 0;
}
