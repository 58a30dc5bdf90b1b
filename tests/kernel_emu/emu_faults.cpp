// Faults the CPU emulation (kvb_emu.hpp) must stop a launch for: a buffer access outside every
// allocation, lanes of a wave at different cross-lane operations, a wave split between a cross-lane
// operation and a barrier, and a cross-lane operation after some of the wave's lanes exited; and the
// buffer range check that must not fault. CPU only, never built for a GPU: run by
// tests/test_kernel_emu.py. Prints one line per check and exits 0 when all pass.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <string>

namespace {

int g_failures = 0;
void check(bool ok, const char* what) {
    std::printf("%s: %s\n", ok ? "ok" : "FAIL", what);
    if (!ok) ++g_failures;
}

// ---- faults the emulation must report
__global__ void oob_kernel(const float* p, float* out) {
    // a resource over 64 floats, read one float past it on lane 63: in range of the resource,
    // outside the 64-float allocation
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(p), (short)0, 65 * 4, 0x00020000);
    out[threadIdx.x] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, (threadIdx.x + 1) * 4, 0, 0));
}
__global__ void clamp_kernel(const float* p, float* out) {
    // the same read through a resource sized to the allocation: lane 63's read is out of the
    // resource's range and returns 0, without touching memory
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(p), (short)0, 64 * 4, 0x00020000);
    out[threadIdx.x] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, (threadIdx.x + 1) * 4, 0, 0));
}
__global__ void divergent_kernel(int* out) {
    if (threadIdx.x < 32) out[threadIdx.x] = __shfl_xor((int)threadIdx.x, 1);
    else out[threadIdx.x] = (int)__ballot(1);
}
__global__ void deadlock_kernel(int* out) {
    if (threadIdx.x == 0) out[0] = __builtin_amdgcn_readfirstlane(1);  // the wave's other lanes never come
    __syncthreads();
}
__global__ void exit_kernel(int* out) {
    if (threadIdx.x >= 32) return;
    out[threadIdx.x] = __shfl_xor((int)threadIdx.x, 1);
}

template <class T>
T* dev(size_t n) {
    void* p = nullptr;
    hipMalloc(&p, n * sizeof(T));
    std::memset(p, 0, n * sizeof(T));
    return static_cast<T*>(p);
}

bool launch_fails(void (*k)(int*), const char* expect) {
    int* out = dev<int>(64);
    hipLaunchKernelGGL(k, dim3(1), dim3(64), 0, nullptr, out);
    const hipError_t e = hipGetLastError();
    const std::string msg = kvbemu_last_error();
    hipFree(out);
    return e == hipErrorLaunchFailure && msg.find(expect) != std::string::npos;
}

}  // namespace

int main() {
    {
        float* p = dev<float>(64);
        float* out = dev<float>(64);
        for (int i = 0; i < 64; ++i) p[i] = (float)i;
        hipLaunchKernelGGL(clamp_kernel, dim3(1), dim3(64), 0, nullptr, p, out);
        bool ok = hipGetLastError() == hipSuccess;
        for (int l = 0; l < 64; ++l) ok = ok && out[l] == (l < 63 ? (float)(l + 1) : 0.0f);
        check(ok, "a buffer load past num_records reads 0");
        hipLaunchKernelGGL(oob_kernel, dim3(1), dim3(64), 0, nullptr, p, out);
        const std::string msg = kvbemu_last_error();
        check(hipGetLastError() == hipErrorLaunchFailure && msg.find("buffer load") != std::string::npos,
              "a buffer load outside every allocation stops the launch");
    }
    check(launch_fails(divergent_kernel, "different cross-lane operations"),
          "lanes of a wave at different cross-lane operations stop the launch");
    check(launch_fails(deadlock_kernel, "deadlock"), "a wave split between a cross-lane operation and a barrier stops the launch");
    check(launch_fails(exit_kernel, "exited"), "a cross-lane operation after some lanes exited stops the launch");
    std::printf("%s: %d failure(s)\n", g_failures ? "FAILED" : "PASSED", g_failures);
    return g_failures ? 1 : 0;
}
