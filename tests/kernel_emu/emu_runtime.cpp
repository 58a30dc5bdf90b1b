// The scheduler and runtime of the CPU emulation declared in kvb_emu.hpp (test infrastructure).
//
// Fibers switch with a small x86-64 context switch (callee-saved registers, MXCSR and the x87
// control word; no system call), so a cross-lane operation costs two switches per lane.
#include "kvb_emu.hpp"

#include <sys/mman.h>
#include <unistd.h>

// Under AddressSanitizer (make -C tests/kernel_emu asan): every plain load and store of the
// kernels is checked too, and the fiber switches are announced to it so that each fiber's stack is
// its own.
#if defined(__has_feature)
#if __has_feature(address_sanitizer)
#define KVBEMU_ASAN 1
#include <sanitizer/asan_interface.h>
#include <sanitizer/common_interface_defs.h>
#endif
#endif

#include <algorithm>
#include <chrono>
#include <cstdarg>
#include <cstdlib>
#include <map>
#include <string>
#include <vector>

// void kvbemu_switch(void** save_sp, void* load_sp): saves the running context's callee-saved
// state on its stack and its stack pointer in *save_sp, then resumes the context whose stack
// pointer is load_sp.
asm(R"(
    .text
    .globl kvbemu_switch
    .hidden kvbemu_switch
    .type kvbemu_switch,@function
kvbemu_switch:
    pushq %rbp
    pushq %rbx
    pushq %r12
    pushq %r13
    pushq %r14
    pushq %r15
    subq $8, %rsp
    stmxcsr (%rsp)
    fnstcw 4(%rsp)
    movq %rsp, (%rdi)
    movq %rsi, %rsp
    ldmxcsr (%rsp)
    fldcw 4(%rsp)
    addq $8, %rsp
    popq %r15
    popq %r14
    popq %r13
    popq %r12
    popq %rbx
    popq %rbp
    ret
    .size kvbemu_switch, .-kvbemu_switch
)");
extern "C" void kvbemu_switch(void** save_sp, void* load_sp);

namespace kvbemu {

Fiber* g_cur = nullptr;
Group* g_grp = nullptr;

namespace {

constexpr size_t kStackBytes = size_t(1) << 19;  // per fiber, below a guard page
constexpr int kMaxThreads = 1024;

void* g_sched_sp = nullptr;  // the scheduler's context while a fiber runs
bool g_failed = false;       // the running launch stopped with an error
std::string g_msg;           // its message
std::string g_last_msg;      // the last launch error's message (kvbemu_last_error)
hipError_t g_last_err = hipSuccess;
std::vector<Fiber> g_fibers;
// the seed of the wave order (KVBEMU_SEED, default 1)
const uint64_t g_seed = [] {
    const char* e = std::getenv("KVBEMU_SEED");
    const uint64_t s = e ? std::strtoull(e, nullptr, 0) : 1;
    return s ? s : 1;
}();
std::vector<char*> g_stacks;
std::map<uintptr_t, size_t> g_allocs;  // base -> bytes: hipMalloc and registered symbols
#ifdef KVBEMU_ASAN
const void* g_sched_bottom = nullptr;  // the scheduler's stack, as AddressSanitizer reports it
size_t g_sched_size = 0;
#endif

// The scheduler resumes fiber f, until it yields or ends.
void switch_to_fiber(Fiber& f) {
#ifdef KVBEMU_ASAN
    void* fake = nullptr;
    __sanitizer_start_switch_fiber(&fake, f.stack, kStackBytes);
#endif
    kvbemu_switch(&g_sched_sp, f.sp);
#ifdef KVBEMU_ASAN
    __sanitizer_finish_switch_fiber(fake, nullptr, nullptr);
#endif
}

// The running fiber hands control back to the scheduler; `ending`: it will never be resumed.
void switch_to_scheduler(bool ending) {
    Fiber* me = g_cur;
#ifdef KVBEMU_ASAN
    void* fake = nullptr;
    __sanitizer_start_switch_fiber(ending ? nullptr : &fake, g_sched_bottom, g_sched_size);
#else
    (void)ending;
#endif
    kvbemu_switch(&me->sp, g_sched_sp);
#ifdef KVBEMU_ASAN
    __sanitizer_finish_switch_fiber(fake, &g_sched_bottom, &g_sched_size);
#endif
}

char* new_stack() {
    const long page = sysconf(_SC_PAGESIZE);
    void* m = mmap(nullptr, kStackBytes + page, PROT_READ | PROT_WRITE, MAP_PRIVATE | MAP_ANONYMOUS, -1, 0);
    if (m == MAP_FAILED) {
        std::fprintf(stderr, "kvbemu: cannot map a fiber stack\n");
        std::abort();
    }
    mprotect(m, page, PROT_NONE);  // overflow faults instead of corrupting the next stack
    return static_cast<char*>(m) + page;
}

[[noreturn]] void fiber_main();

// A fresh context that starts in fiber_main: the frame kvbemu_switch pops (MXCSR and x87 control
// word, six registers, the return address), then a null return address for fiber_main so that it
// is entered with the stack alignment of a call.
void* init_context(char* stack) {
#ifdef KVBEMU_ASAN
    __asan_unpoison_memory_region(stack, kStackBytes);  // (frames of an abandoned fiber left poison)
#endif
    uintptr_t top = reinterpret_cast<uintptr_t>(stack + kStackBytes) & ~uintptr_t(15);
    uint64_t* sp = reinterpret_cast<uint64_t*>(top - 72);
    sp[0] = 0x1F80ull | (0x037Full << 32);  // MXCSR default, x87 control word default
    for (int i = 1; i <= 6; ++i) sp[i] = 0;
    sp[7] = reinterpret_cast<uint64_t>(&fiber_main);
    sp[8] = 0;
    return sp;
}

void fiber_main() {
#ifdef KVBEMU_ASAN
    __sanitizer_finish_switch_fiber(nullptr, &g_sched_bottom, &g_sched_size);
#endif
    (*g_grp->body)();
    Fiber* me = g_cur;
    Group& g = *g_grp;
    me->done = true;
    --g.live;
    ++g.progress;
    WaveSync& w = g.waves[me->wave];
    ++w.exited;
    if (w.arrived > 0)
        fail("a lane of wave %d exited while %d of its lanes wait at %s", me->wave, w.arrived, w.what ? w.what : "?");
    if (g.bar_arrived > 0 && g.bar_arrived == g.live) {
        g.bar_arrived = 0;
        ++g.bar_gen;
    }
    switch_to_scheduler(true);
    __builtin_unreachable();  // a finished fiber is never resumed
}

void set_error(hipError_t e, const std::string& msg) {
    g_last_err = e;
    g_last_msg = msg;
}

}  // namespace

void fail(const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    std::string where;
    if (g_grp && g_cur) {
        char loc[160];
        std::snprintf(loc, sizeof loc, " (workgroup %u,%u,%u, thread %d)", g_grp->bid.x, g_grp->bid.y, g_grp->bid.z,
                      g_cur->linear);
        where = loc;
    }
    g_msg = std::string(buf) + where;
    std::fprintf(stderr, "kvbemu: %s\n", g_msg.c_str());
    if (!g_cur || !g_sched_sp) std::abort();  // outside a launch: nothing to return to
    g_failed = true;
    switch_to_scheduler(true);
    __builtin_unreachable();  // the failed launch's fibers are abandoned, never resumed
}

void yield() { switch_to_scheduler(false); }

void syncthreads() {
    Group& g = *g_grp;
    const uint64_t my = g.bar_gen;
    ++g.progress;
    if (++g.bar_arrived == g.live) {
        g.bar_arrived = 0;
        ++g.bar_gen;
        return;
    }
    while (g.bar_gen == my) yield();
}

void wait_vmem() {}

void track(const void* p, size_t bytes) { g_allocs[reinterpret_cast<uintptr_t>(p)] = bytes; }
void untrack(const void* p) { g_allocs.erase(reinterpret_cast<uintptr_t>(p)); }

void check_access(const void* p, size_t bytes, const char* what) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    auto it = g_allocs.upper_bound(a);
    if (it != g_allocs.begin()) {
        --it;
        if (a >= it->first && a + bytes <= it->first + it->second) return;
        fail("%s of %zu bytes at offset %lld of a %zu-byte allocation", what, bytes, (long long)(a - it->first), it->second);
    }
    fail("%s of %zu bytes below every allocation", what, bytes);
}

hipError_t launch(dim3 grid, dim3 block, const std::function<void()>& body) {
    const long long threads = (long long)block.x * block.y * block.z;
    if (threads <= 0 || threads > kMaxThreads || grid.x == 0 || grid.y == 0 || grid.z == 0) {
        set_error(hipErrorInvalidValue, "launch with an empty grid or more than 1024 threads per workgroup");
        return hipErrorInvalidValue;
    }
    if (g_grp) {
        set_error(hipErrorInvalidValue, "a launch from inside a kernel");
        return hipErrorInvalidValue;
    }
    while ((long long)g_stacks.size() < threads) g_stacks.push_back(new_stack());
    g_fibers.assign((size_t)threads, Fiber{});
    const int nw = (int)((threads + 63) / 64);
    std::vector<WaveSync> waves((size_t)nw);
    std::vector<int> order((size_t)nw);
    for (int w = 0; w < nw; ++w) order[w] = w;
    Group grp;
    grp.grid = Idx{grid.x, grid.y, grid.z};
    grp.block = Idx{block.x, block.y, block.z};
    grp.threads = (int)threads;
    grp.waves = waves.data();
    grp.body = &body;
    g_failed = false;
    for (uint32_t bz = 0; bz < grid.z; ++bz)
        for (uint32_t by = 0; by < grid.y; ++by)
            for (uint32_t bx = 0; bx < grid.x; ++bx) {
                grp.bid = Idx{bx, by, bz};
                grp.live = (int)threads;
                grp.bar_gen = 0;
                grp.bar_arrived = 0;
                for (int w = 0; w < nw; ++w) {
                    waves[w].gen = 0;
                    waves[w].arrived = 0;
                    waves[w].exited = 0;
                    waves[w].lanes = (int)std::min<long long>(64, threads - 64LL * w);
                }
                for (int t = 0; t < (int)threads; ++t) {
                    Fiber& f = g_fibers[t];
                    f.stack = g_stacks[t];
                    f.tid = Idx{(uint32_t)(t % block.x), (uint32_t)((t / block.x) % block.y), (uint32_t)(t / (block.x * block.y))};
                    f.linear = t;
                    f.lane = t & 63;
                    f.wave = t >> 6;
                    f.done = false;
                    f.sp = init_context(f.stack);
                }
                g_grp = &grp;
                // Each pass over the workgroup takes its waves in a fresh order (xorshift from a fixed
                // seed, KVBEMU_SEED to change it), the lanes of a wave in order: waves then meet only
                // where the kernel makes them (barriers, counters in LDS), not because a lower wave
                // always runs first.
                uint64_t rng = g_seed ^ (0x9E3779B97F4A7C15ull * (1 + bx + grid.x * (by + (uint64_t)grid.y * bz)));
                while (grp.live > 0 && !g_failed) {
                    const uint64_t before = grp.progress;
                    for (int i = nw - 1; i > 0; --i) {
                        rng ^= rng << 13;
                        rng ^= rng >> 7;
                        rng ^= rng << 17;
                        std::swap(order[i], order[rng % (uint64_t)(i + 1)]);
                    }
                    for (int wi = 0; wi < nw && !g_failed; ++wi)
                        for (int t = 64 * order[wi]; t < std::min(64 * order[wi] + 64, (int)threads); ++t) {
                            Fiber& f = g_fibers[t];
                            if (f.done) continue;
                            g_cur = &f;
                            switch_to_fiber(f);
                            if (g_failed) break;
                        }
                    if (!g_failed && grp.live > 0 && grp.progress == before) {
                        char buf[200];
                        std::snprintf(buf, sizeof buf,
                                      "deadlock in workgroup %u,%u,%u: %d threads wait and none can go on", bx, by, bz,
                                      grp.live);
                        g_msg = buf;
                        std::fprintf(stderr, "kvbemu: %s\n", buf);
                        g_failed = true;
                    }
                }
                g_cur = nullptr;
                g_grp = nullptr;
                if (g_failed) {
                    set_error(hipErrorLaunchFailure, g_msg);
                    return hipErrorLaunchFailure;
                }
            }
    return hipSuccess;
}

void record(hipEvent_t e);

}  // namespace kvbemu

// ---- runtime API -----------------------------------------------------------------------------------------
struct kvbemu_stream {
    unsigned flags = 0;
    std::vector<std::function<hipError_t()>>* capture = nullptr;  // the graph being captured, if any
};
struct kvbemu_event {
    double t = 0.0;
};
struct kvbemu_graph {
    std::vector<std::function<hipError_t()>> ops;  // captured work, in stream order
};

namespace kvbemu {
hipError_t enqueue(hipStream_t s, std::function<hipError_t()> op) {
    if (s && s->capture) {
        s->capture->push_back(std::move(op));
        return hipSuccess;
    }
    const hipError_t e = op();
    if (e != hipSuccess && g_last_err == hipSuccess) g_last_err = e;
    return e;
}
void record(hipEvent_t e) {
    e->t = std::chrono::duration<double>(std::chrono::steady_clock::now().time_since_epoch()).count();
}
}  // namespace kvbemu

extern "C" const char* kvbemu_last_error(void) { return kvbemu::g_last_msg.c_str(); }

const char* hipGetErrorString(hipError_t e) {
    switch (e) {
        case hipSuccess: return "no error";
        case hipErrorInvalidValue: return "invalid argument";
        case hipErrorOutOfMemory: return "out of memory";
        case hipErrorNoDevice: return "no device";
        case hipErrorInvalidDevice: return "invalid device";
        case hipErrorLaunchFailure: return "emulated launch failed (see kvbemu_last_error)";
        case hipErrorNotSupported: return "not supported by the CPU emulation";
    }
    return "unknown error";
}
hipError_t hipGetLastError() {
    const hipError_t e = kvbemu::g_last_err;
    kvbemu::g_last_err = hipSuccess;
    return e;
}
hipError_t hipGetDeviceCount(int* n) {
    *n = 1;
    return hipSuccess;
}
hipError_t hipGetDevice(int* d) {
    *d = 0;
    return hipSuccess;
}
hipError_t hipSetDevice(int d) { return d == 0 ? hipSuccess : hipErrorInvalidDevice; }
hipError_t hipGetDeviceProperties(hipDeviceProp_t* p, int d) {
    if (d != 0) return hipErrorInvalidDevice;
    std::memset(p, 0, sizeof *p);
    std::snprintf(p->name, sizeof p->name, "CPU emulation of gfx950 (tests only)");
    std::snprintf(p->gcnArchName, sizeof p->gcnArchName, "gfx950-emulated");
    p->multiProcessorCount = 256;  // MI355X's count, so the host picks the launch shapes it picks there
    p->totalGlobalMem = size_t(1) << 34;
    p->sharedMemPerBlock = 160 * 1024;
    return hipSuccess;
}
hipError_t hipDeviceGetAttribute(int* v, hipDeviceAttribute_t a, int d) {
    if (d != 0) return hipErrorInvalidDevice;
    switch (a) {
        case hipDeviceAttributeMultiprocessorCount: *v = 256; return hipSuccess;
        case hipDeviceAttributeMaxSharedMemoryPerMultiprocessor: *v = 160 * 1024; return hipSuccess;
        case hipDeviceAttributeMaxSharedMemoryPerBlock: *v = 64 * 1024; return hipSuccess;
        case hipDeviceAttributeClockRate: *v = 0; return hipSuccess;  // (no clock: not a GPU)
        case hipDeviceAttributeMemoryClockRate: *v = 0; return hipSuccess;
        case hipDeviceAttributeMemoryBusWidth: *v = 0; return hipSuccess;
        case hipDeviceAttributeL2CacheSize: *v = 0; return hipSuccess;
    }
    return hipErrorInvalidValue;
}
// The emulation's own version numbers: 0 stands for "no HIP runtime".
hipError_t hipRuntimeGetVersion(int* v) {
    *v = 0;
    return hipSuccess;
}
hipError_t hipDriverGetVersion(int* v) {
    *v = 0;
    return hipSuccess;
}
hipError_t hipDeviceGetPCIBusId(char* buf, int len, int d) {
    if (d != 0) return hipErrorInvalidDevice;
    std::snprintf(buf, size_t(len), "emulated");
    return hipSuccess;
}
hipError_t hipMemGetInfo(size_t* free_bytes, size_t* total_bytes) {
    *free_bytes = *total_bytes = size_t(1) << 34;
    return hipSuccess;
}
hipError_t hipDeviceSynchronize() { return hipSuccess; }
hipError_t hipMalloc(void** p, size_t bytes) {
    void* m = std::aligned_alloc(256, (std::max<size_t>(bytes, 1) + 255) & ~size_t(255));
    if (!m) return hipErrorOutOfMemory;
    kvbemu::track(m, bytes);
    *p = m;
    return hipSuccess;
}
hipError_t hipFree(void* p) {
    if (!p) return hipSuccess;
    kvbemu::untrack(p);
    std::free(p);
    return hipSuccess;
}
hipError_t hipMemcpy(void* dst, const void* src, size_t bytes, hipMemcpyKind) {
    if (bytes) std::memmove(dst, src, bytes);
    return hipSuccess;
}
hipError_t hipMemcpyAsync(void* dst, const void* src, size_t bytes, hipMemcpyKind k, hipStream_t s) {
    return kvbemu::enqueue(s, [=]() { return hipMemcpy(dst, src, bytes, k); });
}
hipError_t hipMemsetAsync(void* dst, int value, size_t bytes, hipStream_t s) {
    return kvbemu::enqueue(s, [=]() {
        if (bytes) std::memset(dst, value, bytes);
        return hipSuccess;
    });
}
hipError_t hipMemcpyFromSymbol(void* dst, const void* sym, size_t bytes, size_t offset, hipMemcpyKind) {
    std::memcpy(dst, static_cast<const char*>(sym) + offset, bytes);
    return hipSuccess;
}
hipError_t hipGetSymbolAddress(void** p, const void* sym) {
    *p = const_cast<void*>(sym);
    return hipSuccess;
}
hipError_t hipStreamCreateWithFlags(hipStream_t* s, unsigned flags) {
    *s = new kvbemu_stream{flags};
    return hipSuccess;
}
hipError_t hipStreamCreate(hipStream_t* s) { return hipStreamCreateWithFlags(s, 0); }
hipError_t hipStreamDestroy(hipStream_t s) {
    delete s;
    return hipSuccess;
}
// Every operation completes when it is issued, so every wait is already satisfied.
hipError_t hipStreamSynchronize(hipStream_t) { return hipSuccess; }
hipError_t hipStreamWaitEvent(hipStream_t, hipEvent_t, unsigned) { return hipSuccess; }
hipError_t hipEventCreate(hipEvent_t* e) {
    *e = new kvbemu_event{};
    return hipSuccess;
}
hipError_t hipEventCreateWithFlags(hipEvent_t* e, unsigned) { return hipEventCreate(e); }
hipError_t hipEventDestroy(hipEvent_t e) {
    delete e;
    return hipSuccess;
}
hipError_t hipEventRecord(hipEvent_t e, hipStream_t s) {
    return kvbemu::enqueue(s, [=]() {
        kvbemu::record(e);
        return hipSuccess;
    });
}
hipError_t hipEventSynchronize(hipEvent_t) { return hipSuccess; }
hipError_t hipEventElapsedTime(float* ms, hipEvent_t a, hipEvent_t b) {
    *ms = (float)((b->t - a->t) * 1e3);
    return hipSuccess;
}
// Graphs: a capture records the stream's launches, fills, copies and event records as they are
// issued; a launch of the instantiated graph runs them in that order.
hipError_t hipStreamBeginCapture(hipStream_t s, hipStreamCaptureMode) {
    if (!s || s->capture) return hipErrorInvalidValue;
    s->capture = new std::vector<std::function<hipError_t()>>;
    return hipSuccess;
}
hipError_t hipStreamEndCapture(hipStream_t s, hipGraph_t* g) {
    *g = nullptr;
    if (!s || !s->capture) return hipErrorInvalidValue;
    *g = new kvbemu_graph{std::move(*s->capture)};
    delete s->capture;
    s->capture = nullptr;
    return hipSuccess;
}
hipError_t hipGraphCreate(hipGraph_t* g, unsigned) {
    *g = new kvbemu_graph{};
    return hipSuccess;
}
hipError_t hipGraphInstantiate(hipGraphExec_t* e, hipGraph_t g, hipGraphNode_t*, char*, size_t) {
    if (!g) return hipErrorInvalidValue;
    *e = new kvbemu_graph{g->ops};
    return hipSuccess;
}
hipError_t hipGraphLaunch(hipGraphExec_t e, hipStream_t s) {
    if (!e) return hipErrorInvalidValue;
    const kvbemu_graph* graph = e;
    return kvbemu::enqueue(s, [graph]() {
        for (const auto& op : graph->ops)
            if (const hipError_t err = op(); err != hipSuccess) return err;
        return hipSuccess;
    });
}
hipError_t hipGraphDestroy(hipGraph_t g) {
    delete g;
    return hipSuccess;
}
hipError_t hipGraphExecDestroy(hipGraphExec_t e) {
    delete e;
    return hipSuccess;
}
hipError_t hipFuncGetAttributes(hipFuncAttributes* a, const void*) {
    std::memset(a, 0, sizeof *a);
    a->maxThreadsPerBlock = 1024;
    return hipSuccess;
}
hipError_t hipOccupancyMaxActiveBlocksPerMultiprocessor(int* n, const void*, int, size_t) {
    *n = 1;
    return hipSuccess;
}
