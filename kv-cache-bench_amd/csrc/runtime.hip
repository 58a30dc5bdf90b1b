// The C ABI of libkvb_hip.so (include/kvb_hip.h): argument checks, device state, workspaces,
// launches and hipEvent timing. Plays the part of the reference's Objective-C++ host layer
// (src/metal_attn.mm): the same refusals before any GPU work, a grow-only split-K workspace, GPU
// time per submitted step and a pipelined (queue now, collect times later) mode.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>
#include <utility>
#include <vector>

#include "kvb_hip.h"
#include "kvb_kernels.hpp"

namespace {

thread_local std::string g_err;

int fail(int code, std::string msg) {
    g_err = std::move(msg);
    return code;
}

#define KVB_HIP(expr)                                                                         \
    do {                                                                                      \
        const hipError_t e_ = (expr);                                                         \
        if (e_ != hipSuccess) return fail(KVB_ERUNTIME, std::string(#expr) + ": " + hipGetErrorString(e_)); \
    } while (0)

struct Runtime {
    bool ready = false;
    int device = -1;
    hipStream_t own = nullptr;
    hipStream_t stream = nullptr;
    void* ws = nullptr;             // split-K workspace (grow-only)
    size_t ws_bytes = 0;
    void* counters = nullptr;       // fused-merge arrival counters (grow-only, kept at 0 between steps)
    size_t counters_bytes = 0;
    void* scores = nullptr;         // naive scores (grow-only)
    size_t scores_bytes = 0;
    void* flush_buf = nullptr;      // cache-flush source
    hipEvent_t switch_ev = nullptr; // orders a new stream after the old one (kvb_set_stream)
    int cus = 0;                    // compute units: the read probe runs one workgroup per CU
    int pair_mode = KVB_PAIR_AUTO;  // kvb_set_pair_mode
    int merge_mode = KVB_MERGE_AUTO;  // kvb_set_merge_mode
    float* sink = nullptr;          // read-probe sink
    bool pipelined = false;
    std::vector<std::pair<hipEvent_t, hipEvent_t>> timed;
    std::vector<hipEvent_t> spare;
};
Runtime g;

constexpr size_t kFlushBytes = size_t(1) << 30;
constexpr size_t kSinkFloats = kvbk::kReadBwSink;

// ---- the static scratch of kvb_run_paged_noalloc -----------------------------------------------
// The fused-merge arrival counters (KVB_NOALLOC_MAX_GROUPS ints), then the split-K workspace
// (KVB_NOALLOC_WORKSPACE_BYTES). Every GPU the library runs on holds one copy until the process
// ends. In host code `scratch` is only a handle for hipGetSymbolAddress: the device address is
// g.scratch_dev, resolved once per device at set-up (ensure_device), and is what kernels are given.
constexpr size_t kScratchCounterBytes = size_t(KVB_NOALLOC_MAX_GROUPS) * sizeof(int);
constexpr size_t kScratchBytes = kScratchCounterBytes + KVB_NOALLOC_WORKSPACE_BYTES;
static_assert(kScratchCounterBytes % 256 == 0, "the workspace starts 256-byte aligned");
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

struct ScratchOf {
    int device;
    void* dev;  // the device address of `scratch` on `device`
};
std::vector<ScratchOf> g_scratch;
std::string g_scratch_err;  // why the set-up could not resolve it (reported by kvb_run_paged_noalloc)

// Resolves `scratch` on the current device (once per device) and zeroes its counters, which every
// fused launch then leaves at 0 again. Runs at set-up, outside any caller's work: the fill and the
// wait are on the library's own stream. Returns the reason for a failure ("" on success).
std::string resolve_scratch(int device) {
    for (const ScratchOf& s : g_scratch)
        if (s.device == device) return "";
    void* ptr = nullptr;
    if (hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)); e != hipSuccess)
        return std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e);
    if (!ptr) return "hipGetSymbolAddress(scratch) returned a null address";
    if (hipError_t e = kvbk::launch_fill(ptr, kScratchCounterBytes / 16, 0u, g.own); e != hipSuccess)
        return std::string("scratch counter fill: ") + hipGetErrorString(e);
    if (hipError_t e = hipStreamSynchronize(g.own); e != hipSuccess)
        return std::string("scratch counter fill: ") + hipGetErrorString(e);
    g_scratch.push_back({device, ptr});
    return "";
}

void* scratch_of(int device) {
    for (const ScratchOf& s : g_scratch)
        if (s.device == device) return s.dev;
    return nullptr;
}

int ensure_device() {
    if (g.ready) return KVB_OK;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return fail(KVB_ENODEV, "no HIP device");
    KVB_HIP(hipGetDevice(&g.device));
    KVB_HIP(hipDeviceGetAttribute(&g.cus, hipDeviceAttributeMultiprocessorCount, g.device));
    KVB_HIP(hipStreamCreateWithFlags(&g.own, hipStreamNonBlocking));
    if (!g.stream) g.stream = g.own;
    // (a failure here concerns kvb_run_paged_noalloc alone, which reports it)
    g_scratch_err = resolve_scratch(g.device);
    g.ready = true;
    return KVB_OK;
}

int get_event(hipEvent_t* e) {
    if (!g.spare.empty()) {
        *e = g.spare.back();
        g.spare.pop_back();
        return KVB_OK;
    }
    KVB_HIP(hipEventCreate(e));
    return KVB_OK;
}

// Grows a library-owned buffer; waits for queued work first, since it may still use the old one.
int grow(void** buf, size_t* have, size_t need) {
    if (*have >= need && *buf) return KVB_OK;
    KVB_HIP(hipStreamSynchronize(g.stream));
    if (*buf) KVB_HIP(hipFree(*buf));
    *buf = nullptr;
    *have = 0;
    KVB_HIP(hipMalloc(buf, std::max<size_t>(need, 256)));
    *have = std::max<size_t>(need, 256);
    return KVB_OK;
}

// Ends a timed submission: queue the pair (pipelined) or wait and report its GPU time.
int finish(hipEvent_t e0, hipEvent_t e1, double* ms) {
    if (g.pipelined) {
        g.timed.emplace_back(e0, e1);
        if (ms) *ms = 0.0;
        return KVB_OK;
    }
    KVB_HIP(hipEventSynchronize(e1));
    float f = 0.0f;
    KVB_HIP(hipEventElapsedTime(&f, e0, e1));
    g.spare.push_back(e0);
    g.spare.push_back(e1);
    if (ms) *ms = f;
    return KVB_OK;
}

int resolve_part(const kvb_paged_args* a) {
    return a->part_tokens ? a->part_tokens : kvb_auto_part_tokens(a->batch, a->num_kv_heads, a->max_len);
}

int max_parts_of(const kvb_paged_args* a) {
    const int part = resolve_part(a);
    return std::max(1, (int)(((long long)a->max_len + part - 1) / part));
}

// The kernels' cap on a device-side length (live_len): what the block table and the workspace of
// this launch hold, min(max_blocks * page_size, max_parts * part_tokens). The host copy of the
// lengths has been checked against both; the cap keeps the kernels inside the buffers if the device
// copy disagrees.
int len_cap_of(const kvb_paged_args* a) {
    const long long cap = std::min((long long)a->max_blocks * a->page_size, (long long)max_parts_of(a) * resolve_part(a));
    return (int)std::min<long long>(cap, 0x7fffffff);
}

size_t workspace_need(const kvb_paged_args* a) {
    const size_t slots = (size_t)a->batch * a->num_heads * (size_t)max_parts_of(a);
    return slots * (size_t)a->head_dim * sizeof(float) + slots * sizeof(float2);
}

int check_lens(int batch, const int32_t* lens, int max_len, size_t capacity) {
    for (int b = 0; b < batch; ++b) {
        const int len = lens[b];
        if (len < 0 || len > max_len || (size_t)len > capacity)
            return fail(KVB_EINVAL, "sequence " + std::to_string(b) + " has length " + std::to_string(len) +
                                        ", max_len " + std::to_string(max_len) + ", capacity " +
                                        std::to_string(capacity));
    }
    return KVB_OK;
}

int check_shape(int batch, int H, int Hkv, int D) {
    if (batch < 0 || H <= 0 || Hkv <= 0) return fail(KVB_EINVAL, "batch < 0 or a head count <= 0");
    if (D != 64 && D != 128) return fail(KVB_EINVAL, "head_dim must be 64 or 128");
    if (H % Hkv != 0) return fail(KVB_EINVAL, "H % Hkv != 0");
    return KVB_OK;
}

// Every refusal of run_paged (src/metal_attn.mm:72-73, 107-117, 199-201), host-side only.
int validate_paged(const kvb_paged_args* a) {
    if (!a) return fail(KVB_EINVAL, "null arguments");
    if (a->part_tokens < 0 || a->max_len < 0 || a->page_size <= 0)
        return fail(KVB_EINVAL, "part_tokens < 0, max_len < 0 or page_size <= 0");
    if (a->kv_type < KVB_KV_F32 || a->kv_type > KVB_KV_I8) return fail(KVB_EINVAL, "unknown kv_type");
    if (a->kv_type == KVB_KV_I8 && (!a->k_scale || !a->v_scale)) return fail(KVB_EINVAL, "i8 cache without scales");
    if (int st = check_shape(a->batch, a->num_heads, a->num_kv_heads, a->head_dim)) return st;
    if (a->max_blocks < 0) return fail(KVB_EINVAL, "max_blocks < 0");
    if (a->batch > 0 && !a->host_seq_lens) return fail(KVB_EINVAL, "host_seq_lens is required");
    if (int st = check_lens(a->batch, a->host_seq_lens, a->max_len, (size_t)a->max_blocks * (size_t)a->page_size)) return st;
    if (a->batch > 0 && (!a->q || !a->k || !a->v || !a->seq_lens || !a->out || (a->max_blocks > 0 && !a->block_table)))
        return fail(KVB_EINVAL, "null device pointer");
    // launch grid (H / qg, batch, max_parts): y and z are at most 65535
    if (a->batch > 65535) return fail(KVB_EINVAL, "batch > 65535");
    if (max_parts_of(a) > 65535) return fail(KVB_EINVAL, "more than 65535 partitions: part_tokens too small for max_len");
    if (a->workspace && a->workspace_bytes < workspace_need(a))
        return fail(KVB_EINVAL, "workspace smaller than kvb_paged_workspace_bytes()");
    return KVB_OK;
}

int query_heads_per_group(const kvb_paged_args* a) {
    return kvb_heads_per_workgroup(a->num_heads, a->num_kv_heads, a->kv_type, a->share_kv);
}

// Grows the fused-merge counters to B * H ints, zeroed (the kernel leaves them at 0).
int counters_for(const kvb_paged_args* a, int** out) {
    const size_t need = ((size_t)a->batch * a->num_heads * sizeof(int) + 15) / 16 * 16;  // whole fill words
    if (g.counters_bytes < need || !g.counters) {
        if (int st = grow(&g.counters, &g.counters_bytes, need)) return st;
        // zeroed once here (a fill kernel, not a memset node); each fused launch leaves them at 0
        if (hipError_t e = kvbk::launch_fill(g.counters, g.counters_bytes / 16, 0u, g.stream); e != hipSuccess)
            return fail(KVB_ERUNTIME, std::string("counter fill: ") + hipGetErrorString(e));
    }
    *out = static_cast<int*>(g.counters);
    return KVB_OK;
}

// Queues one decode step. fused: one paged_decode that also merges the partitions; otherwise
// paged_decode then paged_reduce. `step` marks the start of the step's first kernel and the end of
// its last; `decode` and `reduce` (two-kernel form only) mark each kernel.
struct StepMarks {
    kvbk::Marks step, decode, reduce;
};

// Work items of a ragged batch in the kernel's longest-first order (one per partition holding
// tokens, one per empty sequence), or 0 for the plain (sequence, partition) grid: sequences of equal
// length gain nothing from reordering, and the order needs one lane per sequence.
int ragged_items(const kvb_paged_args* a, int part) {
    if (a->batch < 2 || a->batch > kvbk::kRaggedMaxBatch || part >= 65536) return 0;
    const int32_t* lens = a->host_seq_lens;
    bool equal = true;
    long long items = 0;
    for (int b = 0; b < a->batch; ++b) {
        equal = equal && lens[b] == lens[0];
        items += std::max(1LL, ((long long)lens[b] + part - 1) / part);
    }
    return equal || items > 65535 ? 0 : (int)items;
}

// counters: the fused merge's arrival counters (zero, at least B * H / qg ints), or null for the
// library's own (grown on demand).
int enqueue_paged(const kvb_paged_args* a, float* part_out, float2* part_ml, bool fused, const StepMarks& mk,
                  bool loads_only = false, int* counters = nullptr) {
    const int part = resolve_part(a);
    const int qg = query_heads_per_group(a);
    kvbk::DecodeParams p{};
    p.q = a->q;
    p.k = a->k;
    p.v = a->v;
    p.block_table = a->block_table;
    p.seq_lens = a->seq_lens;
    p.k_scale = a->k_scale;
    p.v_scale = a->v_scale;
    p.part_out = part_out;
    p.part_ml = part_ml;
    p.num_heads = a->num_heads;
    p.num_kv_heads = a->num_kv_heads;
    p.group = a->num_heads / a->num_kv_heads;
    p.qg = qg;
    p.page_size = a->page_size;
    p.page_div = kvbk::make_fast_div((uint32_t)a->page_size);
    p.tile_in_page = a->page_size % 32 == 0 && part % 32 == 0;
    p.max_blocks = a->max_blocks;
    p.max_parts = max_parts_of(a);
    p.part_tokens = part;
    p.len_cap = len_cap_of(a);
    p.qscale = (1.0f / std::sqrt((float)a->head_dim)) * 1.4426950408889634f;
    p.batch = a->batch;
    p.ragged_items = ragged_items(a, part);
    p.loads_only = loads_only;
    // fused merge when the group's partition (m, l) pairs fit its LDS staging; a workgroup with more
    // output chunks than threads merges in the one-round-trip form only (at most 16 partitions)
    if (fused && qg * p.max_parts > kvbk::fused_merge_slots(a->kv_type, a->head_dim)) fused = false;
    if (fused && !kvbk::fused_merge_many(a->kv_type, qg, a->head_dim) && p.max_parts > 16) fused = false;
    if (fused && g.merge_mode == KVB_MERGE_SEPARATE) fused = false;
    if (fused) {
        p.out = a->out;
        if (counters) p.counters = counters;
        else if (mk.step.describe) p.counters = nullptr;  // (nothing is launched)
        else if (int st = counters_for(a, &p.counters)) return st;
    }
    const bool fast = a->page_size % kvbk::kTile == 0 && part % kvbk::kTile == 0;
    // Two partitions per workgroup when the plain grid holds two or more workgroups per CU: the two
    // workgroups sharing a CU do not share it evenly (the first ends its loop long before the second,
    // which then streams alone); one workgroup per CU was faster (c2 on MI355X, 512 workgroups of 512
    // tokens: 28.3 us per step, against 26.5 us for 256 workgroups of 1024 tokens).
    const long long wgs = (long long)a->batch * (a->num_heads / qg) * p.max_parts;
    p.pair = fast && a->kv_type != KVB_KV_F32 && !p.ragged_items && p.max_parts >= 2 &&
             kvbk::decode_shape(a->kv_type, qg).hs == 1 &&
             part % (2 * kvbk::kTile * kvbk::decode_waves(a->kv_type)) == 0 &&
             (g.pair_mode == KVB_PAIR_ALWAYS || (g.pair_mode == KVB_PAIR_AUTO && wgs >= 2LL * g.cus));
    // blocks one workgroup's range touches: its tokens / page when the page divides them (the range
    // then starts on a page), else at most two more
    const long long span = (p.pair ? 2LL : 1LL) * part;
    const long long nb_max = span % a->page_size == 0 ? span / a->page_size : span / a->page_size + 2;
    p.table_in_lanes = fast && nb_max <= kvbk::kLaneBlocks;
    p.table_in_lds = !fast && nb_max <= kvbk::kTableStage;
    const kvbk::Marks dm{mk.step.start ? mk.step.start : mk.decode.start, fused ? mk.step.stop : mk.decode.stop,
                         mk.step.describe, mk.step.describe_cap};
    const kvbk::Marks rm{mk.reduce.start, mk.step.stop ? mk.step.stop : mk.reduce.stop};
    hipError_t e = hipSuccess;
    switch (a->kv_type) {
        case KVB_KV_F32: e = kvbk::launch_paged_decode_f32(a->head_dim, qg, fast, p, a->batch, g.stream, dm); break;
        case KVB_KV_F16: e = kvbk::launch_paged_decode_f16(a->head_dim, qg, fast, p, a->batch, g.stream, dm); break;
        default: e = kvbk::launch_paged_decode_i8(a->head_dim, qg, fast, p, a->batch, g.stream, dm); break;
    }
    if (e != hipSuccess) return fail(KVB_ERUNTIME, std::string("paged_decode launch: ") + hipGetErrorString(e));
    if (mk.step.describe) {
        if (!fused && !loads_only) {
            const size_t n = std::strlen(mk.step.describe);
            std::snprintf(mk.step.describe + n, mk.step.describe_cap - n, " + paged_reduce");
        }
        return KVB_OK;
    }
    if (fused || loads_only) return KVB_OK;
    kvbk::ReduceParams r{part_out, part_ml, a->seq_lens, a->out, a->num_heads, p.max_parts, part, p.len_cap};
    e = kvbk::launch_paged_reduce(a->head_dim, r, a->batch, g.stream, rm);
    if (e != hipSuccess) return fail(KVB_ERUNTIME, std::string("paged_reduce launch: ") + hipGetErrorString(e));
    return KVB_OK;
}

int workspace_for(const kvb_paged_args* a, float** part_out, float2** part_ml) {
    const size_t slots = (size_t)a->batch * a->num_heads * (size_t)max_parts_of(a);
    char* base = nullptr;
    if (a->workspace) {
        base = static_cast<char*>(a->workspace);
    } else {
        if (int st = grow(&g.ws, &g.ws_bytes, workspace_need(a))) return st;
        base = static_cast<char*>(g.ws);
    }
    *part_out = reinterpret_cast<float*>(base);
    *part_ml = reinterpret_cast<float2*>(base + slots * (size_t)a->head_dim * sizeof(float));
    return KVB_OK;
}

}  // namespace

extern "C" {

int kvb_gpu_available(void) {
    int n = 0;
    return hipGetDeviceCount(&n) == hipSuccess && n > 0;
}

int kvb_device_name(char* buf, size_t cap) {
    if (!buf || cap == 0) return fail(KVB_EINVAL, "null buffer");
    buf[0] = '\0';
    if (int st = ensure_device()) return st;
    hipDeviceProp_t prop;
    KVB_HIP(hipGetDeviceProperties(&prop, g.device));
    if (prop.name[0])  // (the marketing name is empty on some systems: then the architecture leads)
        std::snprintf(buf, cap, "%s (%s, %d CUs)", prop.name, prop.gcnArchName, prop.multiProcessorCount);
    else
        std::snprintf(buf, cap, "%s, %d CUs", prop.gcnArchName, prop.multiProcessorCount);
    return KVB_OK;
}

int kvb_device_info(kvb_device_info_t* info) {
    if (!info) return fail(KVB_EINVAL, "null kvb_device_info_t");
    *info = kvb_device_info_t{};
    if (int st = ensure_device()) return st;
    KVB_HIP(hipRuntimeGetVersion(&info->runtime_version));
    KVB_HIP(hipDriverGetVersion(&info->driver_version));
    hipDeviceProp_t prop;
    KVB_HIP(hipGetDeviceProperties(&prop, g.device));
    std::snprintf(info->name, sizeof(info->name), "%s", prop.name);
    std::snprintf(info->arch, sizeof(info->arch), "%s", prop.gcnArchName);
    KVB_HIP(hipDeviceGetPCIBusId(info->pci_bus_id, sizeof(info->pci_bus_id), g.device));
    info->device = g.device;
    info->compute_units = prop.multiProcessorCount;
    KVB_HIP(hipDeviceGetAttribute(&info->clock_khz, hipDeviceAttributeClockRate, g.device));
    KVB_HIP(hipDeviceGetAttribute(&info->memory_clock_khz, hipDeviceAttributeMemoryClockRate, g.device));
    KVB_HIP(hipDeviceGetAttribute(&info->memory_bus_bits, hipDeviceAttributeMemoryBusWidth, g.device));
    KVB_HIP(hipDeviceGetAttribute(&info->l2_bytes, hipDeviceAttributeL2CacheSize, g.device));
    info->total_memory = prop.totalGlobalMem;
    size_t free_b = 0, total_b = 0;
    KVB_HIP(hipMemGetInfo(&free_b, &total_b));
    info->free_memory = free_b;
    return KVB_OK;
}

int kvb_paged_kernel_name(const kvb_paged_args* a, int loads_only, char* buf, size_t cap) {
    if (!buf || cap == 0) return fail(KVB_EINVAL, "null buffer");
    buf[0] = '\0';
    if (int st = validate_paged(a)) return st;
    if (loads_only && (a->page_size % kvbk::kTile != 0 || resolve_part(a) % kvbk::kTile != 0))
        return fail(KVB_EINVAL, "the loads-only decode needs page_size and part_tokens that are multiples of 16");
    if (int st = ensure_device()) return st;
    if (a->batch == 0) return KVB_OK;
    StepMarks mk;
    mk.step.describe = buf;
    mk.step.describe_cap = cap;
    return enqueue_paged(a, nullptr, nullptr, !loads_only, mk, loads_only != 0);
}

int kvb_run_empty_grid(int workgroups, int threads, double* ms) {
    if (ms) *ms = 0.0;
    if (workgroups < 1 || threads < 1 || threads > 1024 || threads % 64 != 0)
        return fail(KVB_EINVAL, "kvb_run_empty_grid: workgroups >= 1 and threads a multiple of 64 up to 1024");
    if (int st = ensure_device()) return st;
    hipEvent_t e0, e1;
    if (int st = get_event(&e0)) return st;
    if (int st = get_event(&e1)) return st;
    const hipError_t e = kvbk::launch_empty(workgroups, threads, g.stream, {e0, e1});
    if (e != hipSuccess) return fail(KVB_ERUNTIME, std::string("empty grid launch: ") + hipGetErrorString(e));
    return finish(e0, e1, ms);
}

const char* kvb_last_error(void) { return g_err.c_str(); }

// Work already queued on the old stream uses the library's workspace and fused-merge counters, which
// every stream shares: the new stream waits for it (an event recorded on the old stream) before any
// work queued on it afterwards, so two steps never run at once.
int kvb_set_stream(void* stream) {
    if (int st = ensure_device()) return st;
    hipStream_t next = stream ? static_cast<hipStream_t>(stream) : g.own;
    if (next == g.stream) return KVB_OK;
    if (!g.switch_ev) KVB_HIP(hipEventCreateWithFlags(&g.switch_ev, hipEventDisableTiming));
    KVB_HIP(hipEventRecord(g.switch_ev, g.stream));
    KVB_HIP(hipStreamWaitEvent(next, g.switch_ev, 0));
    g.stream = next;
    return KVB_OK;
}

int kvb_set_pair_mode(int mode) {
    if (mode != KVB_PAIR_AUTO && mode != KVB_PAIR_OFF && mode != KVB_PAIR_ALWAYS) return -1;
    const int prev = g.pair_mode;
    g.pair_mode = mode;
    return prev;
}

int kvb_set_merge_mode(int mode) {
    if (mode != KVB_MERGE_AUTO && mode != KVB_MERGE_FUSED && mode != KVB_MERGE_SEPARATE) return -1;
    const int prev = g.merge_mode;
    g.merge_mode = mode;
    return prev;
}

int kvb_synchronize(void) {
    if (int st = ensure_device()) return st;
    KVB_HIP(hipStreamSynchronize(g.stream));
    return KVB_OK;
}

int kvb_buffer_alloc(void** dev, size_t bytes) {
    if (!dev) return fail(KVB_EINVAL, "null output pointer");
    *dev = nullptr;
    if (int st = ensure_device()) return st;
    KVB_HIP(hipMalloc(dev, std::max<size_t>(bytes, 16)));
    return KVB_OK;
}

int kvb_buffer_free(void* dev) {
    if (!dev) return KVB_OK;
    if (int st = ensure_device()) return st;
    KVB_HIP(hipStreamSynchronize(g.stream));
    KVB_HIP(hipFree(dev));
    return KVB_OK;
}

int kvb_copy_h2d(void* dev, const void* host, size_t bytes) {
    if (bytes == 0) return KVB_OK;
    if (!dev || !host) return fail(KVB_EINVAL, "null pointer");
    if (int st = ensure_device()) return st;
    KVB_HIP(hipMemcpyAsync(dev, host, bytes, hipMemcpyHostToDevice, g.stream));
    KVB_HIP(hipStreamSynchronize(g.stream));
    return KVB_OK;
}

int kvb_copy_d2h(void* host, const void* dev, size_t bytes) {
    if (bytes == 0) return KVB_OK;
    if (!dev || !host) return fail(KVB_EINVAL, "null pointer");
    if (int st = ensure_device()) return st;
    KVB_HIP(hipMemcpyAsync(host, dev, bytes, hipMemcpyDeviceToHost, g.stream));
    KVB_HIP(hipStreamSynchronize(g.stream));
    return KVB_OK;
}

int kvb_fill_bytes(void* dev, int value, size_t bytes) {
    if (bytes == 0) return KVB_OK;
    if (!dev) return fail(KVB_EINVAL, "null pointer");
    if (int st = ensure_device()) return st;
    KVB_HIP(hipMemsetAsync(dev, value, bytes, g.stream));
    KVB_HIP(hipStreamSynchronize(g.stream));
    return KVB_OK;
}

int kvb_auto_part_tokens(int batch, int num_kv_heads, int max_len) {
    int part = 512;
    while (part > 64 && (size_t)batch * num_kv_heads * (size_t)((max_len + part - 1) / part) < 512) part /= 2;
    return part;
}

int kvb_heads_per_workgroup(int num_heads, int num_kv_heads, int kv_type, int share_kv) {
    if (num_kv_heads <= 0 || num_heads <= 0 || num_heads % num_kv_heads != 0) return -1;
    if (kv_type != KVB_KV_F32 && kv_type != KVB_KV_F16 && kv_type != KVB_KV_I8) return -1;
    if (!share_kv) return 1;
    const int group = num_heads / num_kv_heads;
    // 32 or 16 heads (fp16, int8): one workgroup whose waves split the heads (kvbk::decode_shape),
    // so each page is read once from HBM for the whole group. fp32 (whose q operands are twice
    // fp16's) runs workgroups of at most 8.
    if (kv_type != KVB_KV_F32) {
        if (group % 32 == 0) return 32;
        if (group % 16 == 0) return 16;
    }
    for (int g = 8; g > 1; --g)
        if (group % g == 0) return g;
    return 1;
}

int kvb_paged_max_parts(const kvb_paged_args* a) {
    if (!a || a->part_tokens < 0 || a->max_len < 0 || a->batch < 0 || a->num_kv_heads <= 0) return -1;
    return max_parts_of(a);
}

size_t kvb_paged_workspace_bytes(const kvb_paged_args* a) {
    if (!a || a->part_tokens < 0 || a->max_len < 0 || a->batch < 0 || a->num_heads <= 0 || a->num_kv_heads <= 0 ||
        (a->head_dim != 64 && a->head_dim != 128))
        return 0;
    return workspace_need(a);
}

int kvb_check_paged(const kvb_paged_args* a) { return validate_paged(a); }

int kvb_run_paged_steps(const kvb_paged_args* a, int steps, double* ms) {
    if (ms) *ms = 0.0;
    if (int st = validate_paged(a)) return st;
    if (steps < 0) return fail(KVB_EINVAL, "steps < 0");
    if (int st = ensure_device()) return st;
    if (a->batch == 0 || steps == 0) return KVB_OK;
    float* part_out = nullptr;
    float2* part_ml = nullptr;
    if (int st = workspace_for(a, &part_out, &part_ml)) return st;
    hipEvent_t e0, e1;
    if (int st = get_event(&e0)) return st;
    if (int st = get_event(&e1)) return st;
    for (int i = 0; i < steps; ++i) {
        StepMarks mk;
        mk.step = {i == 0 ? e0 : nullptr, i == steps - 1 ? e1 : nullptr};
        if (int st = enqueue_paged(a, part_out, part_ml, true, mk)) return st;
    }
    return finish(e0, e1, ms);
}

int kvb_run_paged(const kvb_paged_args* a, double* ms) { return kvb_run_paged_steps(a, 1, ms); }

// A captured decode loop: the executable graph and the workspace it writes.
struct PagedGraph {
    hipGraphExec_t exec = nullptr;
    void* ws = nullptr;        // [split-K workspace][counters]
};

int kvb_graph_capture_paged(const kvb_paged_args* a, int steps, void** graph) {
    if (!graph) return fail(KVB_EINVAL, "null graph handle pointer");
    *graph = nullptr;
    if (int st = validate_paged(a)) return st;
    if (steps < 1) return fail(KVB_EINVAL, "kvb_graph_capture_paged: steps < 1");
    if (a->workspace) return fail(KVB_EINVAL, "kvb_graph_capture_paged takes no workspace: the graph owns its own");
    if (int st = ensure_device()) return st;
    if (g.pipelined) return fail(KVB_EINVAL, "kvb_graph_capture_paged: not in pipelined mode");
    // The graph's own workspace and counters, zeroed by a fill kernel before the capture (each fused
    // launch leaves the counters at 0 again, so every replay starts from zeros).
    const size_t ws_bytes = (workspace_need(a) + 255) / 256 * 256;
    const size_t cnt_bytes = ((size_t)a->batch * a->num_heads * sizeof(int) + 255) / 256 * 256;
    auto* pg = new PagedGraph;
    auto cleanup = [&](int st) {
        if (pg->ws) (void)hipFree(pg->ws);
        delete pg;
        return st;
    };
    if (hipMalloc(&pg->ws, ws_bytes + cnt_bytes) != hipSuccess)
        return cleanup(fail(KVB_ERUNTIME, "kvb_graph_capture_paged: workspace allocation failed"));
    char* base = static_cast<char*>(pg->ws);
    int* counters = reinterpret_cast<int*>(base + ws_bytes);
    if (hipError_t e = kvbk::launch_fill(counters, cnt_bytes / 16, 0u, g.stream); e != hipSuccess)
        return cleanup(fail(KVB_ERUNTIME, std::string("graph counter fill: ") + hipGetErrorString(e)));
    if (hipStreamSynchronize(g.stream) != hipSuccess)
        return cleanup(fail(KVB_ERUNTIME, "kvb_graph_capture_paged: stream synchronize failed"));
    const size_t slots = (size_t)a->batch * a->num_heads * (size_t)max_parts_of(a);
    float* part_out = reinterpret_cast<float*>(base);
    float2* part_ml = reinterpret_cast<float2*>(base + slots * (size_t)a->head_dim * sizeof(float));
    if (a->batch == 0) {  // nothing to capture: an empty graph
        hipGraph_t empty = nullptr;
        if (hipGraphCreate(&empty, 0) != hipSuccess ||
            hipGraphInstantiate(&pg->exec, empty, nullptr, nullptr, 0) != hipSuccess) {
            if (empty) (void)hipGraphDestroy(empty);
            return cleanup(fail(KVB_ERUNTIME, "kvb_graph_capture_paged: empty graph"));
        }
        (void)hipGraphDestroy(empty);
        *graph = pg;
        return KVB_OK;
    }
    hipGraph_t captured = nullptr;
    if (hipStreamBeginCapture(g.stream, hipStreamCaptureModeThreadLocal) != hipSuccess)
        return cleanup(fail(KVB_ERUNTIME, "kvb_graph_capture_paged: hipStreamBeginCapture failed"));
    int st = KVB_OK;
    for (int i = 0; i < steps && st == KVB_OK; ++i) st = enqueue_paged(a, part_out, part_ml, true, StepMarks{}, false, counters);
    const hipError_t ce = hipStreamEndCapture(g.stream, &captured);
    if (st != KVB_OK || ce != hipSuccess) {
        if (captured) (void)hipGraphDestroy(captured);
        return cleanup(st != KVB_OK ? st : fail(KVB_ERUNTIME, std::string("hipStreamEndCapture: ") + hipGetErrorString(ce)));
    }
    const hipError_t ie = hipGraphInstantiate(&pg->exec, captured, nullptr, nullptr, 0);
    (void)hipGraphDestroy(captured);
    if (ie != hipSuccess) return cleanup(fail(KVB_ERUNTIME, std::string("hipGraphInstantiate: ") + hipGetErrorString(ie)));
    *graph = pg;
    return KVB_OK;
}

int kvb_graph_launch(void* graph, double* ms) {
    if (ms) *ms = 0.0;
    if (!graph) return fail(KVB_EINVAL, "null graph");
    if (int st = ensure_device()) return st;
    auto* pg = static_cast<PagedGraph*>(graph);
    hipEvent_t e0, e1;
    if (int st = get_event(&e0)) return st;
    if (int st = get_event(&e1)) return st;
    KVB_HIP(hipEventRecord(e0, g.stream));
    KVB_HIP(hipGraphLaunch(pg->exec, g.stream));
    KVB_HIP(hipEventRecord(e1, g.stream));
    return finish(e0, e1, ms);
}

int kvb_graph_destroy(void* graph) {
    if (!graph) return KVB_OK;
    if (int st = ensure_device()) return st;
    auto* pg = static_cast<PagedGraph*>(graph);
    KVB_HIP(hipStreamSynchronize(g.stream));
    if (pg->exec) KVB_HIP(hipGraphExecDestroy(pg->exec));
    if (pg->ws) KVB_HIP(hipFree(pg->ws));
    delete pg;
    return KVB_OK;
}

// kvb_run_paged's step with the workspace and counters in `scratch` (no allocation, no events, no
// wait). The fused merge needs B * H / qg counters, qg the query heads per workgroup, at most B * H.
int kvb_run_paged_noalloc(const kvb_paged_args* a) {
    if (int st = validate_paged(a)) return st;
    if (a->workspace) return fail(KVB_EINVAL, "kvb_run_paged_noalloc takes no workspace: it uses its static scratch");
    if (workspace_need(a) > KVB_NOALLOC_WORKSPACE_BYTES)
        return fail(KVB_EINVAL, "kvb_run_paged_noalloc: the split-K workspace needs " + std::to_string(workspace_need(a)) +
                                    " bytes, more than its scratch holds (KVB_NOALLOC_WORKSPACE_BYTES = " +
                                    std::to_string((size_t)KVB_NOALLOC_WORKSPACE_BYTES) + "); use larger partitions");
    if ((size_t)a->batch * a->num_heads > KVB_NOALLOC_MAX_GROUPS)
        return fail(KVB_EINVAL, "kvb_run_paged_noalloc: batch * num_heads = " +
                                    std::to_string((size_t)a->batch * a->num_heads) +
                                    " is more than its scratch counters (KVB_NOALLOC_MAX_GROUPS = " +
                                    std::to_string(KVB_NOALLOC_MAX_GROUPS) + ")");
    if (int st = ensure_device()) return st;
    int device = -1;
    KVB_HIP(hipGetDevice(&device));
    if (device != g.device)
        return fail(KVB_EINVAL, "kvb_run_paged_noalloc: the library runs on device " + std::to_string(g.device) +
                                    ", the current device is " + std::to_string(device));
    if (a->batch == 0) return KVB_OK;
    char* base = static_cast<char*>(scratch_of(device));
    if (!base) return fail(KVB_ERUNTIME, "kvb_run_paged_noalloc: no scratch on this device: " + g_scratch_err);
    const size_t slots = (size_t)a->batch * a->num_heads * (size_t)max_parts_of(a);
    float* part_out = reinterpret_cast<float*>(base + kScratchCounterBytes);
    float2* part_ml = reinterpret_cast<float2*>(base + kScratchCounterBytes + slots * (size_t)a->head_dim * sizeof(float));
    return enqueue_paged(a, part_out, part_ml, true, StepMarks{}, false, reinterpret_cast<int*>(base));
}

int kvb_run_paged_split(const kvb_paged_args* a, double* decode_ms, double* reduce_ms) {
    if (decode_ms) *decode_ms = 0.0;
    if (reduce_ms) *reduce_ms = 0.0;
    if (int st = validate_paged(a)) return st;
    if (int st = ensure_device()) return st;
    if (a->batch == 0) return KVB_OK;
    float* part_out = nullptr;
    float2* part_ml = nullptr;
    if (int st = workspace_for(a, &part_out, &part_ml)) return st;
    hipEvent_t e[4];
    for (auto& x : e)
        if (int st = get_event(&x)) return st;
    StepMarks mk;
    mk.decode = {e[0], e[1]};
    mk.reduce = {e[2], e[3]};
    if (int st = enqueue_paged(a, part_out, part_ml, false, mk)) return st;
    KVB_HIP(hipEventSynchronize(e[3]));
    float d = 0.0f, r = 0.0f;
    KVB_HIP(hipEventElapsedTime(&d, e[0], e[1]));
    KVB_HIP(hipEventElapsedTime(&r, e[2], e[3]));
    for (auto& x : e) g.spare.push_back(x);
    if (decode_ms) *decode_ms = d;
    if (reduce_ms) *reduce_ms = r;
    return KVB_OK;
}

int kvb_run_paged_loads(const kvb_paged_args* a, double* ms) {
    if (ms) *ms = 0.0;
    if (int st = validate_paged(a)) return st;
    const int part = resolve_part(a);
    if (a->page_size % kvbk::kTile != 0 || part % kvbk::kTile != 0)
        return fail(KVB_EINVAL, "the loads-only decode needs page_size and part_tokens that are multiples of 16");
    if (int st = ensure_device()) return st;
    if (a->batch == 0) return KVB_OK;
    float* part_out = nullptr;
    float2* part_ml = nullptr;
    if (int st = workspace_for(a, &part_out, &part_ml)) return st;
    hipEvent_t e0, e1;
    if (int st = get_event(&e0)) return st;
    if (int st = get_event(&e1)) return st;
    StepMarks mk;
    mk.decode = {e0, e1};
    if (int st = enqueue_paged(a, part_out, part_ml, false, mk, true)) return st;
    return finish(e0, e1, ms);
}

int kvb_check_write_paged(const kvb_cache_args* a) {
    if (!a) return fail(KVB_EINVAL, "null arguments");
    if (a->kv_type < KVB_KV_F32 || a->kv_type > KVB_KV_I8) return fail(KVB_EINVAL, "unknown kv_type");
    if (a->batch < 0 || a->num_kv_heads <= 0) return fail(KVB_EINVAL, "batch < 0 or num_kv_heads <= 0");
    if (a->head_dim != 64 && a->head_dim != 128) return fail(KVB_EINVAL, "head_dim must be 64 or 128");
    if (a->page_size <= 0 || a->max_blocks < 0 || a->max_len < 0)
        return fail(KVB_EINVAL, "page_size <= 0, max_blocks < 0 or max_len < 0");
    if (a->batch > 65535 || ((long long)a->max_len + a->page_size - 1) / a->page_size > 65535)
        return fail(KVB_EINVAL, "more than 65535 sequences or logical blocks");
    if (a->batch > 0 && !a->host_seq_lens) return fail(KVB_EINVAL, "host_seq_lens is required");
    if (int st = check_lens(a->batch, a->host_seq_lens, a->max_len, (size_t)a->max_blocks * (size_t)a->page_size)) return st;
    if (a->batch > 0 && a->max_len > 0 &&
        (!a->contig || !a->paged || !a->block_table || !a->seq_lens || (a->kv_type == KVB_KV_I8 && !a->scales)))
        return fail(KVB_EINVAL, "null device pointer");
    return KVB_OK;
}

int kvb_write_paged(const kvb_cache_args* a, double* ms) {
    if (ms) *ms = 0.0;
    if (int st = kvb_check_write_paged(a)) return st;
    if (int st = ensure_device()) return st;
    if (a->batch == 0 || a->max_len == 0) return KVB_OK;
    kvbk::CacheWriteParams p{};
    p.contig = a->contig;
    p.paged = a->paged;
    p.scales = a->scales;
    p.block_table = a->block_table;
    p.seq_lens = a->seq_lens;
    p.num_kv_heads = a->num_kv_heads;
    p.head_dim = a->head_dim;
    p.elem_size = a->kv_type == KVB_KV_F32 ? 4 : a->kv_type == KVB_KV_F16 ? 2 : 1;
    p.page_size = a->page_size;
    p.max_blocks = a->max_blocks;
    p.max_len = a->max_len;
    p.quantize = a->kv_type == KVB_KV_I8;
    p.len_cap = (int)std::min((long long)a->max_len, (long long)a->max_blocks * a->page_size);
    hipEvent_t e0, e1;
    if (int st = get_event(&e0)) return st;
    if (int st = get_event(&e1)) return st;
    const int used = (a->max_len + a->page_size - 1) / a->page_size;
    const hipError_t e = kvbk::launch_write_paged(p, a->batch, used, g.stream, {e0, e1});
    if (e != hipSuccess) return fail(KVB_ERUNTIME, std::string("write_paged launch: ") + hipGetErrorString(e));
    return finish(e0, e1, ms);
}

int kvb_check_naive(const kvb_naive_args* a) {
    if (!a) return fail(KVB_EINVAL, "null arguments");
    if (a->kv_type == KVB_KV_I8) return fail(KVB_EINVAL, "naive kernels take f32 or f16 caches");
    if (a->kv_type != KVB_KV_F32 && a->kv_type != KVB_KV_F16) return fail(KVB_EINVAL, "unknown kv_type");
    if (int st = check_shape(a->batch, a->num_heads, a->num_kv_heads, a->head_dim)) return st;
    if (a->max_len < 0) return fail(KVB_EINVAL, "max_len < 0");
    // launch grids (max_len / 16, H, batch) and (H, batch): y and z are at most 65535
    if (a->batch > 65535 || a->num_heads > 65535) return fail(KVB_EINVAL, "batch or num_heads > 65535");
    if (a->batch > 0 && !a->host_seq_lens) return fail(KVB_EINVAL, "host_seq_lens is required");
    if (int st = check_lens(a->batch, a->host_seq_lens, a->max_len, (size_t)a->max_len)) return st;
    if (a->batch > 0 && (!a->q || !a->seq_lens || !a->out || (a->max_len > 0 && (!a->k || !a->v))))
        return fail(KVB_EINVAL, "null device pointer");
    return KVB_OK;
}

int kvb_run_naive(const kvb_naive_args* a, double* ms) {
    if (ms) *ms = 0.0;
    if (int st = kvb_check_naive(a)) return st;
    if (int st = ensure_device()) return st;
    if (a->batch == 0) return KVB_OK;
    const size_t need = (size_t)a->batch * a->num_heads * (size_t)std::max(a->max_len, 1) * sizeof(float);
    if (int st = grow(&g.scores, &g.scores_bytes, need)) return st;
    kvbk::NaiveParams p{a->q, a->k, a->v, a->seq_lens, static_cast<float*>(g.scores), a->out,
                        a->num_heads, a->num_kv_heads, a->max_len, 1.0f / std::sqrt((float)a->head_dim)};
    hipEvent_t e0, e1;
    if (int st = get_event(&e0)) return st;
    if (int st = get_event(&e1)) return st;
    const hipError_t e = kvbk::launch_naive(a->kv_type, a->head_dim, a->num_heads / a->num_kv_heads, p, a->batch,
                                            g.stream, {e0, e1});
    if (e != hipSuccess) return fail(KVB_ERUNTIME, std::string("naive launch: ") + hipGetErrorString(e));
    return finish(e0, e1, ms);
}

int kvb_run_attention_fp64(const kvb_naive_args* a, double* ms) {
    if (ms) *ms = 0.0;
    if (int st = kvb_check_naive(a)) return st;
    if (int st = ensure_device()) return st;
    if (a->batch == 0) return KVB_OK;
    kvbk::NaiveParams p{a->q, a->k, a->v, a->seq_lens, nullptr, a->out,
                        a->num_heads, a->num_kv_heads, a->max_len, 1.0f / std::sqrt((float)a->head_dim)};
    hipEvent_t e0, e1;
    if (int st = get_event(&e0)) return st;
    if (int st = get_event(&e1)) return st;
    const hipError_t e = kvbk::launch_attention_fp64(a->kv_type, a->head_dim, a->num_heads / a->num_kv_heads, p,
                                                     a->batch, g.stream, {e0, e1});
    if (e != hipSuccess) return fail(KVB_ERUNTIME, std::string("attention_fp64 launch: ") + hipGetErrorString(e));
    return finish(e0, e1, ms);
}

int kvb_begin_pipelined(void) {
    if (int st = ensure_device()) return st;
    g.pipelined = true;
    g.timed.clear();
    return KVB_OK;
}

size_t kvb_pipelined_pending(void) { return g.timed.size(); }

int kvb_end_pipelined(double* ms, size_t cap, size_t* count) {
    if (count) *count = 0;
    if (int st = ensure_device()) return st;
    g.pipelined = false;
    std::vector<std::pair<hipEvent_t, hipEvent_t>> timed;
    timed.swap(g.timed);
    size_t i = 0;
    int status = KVB_OK;
    for (auto& [e0, e1] : timed) {
        float f = 0.0f;
        if (status == KVB_OK) {
            hipError_t e = hipEventSynchronize(e1);
            if (e == hipSuccess) e = hipEventElapsedTime(&f, e0, e1);
            if (e != hipSuccess) status = fail(KVB_ERUNTIME, std::string("end_pipelined: ") + hipGetErrorString(e));
        }
        if (ms && i < cap) ms[i] = f;
        ++i;
        g.spare.push_back(e0);
        g.spare.push_back(e1);
    }
    if (count) *count = i;
    return status;
}

int kvb_run_read_bandwidth(const void* dev, size_t bytes, double* ms) {
    if (ms) *ms = 0.0;
    if (!dev || bytes == 0 || bytes % 16 != 0) return fail(KVB_EINVAL, "read probe needs a non-empty buffer of 16-byte words");
    if (int st = ensure_device()) return st;
    if (!g.sink) KVB_HIP(hipMalloc(&g.sink, kSinkFloats * sizeof(float)));
    hipEvent_t e0, e1;
    if (int st = get_event(&e0)) return st;
    if (int st = get_event(&e1)) return st;
    const hipError_t e = kvbk::launch_read_bw(dev, bytes / 16, g.cus, g.sink, g.stream, {e0, e1});
    if (e != hipSuccess) return fail(KVB_ERUNTIME, std::string("read_bw launch: ") + hipGetErrorString(e));
    return finish(e0, e1, ms);
}

// Reads (not writes) a 1 GiB buffer with ordinary loads: they allocate in the L2s and the 256 MB MALL
// and so evict what was there, and leave no dirty lines whose write-back would compete with the next
// timed run for HBM bandwidth. (Non-temporal loads, the probe's, do not evict the MALL: measured on
// MI355X, a step of the 134 MB c2 cache after such a flush took 26.7 us against 28.0 us after this
// one, and c3 46.1 against 47.3-48.1; the 537 MB c4 was 82.8 after either.)
int kvb_flush_gpu_caches(void) {
    if (int st = ensure_device()) return st;
    if (!g.sink) KVB_HIP(hipMalloc(&g.sink, kSinkFloats * sizeof(float)));
    if (!g.flush_buf) {
        KVB_HIP(hipMalloc(&g.flush_buf, kFlushBytes));
        const hipError_t e = kvbk::launch_fill(g.flush_buf, kFlushBytes / 16, 0x3f800000u, g.stream);
        if (e != hipSuccess) return fail(KVB_ERUNTIME, std::string("flush fill: ") + hipGetErrorString(e));
    }
    const hipError_t e = kvbk::launch_read_bw(g.flush_buf, kFlushBytes / 16, g.cus, g.sink, g.stream, {}, false);
    if (e != hipSuccess) return fail(KVB_ERUNTIME, std::string("flush launch: ") + hipGetErrorString(e));
    return KVB_OK;
}

}  // extern "C"
