// C++20 interface to the MI355X decode-attention kernels: the reference's src/metal_attn.hpp
// (lines 11-108) with the same names, argument meaning and exceptions, implemented over the C ABI
// of include/kvb_hip.h. Tests and benchmarks stay ordinary C++.
#pragma once

#include <cstddef>
#include <memory>
#include <span>
#include <string>
#include <vector>

#include "kvb/reference.hpp"
#include "kvb_hip.h"

namespace kvb {

bool gpu_available();
// The reference's name for gpu_available() (src/metal_attn.hpp:13), kept so callers switch over unchanged.
inline bool metal_available() { return gpu_available(); }
std::string device_name();

// Device memory in HBM with a host mirror. The reference's Buffer is shared CPU/GPU storage
// (src/metal_attn.hpp:16-33); on a discrete GPU the two copies are kept in step here: data()/as()
// give the host copy for reading and writing (fetching the device copy first if a kernel wrote it
// since), and the run_* calls upload host writes before launching. So "fill on the host, run,
// read on the host" works as with the reference, and a timed loop that does not touch data()
// moves no bytes over PCIe. The host copy is allocated on first use.
class Buffer {
public:
    explicit Buffer(size_t bytes);
    ~Buffer();
    Buffer(const Buffer&) = delete;
    Buffer& operator=(const Buffer&) = delete;
    void* data() const;                // host copy, may be written: the device copy is refreshed before the next kernel
    const void* host() const;          // host copy, read only (no upload follows)
    size_t size() const { return bytes_; }
    template <class T> T* as() const { return static_cast<T*>(data()); }
    void* handle() const { return dev_; }  // device pointer
    // For the launch code: uploads pending host writes and returns the device pointer; after a kernel
    // writes the buffer, mark_device_written() makes the next host access fetch it.
    void* device() const;
    void mark_device_written() const;

private:
    enum State { kZero, kHostNewer, kSynced, kDeviceNewer };
    void ensure_host() const;
    void* dev_ = nullptr;
    size_t bytes_ = 0;
    mutable std::unique_ptr<unsigned char[]> host_;
    mutable State state_ = kZero;  // kZero: neither copy written yet (both read as zeros)
};

// i8: int8 values with one fp32 scale per (block, KV head) for K and V (quantize_to_paged_i8).
enum class KvType { f32, f16, i8 };
inline const char* name(KvType t) { return t == KvType::f32 ? "f32" : t == KvType::f16 ? "f16" : "i8"; }
inline size_t elem_size(KvType t) { return t == KvType::f32 ? 4 : t == KvType::f16 ? 2 : 1; }

// The reference's simdgroups per workgroup (src/metal_attn.hpp:41). Here paged_decode workgroups
// have 4 wave64s, one per SIMD, for every storage type.
constexpr int kSimdGroups = 4;

// Split-K partition size used when PagedArgs::part_tokens is 0 (src/metal_attn.hpp:43-51): the
// largest power of two in [64, 512] that still yields at least 512 (sequence, KV head,
// partition) triples.
inline int auto_part_tokens(const Shape& s, int max_len) {
    int part = 512;
    while (part > 64 && size_t(s.batch) * s.num_kv_heads * ((max_len + part - 1) / part) < 512) part /= 2;
    return part;
}

// The MI355X partition policy: the largest power of two in [min_part, max_part] whose workgroup
// count B * ceil(H / qg) * ceil(max_len / part) still reaches `min_groups` (qg: the query heads one
// workgroup serves, kvb_heads_per_workgroup). Longer partitions mean fewer partial results to merge and a shorter prologue
// per token; enough workgroups keep enough bytes in flight. Measured on MI355X (c4): fastest at
// one workgroup per CU (min_groups 256, the default).
int mi355x_part_tokens(const Shape& s, int max_len, int min_groups = 256, int min_part = 256, int max_part = 4096);
// The policy for a batch given its lengths. Lengths that are not all equal make a ragged batch,
// which runs in the longest-first work order. Its partition trades the schedule's end (finer pieces
// with shorter partitions) against each workgroup's fixed cost (prologue, epilogue, merge), paid
// once per partition. The partition is capped at ragged_part_cap(max_len): 2048 while the longest
// sequence is under two 3584-token partitions, 4096 once it spans seven 4096-token ones (28672
// tokens: uniform draws up to 32768 rarely reach 32768 itself), 3584 (7 x 512) between. Measured on MI355X, 32 q / 8 KV heads, head_dim 128, page 64, cold steps, us at
// partitions 2048 / 3584 / 4096 (the cap's choice marked *):
//   64 lengths ~U[1, 4096]:   fp16 95.8* / 100.6 / 109.7; int8 58.2* / 60.3 / 62.8
//   64 lengths ~U[1, 8192]:   fp16 175.7 / 176.0* / 182.3; int8 99.6 / 99.6* / 102.6
//   128 lengths ~U[1, 8192]:  fp16 337.8 / 333.2* / 329.4; int8 190.3 / 183.4* / 180.1
//   32 lengths ~U[1, 16384]:  fp16 182.4-182.7 / 181.8-183.5* / 186.7; int8 103.3-104.4 / 102.0-102.4* / 104.0
//   c5, 72 lengths ~U[1, 16384]: fp16 333.9-335.8 / 328.6-332.3* / 341.0-341.5;
//       int8 183.6-184.5 / 182.1-183.1* / 185.5-186.7
//   64 lengths ~U[1, 32768]:  fp16 688.9 / 676.5 / 671.9*; int8 375.8 / 363.8 / 360.0*
//   16 lengths ~U[1, 65536]:  fp16 399.6 / 404.0 / 389.9*; int8 222.3 / 220.3 / 213.4*
// Sizes in between were not better: c5 at 2560-3328 and 3840 ran 0-1.5% slower than at 3584, and
// 32 lengths ~U[1, 16384] ran 2.5-3% slower at 2560 (fp16) than at 2048 or 3584.
// With pages under 64 tokens a partition over 4096 / 64 pages spans more than 64 blocks, whose ids
// the kernel then reads per tile instead of keeping them in lanes; a caller with such pages may
// pass max_part = 64 * page_size.
constexpr int kRaggedShortCap = 2048, kRaggedCap = 3584, kRaggedLongCap = 4096;
int ragged_part_cap(int max_len);
int mi355x_part_tokens(const Shape& s, std::span<const int> lens, int min_groups = 256, int min_part = 256,
                       int max_part = 4096);
// min_groups of the policy: 256 (one workgroup per CU), or 512 (two) when a K or V row is under
// 128 bytes (int8 at head_dim 64), where a 4096-token workgroup streams only 512 KB. Measured on
// MI355X, c4's shape at head_dim 64, int8: 29.5 us at 2048-token partitions (512 workgroups)
// against 33.8 us at 4096; fp16 and head_dim 128 are fastest at 256 workgroups.
inline int mi355x_min_groups(KvType t, int head_dim = 128) { return elem_size(t) * head_dim < 128 ? 512 : 256; }

struct PagedArgs {
    Shape shape;
    KvType type = KvType::f32;
    int page_size = 16;
    int max_blocks = 0;      // PagedLayout::max_blocks
    int max_len = 0;         // longest sequence, sizes the split-K workspace; 0: all empty, out is 0
    int part_tokens = 0;     // split-K partition size, 0 = auto_part_tokens()
    const Buffer* q;         // float [B][H][D]
    const Buffer* k;         // type  [blocks][Hkv][page][D]
    const Buffer* v;
    const Buffer* block_table;  // int32 [B][max_blocks]
    const Buffer* seq_lens;     // int32 [B]
    const Buffer* out;          // float [B][H][D]
    bool share_kv = true;       // false: one workgroup per query head (GQA ablation)
    const Buffer* k_scale = nullptr;  // float [blocks][Hkv], required for KvType::i8
    const Buffer* v_scale = nullptr;
    const Buffer* workspace = nullptr;  // optional split-K workspace (kvb_paged_workspace_bytes)
};

struct NaiveArgs {
    Shape shape;
    KvType type = KvType::f32;
    int max_len = 0;  // row stride of the contiguous cache
    const Buffer* q;
    const Buffer* k;  // type [B][Hkv][max_len][D]
    const Buffer* v;
    const Buffer* seq_lens;
    const Buffer* out;
};

// The paged cache written on the GPU from a contiguous cache in HBM: scatter_to_paged for f32/f16
// and quantize_to_paged_i8 for i8 (fp32 input; scales required), the reference's host-side writers
// (src/reference.hpp:60-68, src/reference.cpp:32-51) with the same bytes and scales. Only live
// tokens are written.
struct CacheWriteArgs {
    Shape shape;                 // batch, num_kv_heads, head_dim (64 or 128); num_heads is unused
    KvType type = KvType::f32;
    int page_size = 16;
    int max_blocks = 0;
    int max_len = 0;             // row stride of the contiguous cache
    const Buffer* contig;        // type [B][Hkv][max_len][D] (fp32 for i8)
    const Buffer* paged;         // type [blocks][Hkv][page][D]
    const Buffer* scales = nullptr;  // float [blocks][Hkv], i8 only
    const Buffer* block_table;   // int32 [B][max_blocks]
    const Buffer* seq_lens;      // int32 [B]
};
double write_paged(const CacheWriteArgs&);

// Each call queues the kernels on one stream, waits, and returns their GPU time in milliseconds,
// from the first kernel's start to the last kernel's end (events stamped by the dispatches). Throws std::invalid_argument, before any GPU work, for a sequence length below
// 0, above max_len, or (paged) above max_blocks * page_size, and for the other refusals of
// kvb_run_paged; std::runtime_error for device failures (src/metal_attn.hpp:82-87).
double run_paged(const PagedArgs&);
double run_naive(const NaiveArgs&);
// The reference's fp64 attention_reference on the GPU (same arguments as run_naive; f32/f16): the
// accuracy reference of kvbench --accuracy / --dump. Not a fast path.
double run_attention_fp64(const NaiveArgs&);

// `steps` decode steps on the same inputs, back to back on one stream (src/metal_attn.hpp:89-91).
double run_paged_steps(const PagedArgs&, int steps);

// `steps` decode steps captured into a HIP graph (kvb_graph_capture_paged; not in the reference,
// whose steps are command buffers), for loops that replay a fixed step with one launch. launch()
// replays them on the library's stream and returns their GPU milliseconds (0 in pipelined mode).
// The graph owns its workspace and keeps the buffers of its PagedArgs by address: keep them alive,
// and their shapes unchanged, while it exists. Throws as run_paged does.
class PagedGraph {
public:
    PagedGraph(const PagedArgs&, int steps);
    ~PagedGraph();
    PagedGraph(const PagedGraph&) = delete;
    PagedGraph& operator=(const PagedGraph&) = delete;
    double launch();

private:
    const PagedArgs* args_;
    void* handle_ = nullptr;
};

// One decode step with the GPU time of each kernel.
struct KernelTimes {
    double decode_ms = 0, reduce_ms = 0;
};
KernelTimes run_paged_split(const PagedArgs&);

// The decode's loads alone (kvb_run_paged_loads; not in the reference): every K/V and scale load of
// paged_decode in the same order, no arithmetic, output not written. Returns GPU milliseconds.
double run_paged_loads(const PagedArgs&);

// Between begin_pipelined() and end_pipelined(), run_*() and flush_gpu_caches() queue their work
// without waiting (run_*() return 0); end_pipelined() waits and returns the GPU time of every
// run_*() call in order (src/metal_attn.hpp:93-99). On one HIP stream the runs execute one at a
// time, back to back.
void begin_pipelined();
std::vector<double> end_pipelined();

// Reads `src` once with a streaming kernel over every CU; returns GPU milliseconds.
double run_read_bandwidth(const Buffer& src);

// Reads a 1 GiB scratch buffer, more than the MALL and L2s hold, so the next run starts cold.
void flush_gpu_caches();

// The C ABI view of `a` (device pointers resolved, host writes uploaded).
kvb_paged_args c_args(const PagedArgs& a);

}  // namespace kvb
