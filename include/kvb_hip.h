/*
 * kvb_hip.h -- C ABI of libkvb_hip.so, the MI355X (gfx950) paged-KV decode-attention library.
 *
 * This is the drop-in boundary: it replaces the Objective-C++/Metal host layer behind the
 * reference's C++ interface (chipontix/kv-cache-bench src/metal_attn.hpp:11-108, implemented in
 * src/metal_attn.mm). Every entry point takes plain pointers and sizes; device pointers come
 * from kvb_buffer_alloc (or any hipMalloc'd memory of the current device). Calls are
 * single-threaded and not reentrant, like the reference (src/metal_attn.mm:40-42).
 *
 * Status codes: KVB_OK, KVB_EINVAL (bad arguments, refused before any GPU work: the reference's
 * std::invalid_argument), KVB_ERUNTIME (a HIP failure: std::runtime_error), KVB_ENODEV (no GPU:
 * the reference's metal_available() == false, exit code 77 in its tests). kvb_last_error()
 * describes the last failing call.
 */
#ifndef KVB_HIP_H
#define KVB_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { KVB_OK = 0, KVB_EINVAL = 1, KVB_ERUNTIME = 2, KVB_ENODEV = 3 };

/* KV storage types (KvType, src/metal_attn.hpp:35-39). I8 carries one fp32 scale per
 * (physical block, KV head) for K and one for V. */
enum { KVB_KV_F32 = 0, KVB_KV_F16 = 1, KVB_KV_I8 = 2 };

/* ---- device ------------------------------------------------------------------------------ */

/* 1 if a HIP device is present (metal_available, src/metal_attn.hpp:13). */
int kvb_gpu_available(void);
/* Device name into buf (device_name, src/metal_attn.hpp:14). */
int kvb_device_name(char* buf, size_t cap);
/* What the environment record of a result holds about the device and the HIP stack (the counterpart
 * of the reference's scripts/env.sh, which records machine, toolchain and load beside its results). */
typedef struct kvb_device_info_t {
    int runtime_version;  /* hipRuntimeGetVersion */
    int driver_version;   /* hipDriverGetVersion */
    int device;           /* the library's device ordinal */
    int compute_units;
    int clock_khz;        /* peak shader clock (hipDeviceAttributeClockRate) */
    int memory_clock_khz; /* hipDeviceAttributeMemoryClockRate */
    int memory_bus_bits;
    int l2_bytes;         /* one XCD's L2 as the runtime reports it */
    size_t total_memory;
    size_t free_memory;   /* at the call */
    char name[256];
    char arch[64];        /* gcnArchName, e.g. gfx950:sramecc+:xnack- */
    char pci_bus_id[32];
} kvb_device_info_t;
/* Fills *info for the library's device. No reference counterpart beyond device_name. */
int kvb_device_info(kvb_device_info_t* info);
/* Message of the last call that did not return KVB_OK ("" if none). */
const char* kvb_last_error(void);
/* Runs the library's work on `stream` (a hipStream_t; NULL = the library's own stream, created
 * at default priority). Timing events are recorded on the same stream. Work queued on the new
 * stream after this call waits for everything already queued on the previous one (an event), since
 * every stream shares the library's workspace and merge counters: switching never lets two steps
 * run at once. No reference counterpart: lets a caller that owns a stream (a serving loop,
 * PyTorch) order decode steps with its own work. */
int kvb_set_stream(void* stream);
/* Waits for all work the library has queued (on the current stream, which waits for the earlier ones). */
int kvb_synchronize(void);

/* ---- memory (Buffer, src/metal_attn.hpp:16-33) ------------------------------------------- */
/* The reference's Buffer is shared CPU/GPU storage; on MI355X the device copy lives in HBM and
 * the C++ host layer keeps a host mirror, moved with these copies. */
int kvb_buffer_alloc(void** dev, size_t bytes); /* min 16 bytes, like src/metal_attn.mm:142 */
int kvb_buffer_free(void* dev);
int kvb_copy_h2d(void* dev, const void* host, size_t bytes);
int kvb_copy_d2h(void* host, const void* dev, size_t bytes);
int kvb_fill_bytes(void* dev, int value, size_t bytes);

/* ---- paged decode (PagedArgs, src/metal_attn.hpp:53-69) ---------------------------------- */
typedef struct kvb_paged_args {
    int batch;        /* B: sequences, one new query token each */
    int num_heads;    /* H: query heads */
    int num_kv_heads; /* Hkv: KV heads, H % Hkv == 0; query head h reads KV head h / (H / Hkv) */
    int head_dim;     /* D: 64 or 128 */
    int kv_type;      /* KVB_KV_F32 | KVB_KV_F16 | KVB_KV_I8 */
    int page_size;    /* tokens per physical block */
    int max_blocks;   /* row stride of block_table */
    int max_len;      /* longest sequence; sizes the split-K workspace; 0: every output is 0 */
    int part_tokens;  /* split-K partition size in tokens, 0 = kvb_auto_part_tokens() */
    int share_kv;     /* 1: one workgroup serves every query head of a KV head (reads K/V once per
                         group); 0: one workgroup per query head (the GQA ablation) */
    const float* q;              /* device, float [B][H][D] */
    const void* k;               /* device, kv_type [blocks][Hkv][page_size][D] */
    const void* v;               /* device, same layout as k */
    const int32_t* block_table;  /* device, int32 [B][max_blocks]; logical block i of sequence b
                                    lives in physical block block_table[b*max_blocks + i] */
    const int32_t* seq_lens;     /* device, int32 [B] */
    const int32_t* host_seq_lens;/* host copy of seq_lens, equal to it: capacity check, launch size.
                                    If the device copy disagrees, the kernels clamp each of its lengths
                                    to [0, min(max_blocks * page_size, max_parts * part)] and read a -1
                                    table entry as an empty page, so they stay inside the table rows and
                                    the workspace; the output is then unspecified. Block ids themselves
                                    are trusted (the pool's size is not an argument), as in the reference. */
    float* out;                  /* device, float [B][H][D] */
    const float* k_scale;        /* device, float [blocks][Hkv]; required for I8 */
    const float* v_scale;
    /* Optional caller-owned split-K workspace (NULL: the library's grow-only workspace). Layout:
     * part_out float [B][H][max_parts][D], then part_ml float2 [B][H][max_parts] = (m, l), with m
     * the partition's max score (natural-log units) and l its exp-sum; see
     * kvb_paged_workspace_bytes. Only slots of non-empty partitions are written. */
    void* workspace;
    size_t workspace_bytes;
} kvb_paged_args;

/* Split-K partition size used when part_tokens == 0 (auto_part_tokens, src/metal_attn.hpp:43-51):
 * the largest power of two in [64, 512] with batch * Hkv * ceil(max_len / part) >= 512. */
int kvb_auto_part_tokens(int batch, int num_kv_heads, int max_len);
/* Partitions per (sequence, head) in the workspace: max(1, ceil(max_len / part)) with part
 * resolved as kvb_run_paged does (src/metal_attn.mm:160-161). Returns -1 on bad arguments. */
int kvb_paged_max_parts(const kvb_paged_args* a);
/* Bytes of the workspace a call with these arguments uses (0 on bad arguments). */
size_t kvb_paged_workspace_bytes(const kvb_paged_args* a);
/* Query heads one paged_decode workgroup serves, which read each K/V page once together: with
 * share_kv and an f16 or i8 cache, 32 or 16 when it divides the group num_heads / num_kv_heads;
 * otherwise the largest divisor of the group that is at most 8 (a group of 7 is one workgroup per
 * KV head, a group of 12 two of 6, a group of 64 two of 32); without share_kv, 1. The reference's
 * kernel serves the whole group from one threadgroup (QG = GROUP, src/metal_attn.mm:64-80); here
 * a wave's score MFMA holds up to 8 heads in two columns each, or 16 in one column each (f16, i8),
 * and a workgroup of 32 heads splits them over two sets of waves that walk the same tiles (f16:
 * each tile loaded once and shared through LDS). Returns -1 on bad arguments
 * (num_kv_heads <= 0, num_heads not a positive multiple of it, kv_type not a kvb_kv_type). */
int kvb_heads_per_workgroup(int num_heads, int num_kv_heads, int kv_type, int share_kv);

/* The refusals of kvb_run_paged alone (KVB_OK or KVB_EINVAL): reads only host_seq_lens and the
 * sizes, needs no GPU. Lets a host layer refuse before it uploads anything. */
int kvb_check_paged(const kvb_paged_args* a);

/* One decode step (run_paged, src/metal_attn.hpp:86): the reference's paged_decode + paged_reduce
 * as one launch of paged_decode whose last workgroup per (sequence, KV-head group) merges the
 * partitions; two kernels (paged_decode, then paged_reduce) when a group's (m, l) pairs exceed what
 * that merge stages in LDS: query heads per group x max_parts > 4 waves x 32 tokens x head_dim x
 * elem_size / 8 (at head_dim 128: 4096 for f16, 8192 for f32, 2048 for i8; half that at 64), or
 * when max_parts > 16 and a workgroup (kvb_heads_per_workgroup) serves 16 f16 query heads, or 32
 * heads at head_dim 128 (f16, i8), or 32 f16 heads at 64.
 * Either form gives the same bits. *ms = GPU time
 * from before the first kernel to after the last (hipEvent pair); 0 in pipelined mode. Refuses (KVB_EINVAL, before any GPU work, output untouched) part_tokens < 0, max_len < 0,
 * page_size <= 0, I8 without scales, a length < 0 or > max_len or > max_blocks * page_size,
 * head_dim not 64/128, H % Hkv != 0 (src/metal_attn.mm:72-73, 107-117, 199-201). */
int kvb_run_paged(const kvb_paged_args* a, double* ms);
/* No counterpart in the reference: for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc). kvb_run_paged's decode step,
 * with the same arguments, refusals, kernels and output bits, but the split-K workspace and the
 * fused-merge counters live in a static device array of the library (KVB_NOALLOC_WORKSPACE_BYTES of
 * workspace plus KVB_NOALLOC_MAX_GROUPS counters, held by every GPU the library runs on until the
 * process ends). It allocates nothing, records no events and does not wait: the step is queued on
 * the library's current stream (kvb_set_stream); read `out` after kvb_synchronize or the caller's
 * own ordering. KVB_EINVAL (before any GPU work) for a->workspace set, a workspace need
 * (kvb_paged_workspace_bytes) above KVB_NOALLOC_WORKSPACE_BYTES, batch * num_heads above
 * KVB_NOALLOC_MAX_GROUPS, or a current device other than the library's. The library's set-up, on
 * its first call of any entry point, resolves the array's address and zeroes its counters (which
 * every step leaves at 0): make that first call outside graph capture. Every call on one GPU shares
 * the one array: calls that overlap on a GPU (on streams not ordered with each other) race. */
#define KVB_NOALLOC_WORKSPACE_BYTES (16u << 20)
#define KVB_NOALLOC_MAX_GROUPS 16384
int kvb_run_paged_noalloc(const kvb_paged_args* a);
/* `steps` decode steps on the same inputs, back to back on one stream, one event pair around them
 * (run_paged_steps, src/metal_attn.hpp:91). */
int kvb_run_paged_steps(const kvb_paged_args* a, int steps, double* ms);
/* No counterpart in the reference (its steps are Metal command buffers): kvb_run_paged_steps' `steps`
 * decode steps captured once into a HIP graph, for serving loops that replay a fixed step with one
 * launch. The graph owns its split-K workspace and merge counters (allocated and zeroed here, before
 * the capture, and freed by kvb_graph_destroy), so no later call can move them; it holds the
 * caller's pointers from `a` (q, k, v, tables, lengths, scales, out), which must stay valid and keep
 * their shapes while it exists. The captured steps are the same kernels, in the same order, as
 * kvb_run_paged_steps: the same bits. They allocate nothing and contain no memset node. The grid
 * and the work order are fixed at capture from host_seq_lens. Equal lengths at capture (the plain
 * grid): each replay serves the device seq_lens as they are then, clamped to the captured max_len.
 * Lengths not all equal (the longest-first order): every replay needs device seq_lens equal to the
 * captured host_seq_lens; lengths that make a different number of work items turn the replay into a
 * no-op that leaves out as it was and reports no error. Same refusals as kvb_run_paged, plus
 * KVB_EINVAL for steps < 1, a->workspace set, or pipelined mode. *graph receives an opaque handle. */
int kvb_graph_capture_paged(const kvb_paged_args* a, int steps, void** graph);
/* Launches a captured graph on the library's current stream. *ms = GPU time of the launch (hipEvent
 * pair); 0 in pipelined mode. KVB_EINVAL for a null handle. */
int kvb_graph_launch(void* graph, double* ms);
/* Waits for the library's stream, then frees the graph and its workspace. Null is a no-op. */
int kvb_graph_destroy(void* graph);
/* One synchronous decode step in the reference's two-kernel form, timed per kernel: *decode_ms and
 * *reduce_ms are the hipEvent times of paged_decode (no merge) and of paged_reduce. Not in the
 * reference (its timing is per command buffer, src/metal_attn.mm:119-130). */
int kvb_run_paged_split(const kvb_paged_args* a, double* decode_ms, double* reduce_ms);
/* Measurement aid, not in the reference: the paged_decode launch of kvb_run_paged_split with the
 * arithmetic taken out. Same grid and work order; every K/V load (and, for I8, every scale load)
 * is issued in the same order and the registers are consumed by XORs. The output is not written
 * (the library's workspace is scratch, as always). *ms = its hipEvent time: the time of
 * the decode's memory traffic alone, which bounds the decode kernel from below. Same refusals as
 * kvb_run_paged, plus KVB_EINVAL unless page_size and the partition are multiples of 16. */
int kvb_run_paged_loads(const kvb_paged_args* a, double* ms);
/* Measurement aid, not in the reference: one launch of a kernel that does nothing, `workgroups`
 * workgroups of `threads` threads (a multiple of 64, at most 1024), timed like a decode step (events
 * stamped by the dispatch): the floor that dispatch and completion put under any kernel of that grid.
 * KVB_EINVAL for other sizes. */
int kvb_run_empty_grid(int workgroups, int threads, double* ms);
/* Not in the reference: the name of the paged_decode kernel that kvb_run_paged (loads_only 0) or
 * kvb_run_paged_loads (1) launches for these arguments, as rocprofv3 prints it, followed by
 * " + paged_reduce" where the step falls back to the two-kernel form; nothing is launched. A
 * profile of a run is attached to a result only when the names agree. Same refusals as those calls. */
int kvb_paged_kernel_name(const kvb_paged_args* a, int loads_only, char* buf, size_t cap);
/* Tuning switch, not in the reference: when a decode workgroup computes two consecutive partitions
 * instead of one. KVB_PAIR_AUTO (the default): when the plain (sequence, partition) grid would put
 * two or more workgroups on every CU; KVB_PAIR_OFF: never; KVB_PAIR_ALWAYS: whenever it is allowed.
 * It is allowed for f16 and i8 caches with page_size and the partition multiples of 16, the
 * partition a multiple of 128, at least two partitions, and equal lengths (or one sequence). Every
 * setting gives the same bits: each partition is computed by the same waves, in the same order.
 * Returns the previous setting, or -1 for an unknown one (nothing changed). Applies to every later
 * decode step of the process. */
#define KVB_PAIR_AUTO 0
#define KVB_PAIR_OFF 1
#define KVB_PAIR_ALWAYS 2
int kvb_set_pair_mode(int mode);
/* Tuning switch, not in the reference: where kvb_run_paged, kvb_run_paged_steps and the captured
 * graph merge a step's partitions (the reference's paged_reduce, src/metal_attn.mm:184-194).
 * KVB_MERGE_FUSED: in paged_decode itself (the last workgroup of each group merges it) wherever the
 * fused merge can take the group; KVB_MERGE_SEPARATE: always as a second kernel, paged_reduce, which
 * spreads the merge over a workgroup per (sequence, head). KVB_MERGE_AUTO (the default) is
 * KVB_MERGE_FUSED: on MI355X the fused step was the faster at 8 to 64 partitions per sequence
 * (the reference's default sweep, batch 2, 32 query / 8 KV heads: e.g. f16 at 8192 tokens, 32
 * partitions, 20.7-21.0 us fused against 22.5 us separate). Every setting gives the same bits.
 * Returns the previous setting, or -1 for an unknown one (nothing changed). Applies to every later
 * decode step of the process. */
#define KVB_MERGE_AUTO 0
#define KVB_MERGE_FUSED 1
#define KVB_MERGE_SEPARATE 2
int kvb_set_merge_mode(int mode);

/* ---- cache writers on the GPU --------------------------------------------------------------
 * The producers of the paged cache the decode reads, as the reference runs them on the host:
 * scatter_to_paged (src/reference.hpp:60-68) for F32/F16 and quantize_to_paged_i8
 * (src/reference.cpp:32-51) for I8, with the same bytes and scales. Only live tokens' rows (and,
 * for I8, the scales of live (block, KV head) pairs) are written; the rest of the pool is left as
 * it was. */
typedef struct kvb_cache_args {
    int batch;        /* B */
    int num_kv_heads; /* Hkv */
    int head_dim;     /* D: 64 or 128 */
    int kv_type;      /* KVB_KV_F32 / KVB_KV_F16: copy; KVB_KV_I8: quantise fp32 input */
    int page_size;
    int max_blocks;   /* row stride of block_table */
    int max_len;      /* row stride (in tokens) of the contiguous cache */
    const void* contig;          /* device, [B][Hkv][max_len][D]: kv_type values, fp32 for I8 */
    void* paged;                 /* device, [blocks][Hkv][page_size][D] of kv_type */
    float* scales;               /* device, float [blocks][Hkv]; required for I8 */
    const int32_t* block_table;  /* device, int32 [B][max_blocks] */
    const int32_t* seq_lens;     /* device, int32 [B] */
    const int32_t* host_seq_lens;/* host copy of seq_lens, read by the capacity check */
} kvb_cache_args;

/* Writes the paged cache; *ms = the kernel's GPU time (0 in pipelined mode). Refuses (KVB_EINVAL,
 * before any GPU work) bad sizes, head_dim not 64/128, a length < 0 or > max_len or
 * > max_blocks * page_size, I8 without scales, null device pointers. */
int kvb_write_paged(const kvb_cache_args* a, double* ms);
/* The refusals of kvb_write_paged alone; needs no GPU. */
int kvb_check_write_paged(const kvb_cache_args* a);

/* ---- naive 3-pass baseline (NaiveArgs / run_naive, src/metal_attn.hpp:71-87) ------------- */
typedef struct kvb_naive_args {
    int batch, num_heads, num_kv_heads, head_dim;
    int kv_type;                 /* KVB_KV_F32 or KVB_KV_F16 */
    int max_len;                 /* row stride of the contiguous cache */
    const float* q;              /* device, float [B][H][D] */
    const void* k;               /* device, kv_type [B][Hkv][max_len][D] */
    const void* v;
    const int32_t* seq_lens;     /* device, int32 [B] */
    const int32_t* host_seq_lens;/* host copy of seq_lens */
    float* out;                  /* device, float [B][H][D] */
} kvb_naive_args;
/* scores -> softmax -> PV with the scores in global memory. Refuses I8 and lengths < 0 or
 * > max_len (src/metal_attn.mm:211-247). */
int kvb_run_naive(const kvb_naive_args* a, double* ms);
/* The refusals of kvb_run_naive alone. */
int kvb_check_naive(const kvb_naive_args* a);
/* The reference's fp64 attention_reference (src/reference.cpp:65-100) on the GPU, with the same
 * arguments as kvb_run_naive: out (fp32) = two-pass fp64 softmax attention over the contiguous
 * f32 or f16 cache, 0 for an empty sequence. Not a fast path: the accuracy reference of the
 * benchmark's --accuracy and --dump modes (bench/bench.cpp:130-215). */
int kvb_run_attention_fp64(const kvb_naive_args* a, double* ms);

/* ---- timing modes (src/metal_attn.hpp:93-99) --------------------------------------------- */
/* Between begin and end, run_* queue their work without waiting and return 0; end waits and
 * writes the GPU time of each timed run_* call in order (up to cap values, *count = number of
 * runs). The flush is queued but not timed, as in src/metal_attn.mm:266-276. */
int kvb_begin_pipelined(void);
/* Timed runs queued since kvb_begin_pipelined (the size end_pipelined needs). */
size_t kvb_pipelined_pending(void);
int kvb_end_pipelined(double* ms, size_t cap, size_t* count);

/* ---- probes ------------------------------------------------------------------------------ */
/* Streams `bytes` (a multiple of 16) of `dev` once with non-temporal 128-bit loads over every CU; *ms
 * is the kernel's GPU time (run_read_bandwidth, src/metal_attn.hpp:102). */
int kvb_run_read_bandwidth(const void* dev, size_t bytes, double* ms);
/* Reads a 1 GiB scratch buffer (more than the 256 MB MALL plus the L2s) with ordinary loads, which
 * allocate in those caches, so the next timed run starts cold (flush_gpu_caches,
 * src/metal_attn.hpp:106, whose 256 MiB blit fill writes instead: reading evicts as well and leaves
 * no dirty lines to write back during the timed run). */
int kvb_flush_gpu_caches(void);

#ifdef __cplusplus
}
#endif
#endif /* KVB_HIP_H */
