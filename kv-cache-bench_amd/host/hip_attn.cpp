// C++ interface (include/kvb/hip_attn.hpp) over the C ABI of libkvb_hip.so: buffers with a host
// mirror, argument translation, and the reference's exceptions (src/metal_attn.mm:57-59, 134-293).
#include "kvb/hip_attn.hpp"

#include <algorithm>
#include <cstring>
#include <stdexcept>
#include <string>

namespace kvb {
namespace {

[[noreturn]] void raise(int status, const char* what) {
    const std::string msg = std::string(what) + ": " + kvb_last_error();
    if (status == KVB_EINVAL) throw std::invalid_argument(msg);
    throw std::runtime_error(msg);
}

void check(int status, const char* what) {
    if (status != KVB_OK) raise(status, what);
}

int c_type(KvType t) { return t == KvType::f32 ? KVB_KV_F32 : t == KvType::f16 ? KVB_KV_F16 : KVB_KV_I8; }

const void* dev(const Buffer* b) { return b ? b->handle() : nullptr; }

// The C view without uploading anything: device pointers as allocated, host lengths for the checks.
kvb_paged_args view(const PagedArgs& a) {
    kvb_paged_args c{};
    c.batch = a.shape.batch;
    c.num_heads = a.shape.num_heads;
    c.num_kv_heads = a.shape.num_kv_heads;
    c.head_dim = a.shape.head_dim;
    c.kv_type = c_type(a.type);
    c.page_size = a.page_size;
    c.max_blocks = a.max_blocks;
    c.max_len = a.max_len;
    c.part_tokens = a.part_tokens;
    c.share_kv = a.share_kv ? 1 : 0;
    c.q = static_cast<const float*>(dev(a.q));
    c.k = dev(a.k);
    c.v = dev(a.v);
    c.block_table = static_cast<const int32_t*>(dev(a.block_table));
    c.seq_lens = static_cast<const int32_t*>(dev(a.seq_lens));
    c.host_seq_lens = a.seq_lens ? static_cast<const int32_t*>(a.seq_lens->host()) : nullptr;
    c.out = static_cast<float*>(const_cast<void*>(dev(a.out)));
    c.k_scale = static_cast<const float*>(dev(a.k_scale));
    c.v_scale = static_cast<const float*>(dev(a.v_scale));
    c.workspace = a.workspace ? a.workspace->handle() : nullptr;
    c.workspace_bytes = a.workspace ? a.workspace->size() : 0;
    return c;
}

void upload_inputs(const PagedArgs& a) {
    for (const Buffer* b : {a.q, a.k, a.v, a.block_table, a.seq_lens, a.out, a.k_scale, a.v_scale})
        if (b) b->device();
}

void mark_written(const PagedArgs& a) {
    a.out->mark_device_written();
    if (a.workspace) a.workspace->mark_device_written();
}

}  // namespace

bool gpu_available() { return kvb_gpu_available() != 0; }

std::string device_name() {
    char buf[256];
    return kvb_device_name(buf, sizeof buf) == KVB_OK ? std::string(buf) : std::string();
}

// ---- Buffer ----------------------------------------------------------------------------------------

Buffer::Buffer(size_t bytes) : bytes_(bytes) { check(kvb_buffer_alloc(&dev_, bytes), "Buffer allocation"); }

Buffer::~Buffer() { kvb_buffer_free(dev_); }

void Buffer::ensure_host() const {
    if (!host_) {
        host_.reset(new unsigned char[bytes_ ? bytes_ : 1]);
        if (state_ == kZero) {
            std::memset(host_.get(), 0, bytes_);
            return;
        }
        check(kvb_copy_d2h(host_.get(), dev_, bytes_), "Buffer download");
        state_ = kSynced;
        return;
    }
    if (state_ == kDeviceNewer) {
        check(kvb_copy_d2h(host_.get(), dev_, bytes_), "Buffer download");
        state_ = kSynced;
    }
}

void* Buffer::data() const {
    ensure_host();
    state_ = kHostNewer;
    return host_.get();
}

const void* Buffer::host() const {
    ensure_host();
    return host_.get();
}

void* Buffer::device() const {
    if (state_ == kHostNewer) {
        check(kvb_copy_h2d(dev_, host_.get(), bytes_), "Buffer upload");
        state_ = kSynced;
    } else if (state_ == kZero) {
        check(kvb_fill_bytes(dev_, 0, bytes_), "Buffer zero fill");
        state_ = kSynced;
    }
    return dev_;
}

void Buffer::mark_device_written() const { state_ = kDeviceNewer; }

// ---- runs --------------------------------------------------------------------------------------------

int mi355x_part_tokens(const Shape& s, int max_len, int min_groups, int min_part, int max_part) {
    // (f16/i8 workgroups: a group of 16 or 32 is one workgroup per KV head)
    const int qg = std::max(1, kvb_heads_per_workgroup(s.num_heads, s.num_kv_heads, KVB_KV_F16, 1));
    const long long per_part = (long long)s.batch * (s.num_heads / qg);
    int part = max_part;
    while (part > min_part && per_part * ((max_len + part - 1) / part) < min_groups) part /= 2;
    return part;
}

int mi355x_part_tokens(const Shape& s, std::span<const int> lens, int min_groups, int min_part, int max_part) {
    int max_len = 0;
    bool ragged = false;
    for (int len : lens) {
        max_len = std::max(max_len, len);
        ragged = ragged || len != lens[0];
    }
    const int part = mi355x_part_tokens(s, max_len, min_groups, min_part, max_part);
    return ragged ? std::max(std::min(min_part, part), std::min(part, ragged_part_cap(max_len))) : part;
}

int ragged_part_cap(int max_len) {
    if (max_len >= 7 * kRaggedLongCap) return kRaggedLongCap;
    return max_len >= 2 * kRaggedCap ? kRaggedCap : kRaggedShortCap;
}

kvb_paged_args c_args(const PagedArgs& a) {
    upload_inputs(a);
    return view(a);
}

double run_paged_steps(const PagedArgs& a, int steps) {
    kvb_paged_args c = view(a);
    check(kvb_check_paged(&c), "run_paged");  // refuse before anything reaches the GPU
    upload_inputs(a);
    double ms = 0;
    check(kvb_run_paged_steps(&c, steps, &ms), "run_paged");
    mark_written(a);
    return ms;
}

double run_paged(const PagedArgs& a) { return run_paged_steps(a, 1); }

PagedGraph::PagedGraph(const PagedArgs& a, int steps) : args_(&a) {
    kvb_paged_args c = view(a);
    check(kvb_check_paged(&c), "capture_paged_graph");
    upload_inputs(a);
    check(kvb_graph_capture_paged(&c, steps, &handle_), "capture_paged_graph");
}

PagedGraph::~PagedGraph() { (void)kvb_graph_destroy(handle_); }

double PagedGraph::launch() {
    double ms = 0;
    check(kvb_graph_launch(handle_, &ms), "graph_launch");
    mark_written(*args_);
    return ms;
}

KernelTimes run_paged_split(const PagedArgs& a) {
    kvb_paged_args c = view(a);
    check(kvb_check_paged(&c), "run_paged_split");
    upload_inputs(a);
    KernelTimes t;
    check(kvb_run_paged_split(&c, &t.decode_ms, &t.reduce_ms), "run_paged_split");
    mark_written(a);
    return t;
}

double run_paged_loads(const PagedArgs& a) {
    kvb_paged_args c = view(a);
    check(kvb_check_paged(&c), "run_paged_loads");
    upload_inputs(a);
    double ms = 0;
    check(kvb_run_paged_loads(&c, &ms), "run_paged_loads");
    return ms;
}

namespace {
kvb_naive_args naive_view(const NaiveArgs& a) {
    kvb_naive_args c{};
    c.batch = a.shape.batch;
    c.num_heads = a.shape.num_heads;
    c.num_kv_heads = a.shape.num_kv_heads;
    c.head_dim = a.shape.head_dim;
    c.kv_type = c_type(a.type);
    c.max_len = a.max_len;
    c.q = static_cast<const float*>(dev(a.q));
    c.k = dev(a.k);
    c.v = dev(a.v);
    c.seq_lens = static_cast<const int32_t*>(dev(a.seq_lens));
    c.host_seq_lens = a.seq_lens ? static_cast<const int32_t*>(a.seq_lens->host()) : nullptr;
    c.out = static_cast<float*>(const_cast<void*>(dev(a.out)));
    return c;
}
}  // namespace

double run_attention_fp64(const NaiveArgs& a) {
    kvb_naive_args c = naive_view(a);
    check(kvb_check_naive(&c), "run_attention_fp64");
    for (const Buffer* b : {a.q, a.k, a.v, a.seq_lens, a.out})
        if (b) b->device();
    double ms = 0;
    check(kvb_run_attention_fp64(&c, &ms), "run_attention_fp64");
    a.out->mark_device_written();
    return ms;
}

double run_naive(const NaiveArgs& a) {
    kvb_naive_args c{};
    c.batch = a.shape.batch;
    c.num_heads = a.shape.num_heads;
    c.num_kv_heads = a.shape.num_kv_heads;
    c.head_dim = a.shape.head_dim;
    c.kv_type = c_type(a.type);
    c.max_len = a.max_len;
    c.q = static_cast<const float*>(dev(a.q));
    c.k = dev(a.k);
    c.v = dev(a.v);
    c.seq_lens = static_cast<const int32_t*>(dev(a.seq_lens));
    c.host_seq_lens = a.seq_lens ? static_cast<const int32_t*>(a.seq_lens->host()) : nullptr;
    c.out = static_cast<float*>(const_cast<void*>(dev(a.out)));
    check(kvb_check_naive(&c), "run_naive");
    for (const Buffer* b : {a.q, a.k, a.v, a.seq_lens, a.out})
        if (b) b->device();
    double ms = 0;
    check(kvb_run_naive(&c, &ms), "run_naive");
    a.out->mark_device_written();
    return ms;
}

double write_paged(const CacheWriteArgs& a) {
    kvb_cache_args c{};
    c.batch = a.shape.batch;
    c.num_kv_heads = a.shape.num_kv_heads;
    c.head_dim = a.shape.head_dim;
    c.kv_type = c_type(a.type);
    c.page_size = a.page_size;
    c.max_blocks = a.max_blocks;
    c.max_len = a.max_len;
    c.contig = dev(a.contig);
    c.paged = const_cast<void*>(dev(a.paged));
    c.scales = static_cast<float*>(const_cast<void*>(dev(a.scales)));
    c.block_table = static_cast<const int32_t*>(dev(a.block_table));
    c.seq_lens = static_cast<const int32_t*>(dev(a.seq_lens));
    c.host_seq_lens = a.seq_lens ? static_cast<const int32_t*>(a.seq_lens->host()) : nullptr;
    check(kvb_check_write_paged(&c), "write_paged");
    // the pool (and scales) keep what is not written: bring any host writes over first
    for (const Buffer* b : {a.contig, a.paged, a.scales, a.block_table, a.seq_lens})
        if (b) b->device();
    double ms = 0;
    check(kvb_write_paged(&c, &ms), "write_paged");
    a.paged->mark_device_written();
    if (a.scales) a.scales->mark_device_written();
    return ms;
}

void begin_pipelined() { check(kvb_begin_pipelined(), "begin_pipelined"); }

std::vector<double> end_pipelined() {
    std::vector<double> ms(kvb_pipelined_pending());
    size_t n = 0;
    check(kvb_end_pipelined(ms.data(), ms.size(), &n), "end_pipelined");
    ms.resize(std::min(n, ms.size()));
    return ms;
}

double run_read_bandwidth(const Buffer& src) {
    src.device();
    double ms = 0;
    check(kvb_run_read_bandwidth(src.handle(), src.size() / 16 * 16, &ms), "run_read_bandwidth");
    return ms;
}

void flush_gpu_caches() { check(kvb_flush_gpu_caches(), "flush_gpu_caches"); }

}  // namespace kvb
