// kvbench: the decode-step benchmark of this build, CSV on stdout.
//
// Interface: the flags, CSV columns and row names of the reference's bench/bench.cpp (flags at
// :48-84; headers at :124, :156, :187, :212; impl names gpu_naive, cpu_ref_fp64, gpu_paged,
// gpu_paged_per_head, ours; layouts contiguous, paged16; err_vs stored, fp32_data), so its consumer
// (scripts/tables.py) reads this output. Each header starts with the reference's columns; this
// build's columns follow them. This build adds the gpu_paged_loads rows (--loads: the decode's loads
// alone) and the flags --loads, --config, --pool, --dist, --bw-bytes, --cpu-ref, --merge
// (kvb_set_merge_mode: auto, fused or separate) and --schema (print each mode's header, no GPU
// needed).
//
// Modes, one per run: the sweep (default), --bw, --dump=DIR, --chain=N, --accuracy.
// Timing: GPU time from hipEvent pairs stamped by the kernel dispatches; before each timed run a
// 1 GiB read flushes the MALL and L2s (unless --no-flush); runs are queued back to back (pipelined)
// unless --sync; the median, min and max of --reps runs after --warmup are reported.
// fp64 references: --accuracy, --dump and the chain's max_err use the GPU's fp64 attention
// (run_attention_fp64). The cpu_ref_fp64 rows time the reference's own CPU path, its
// attention_reference, from the reference's kvref built as a shared library and named by
// --cpu-ref=LIB; this program does not link it, and without --cpu-ref there are no such rows.
#include <dlfcn.h>
#include <unistd.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <map>
#include <span>
#include <string>
#include <thread>
#include <vector>

#include "kvb/workload.hpp"
#include "kvb_hip.h"

namespace {

using namespace kvb;
using Clock = std::chrono::steady_clock;

// ---- options ---------------------------------------------------------------------------------

struct Options {
    Shape shape{2, 32, 8, 128};
    std::vector<int> lens{512, 1024, 2048, 4096, 8192, 16384, 32768}, pages{16, 32, 64, 128}, parts{0};
    std::vector<KvType> types{KvType::f32, KvType::f16, KvType::i8};
    int reps = 30, warmup = 3, cpu_reps = 3, chain = 0;
    bool graph = false;  // --graph: the chain's paged rows also replayed from a captured HIP graph
    bool naive = true, cpu = true, flush = true, per_head = false, bw = false, sync = false, accuracy = false,
         loads = false, schema = false;
    std::string dump, config, cpu_ref;
    Dist dist = Dist::uniform;
    double pool = 1.0;
    int merge = KVB_MERGE_AUTO;  // --merge: kvb_set_merge_mode
    size_t bw_bytes = size_t(512) << 20;  // past the 256 MB MALL
};

std::vector<int> int_list(const char* s) {
    std::vector<int> v;
    for (const char* p = s; *p;) {
        char* end = nullptr;
        v.push_back(int(std::strtol(p, &end, 10)));
        p = *end == ',' ? end + 1 : end;
        if (end == p && *p) break;
    }
    return v;
}

// Every flag is a row of this table: a name, whether it takes "=value", and what it sets.
struct Flag {
    const char* name;
    bool valued;
    std::function<void(Options&, const char*)> set;
};

const std::vector<Flag>& flags() {
    static const std::vector<Flag> table = {
        {"--batch", true, [](Options& o, const char* v) { o.shape.batch = std::atoi(v); }},
        {"--heads", true, [](Options& o, const char* v) { o.shape.num_heads = std::atoi(v); }},
        {"--kv-heads", true, [](Options& o, const char* v) { o.shape.num_kv_heads = std::atoi(v); }},
        {"--dim", true, [](Options& o, const char* v) { o.shape.head_dim = std::atoi(v); }},
        {"--lens", true, [](Options& o, const char* v) { o.lens = int_list(v); }},
        {"--pages", true, [](Options& o, const char* v) { o.pages = int_list(v); }},
        {"--parts", true, [](Options& o, const char* v) { o.parts = int_list(v); }},
        {"--reps", true, [](Options& o, const char* v) { o.reps = std::atoi(v); }},
        {"--warmup", true, [](Options& o, const char* v) { o.warmup = std::atoi(v); }},
        {"--cpu-reps", true, [](Options& o, const char* v) { o.cpu_reps = std::atoi(v); }},
        {"--chain", true, [](Options& o, const char* v) { o.chain = std::atoi(v); }},
        {"--graph", false, [](Options& o, const char*) { o.graph = true; }},
        {"--dump", true, [](Options& o, const char* v) { o.dump = v; }},
        {"--types", true,
         [](Options& o, const char* v) {
             o.types.clear();
             for (KvType t : {KvType::f32, KvType::f16, KvType::i8})
                 if (std::strstr(v, name(t))) o.types.push_back(t);
         }},
        {"--no-naive", false, [](Options& o, const char*) { o.naive = false; }},
        {"--no-cpu", false, [](Options& o, const char*) { o.cpu = false; }},
        {"--no-flush", false, [](Options& o, const char*) { o.flush = false; }},
        {"--per-head", false, [](Options& o, const char*) { o.per_head = true; }},
        {"--bw", false, [](Options& o, const char*) { o.bw = true; }},
        {"--sync", false, [](Options& o, const char*) { o.sync = true; }},
        {"--accuracy", false, [](Options& o, const char*) { o.accuracy = true; }},
        // this build's
        {"--loads", false, [](Options& o, const char*) { o.loads = true; }},
        {"--config", true, [](Options& o, const char* v) { o.config = v; }},
        {"--pool", true, [](Options& o, const char* v) { o.pool = std::atof(v); }},
        {"--merge", true,
         [](Options& o, const char* v) {
             o.merge = !std::strcmp(v, "fused") ? KVB_MERGE_FUSED : !std::strcmp(v, "separate") ? KVB_MERGE_SEPARATE
                     : !std::strcmp(v, "auto")  ? KVB_MERGE_AUTO
                                                : -1;
         }},
        {"--dist", true, [](Options& o, const char* v) { o.dist = std::strcmp(v, "normal") ? Dist::uniform : Dist::normal; }},
        {"--bw-bytes", true, [](Options& o, const char* v) { o.bw_bytes = size_t(std::atof(v)); }},
        {"--cpu-ref", true, [](Options& o, const char* v) { o.cpu_ref = v; }},
        {"--schema", false, [](Options& o, const char*) { o.schema = true; }},
    };
    return table;
}

bool parse(int argc, char** argv, Options& o) {
    for (int i = 1; i < argc; ++i) {
        const char* a = argv[i];
        const Flag* hit = nullptr;
        const char* value = nullptr;
        for (const Flag& f : flags()) {
            const size_t n = std::strlen(f.name);
            if (std::strncmp(a, f.name, n) != 0) continue;
            if (f.valued && a[n] == '=') hit = &f, value = a + n + 1;
            else if (!f.valued && a[n] == '\0') hit = &f;
            if (hit) break;
        }
        if (!hit) {
            std::fprintf(stderr, "unknown argument %s\n", a);
            return false;
        }
        hit->set(o, value);
    }
    return true;
}

// The BASELINE configurations as sweeps of one point each (N(0,1) data, their page, partition and
// pool); the ragged c5 is bench.py's.
bool apply_config(Options& o) {
    struct Config {
        const char* name;
        Shape shape;
        int len, page;
        KvType type;
        double pool;
    };
    static const Config configs[] = {
        {"c1", {1, 32, 8, 128}, 512, 16, KvType::f32, 2.0},
        {"c2", {8, 32, 8, 128}, 4096, 16, KvType::f16, 1.5},
        {"c3", {16, 32, 8, 128}, 8192, 64, KvType::i8, 1.0},
        {"c4", {4, 64, 8, 128}, 32768, 128, KvType::f16, 1.25},
    };
    if (o.config.empty()) return true;
    for (const Config& c : configs) {
        if (o.config != c.name) continue;
        o.shape = c.shape;
        o.lens = {c.len};
        o.pages = {c.page};
        o.types = {c.type};
        o.pool = c.pool;
        o.dist = Dist::normal;
        // c1 and c2 name their partitions; c3 and c4 take the MI355X policy's
        if (o.config == "c1") o.parts = {128};
        else if (o.config == "c2") o.parts = {512};
        else o.parts = {mi355x_part_tokens(c.shape, c.len, mi355x_min_groups(c.type, c.shape.head_dim))};
        return true;
    }
    std::fprintf(stderr, "unknown config %s (c1..c4)\n", o.config.c_str());
    return false;
}

// ---- CSV tables with named columns -------------------------------------------------------------

// A mode's columns: the reference's header, then this build's additions.
struct Schema {
    const char* mode;
    std::vector<std::string> reference, own;
    std::string header() const {
        std::string h;
        for (const auto* part : {&reference, &own})
            for (const std::string& c : *part) h += (h.empty() ? "" : ",") + c;
        return h;
    }
};

const Schema kSweepSchema{"sweep",
                          {"impl", "dtype", "batch", "seq_len", "page", "part", "reps", "median_us", "min_us", "max_us",
                           "gbps", "max_diff_vs_naive", "kv_bytes"},
                          {"decode_us", "reduce_us"}};
const Schema kBwSchema{"bw", {"impl", "bytes", "reps", "median_us", "min_us", "max_us", "gbps"}, {}};
const Schema kChainSchema{"chain",
                          {"impl", "layout", "dtype", "batch", "seq_len", "chain", "reps", "median_us", "min_us",
                           "max_us", "gbps", "max_err", "err_vs"},
                          {"gpu_us"}};
const Schema kAccuracySchema{"accuracy", {"data", "dtype", "seq_len", "page", "max_abs_err", "rms_err"}, {}};

class Table {
public:
    explicit Table(const Schema& schema) {
        cols_ = schema.reference;
        cols_.insert(cols_.end(), schema.own.begin(), schema.own.end());
        for (size_t i = 0; i < cols_.size(); ++i) index_[cols_[i]] = i;
        std::printf("%s\n", schema.header().c_str());
    }

    class Row {
    public:
        explicit Row(const Table& t) : t_(t), cells_(t.cols_.size()) {}
        Row& text(const char* col, const std::string& v) { return put(col, v); }
        Row& count(const char* col, long long v) { return put(col, std::to_string(v)); }
        Row& fixed(const char* col, double v, int digits) { return put(col, format("%.*f", digits, v)); }
        Row& general(const char* col, double v) { return put(col, format("%.3g", v)); }
        void emit() const {
            std::string line;
            for (size_t i = 0; i < cells_.size(); ++i) line += (i ? "," : "") + cells_[i];
            std::printf("%s\n", line.c_str());
            std::fflush(stdout);
        }

    private:
        Row& put(const char* col, std::string v) {
            const auto it = t_.index_.find(col);
            if (it == t_.index_.end()) {
                std::fprintf(stderr, "kvbench: no column %s\n", col);
                std::abort();
            }
            cells_[it->second] = std::move(v);
            return *this;
        }
        template <class... A>
        static std::string format(const char* f, A... a) {
            char buf[64];
            std::snprintf(buf, sizeof buf, f, a...);
            return buf;
        }
        const Table& t_;
        std::vector<std::string> cells_;
    };
    Row row() const { return Row(*this); }

private:
    std::vector<std::string> cols_;
    std::map<std::string, size_t> index_;
};

// ---- timing ------------------------------------------------------------------------------------

struct Sample {
    double median = 0, min = 0, max = 0;  // milliseconds
    double median_us() const { return median * 1e3; }
};

Sample summarise(std::vector<double> ms) {
    Sample s;
    if (ms.empty()) return s;
    std::sort(ms.begin(), ms.end());
    const size_t n = ms.size();
    s.median = n % 2 ? ms[n / 2] : 0.5 * (ms[n / 2 - 1] + ms[n / 2]);
    s.min = ms.front();
    s.max = ms.back();
    return s;
}

// Times a GPU step (a function returning its GPU milliseconds, 0 when queued in pipelined mode).
class GpuTimer {
public:
    explicit GpuTimer(const Options& o) : o_(o) {}
    Sample operator()(const std::function<double()>& step) const {
        std::vector<double> ms;
        if (!o_.sync) begin_pipelined();
        for (int i = 0; i < o_.warmup + o_.reps; ++i) {
            if (i >= o_.warmup && o_.flush) flush_gpu_caches();
            const double t = step();
            if (o_.sync && i >= o_.warmup) ms.push_back(t);
        }
        if (!o_.sync) {
            ms = end_pipelined();
            ms.erase(ms.begin(), ms.begin() + std::min<size_t>(ms.size(), size_t(o_.warmup)));
        }
        return summarise(ms);
    }

private:
    const Options& o_;
};

double gbps(double bytes, const Sample& s) { return s.median > 0 ? bytes / (s.median * 1e-3) / 1e9 : 0.0; }

// ---- the reference's CPU path, loaded at run time ------------------------------------------------

// attention_reference<float> and <half_t> from the reference's kvref (src/reference.cpp:65-100),
// looked up by their C++ names in a shared library the caller names.
class CpuReference {
public:
    explicit CpuReference(const std::string& path) {
        if (path.empty()) return;
        lib_ = dlopen(path.c_str(), RTLD_NOW | RTLD_LOCAL);
        if (!lib_) {
            std::fprintf(stderr, "kvbench: --cpu-ref: %s\n", dlerror());
            return;
        }
        f32_ = reinterpret_cast<Fn<float>>(dlsym(lib_, kF32));
        f16_ = reinterpret_cast<Fn<half_t>>(dlsym(lib_, kF16));
        if (!f32_ || !f16_) std::fprintf(stderr, "kvbench: --cpu-ref: %s has no attention_reference\n", path.c_str());
    }
    ~CpuReference() {
        if (lib_) dlclose(lib_);
    }
    CpuReference(const CpuReference&) = delete;
    CpuReference& operator=(const CpuReference&) = delete;
    bool available() const { return f32_ && f16_; }

    // The workload's fp64 reference on its contiguous cache (f32 or f16 values as stored).
    void run(const Workload& w, float* out, int threads) const {
        const float scale = 1.0f / std::sqrt(float(w.shape.head_dim));
        const float* q = static_cast<const float*>(w.q->host());
        if (w.type == KvType::f16)
            f16_(w.shape, w.lens, w.max_len, q, static_cast<const half_t*>(w.k->host()),
                 static_cast<const half_t*>(w.v->host()), out, scale, threads);
        else
            f32_(w.shape, w.lens, w.max_len, q, static_cast<const float*>(w.k->host()),
                 static_cast<const float*>(w.v->host()), out, scale, threads);
    }

private:
    template <class T>
    using Fn = void (*)(const Shape&, std::span<const int>, int, const float*, const T*, const T*, float*, float, int);
    static constexpr const char* kF32 =
        "_ZN3kvb19attention_referenceIfEEvRKNS_5ShapeESt4spanIKiLm18446744073709551615EEiPKfPKT_SB_Pffi";
    static constexpr const char* kF16 =
        "_ZN3kvb19attention_referenceIDF16_EEvRKNS_5ShapeESt4spanIKiLm18446744073709551615EEiPKfPKT_SB_Pffi";
    void* lib_ = nullptr;
    Fn<float> f32_ = nullptr;
    Fn<half_t> f16_ = nullptr;
};

// ---- shared pieces --------------------------------------------------------------------------------

Workload workload(const Options& o, KvType type, int L, bool varied = false) {
    return Workload(o.shape, type, std::vector<int>(size_t(o.shape.batch), L), uint64_t(L), 3.0f, false, varied,
                    o.dist);
}

// fp64 attention on the GPU over the workload's contiguous cache: the stored values for f32/f16, the
// unquantised fp32 data for i8 (an i8 workload keeps fp32 K and V).
std::vector<float> gpu_fp64(const Workload& w) {
    Buffer out(w.out_floats() * sizeof(float));
    NaiveArgs a = w.naive_args(out);
    if (a.type == KvType::i8) a.type = KvType::f32;
    run_attention_fp64(a);
    const float* p = out.as<float>();
    return std::vector<float>(p, p + w.out_floats());
}

int resolved_part(const Workload& w, int part) { return part ? part : auto_part_tokens(w.shape, w.max_len); }

// ---- modes -----------------------------------------------------------------------------------------

int mode_bw(const Options& o, const GpuTimer& timer) {
    Buffer src(o.bw_bytes / 16 * 16);
    std::fill_n(src.as<float>(), src.size() / sizeof(float), 1.0f);
    const Table t(kBwSchema);
    const Sample s = timer([&] { return run_read_bandwidth(src); });
    t.row()
        .text("impl", "read_bw")
        .count("bytes", (long long)src.size())
        .count("reps", o.reps)
        .fixed("median_us", s.median_us(), 2)
        .fixed("min_us", s.min * 1e3, 2)
        .fixed("max_us", s.max * 1e3, 2)
        .fixed("gbps", gbps(double(src.size()), s), 1)
        .emit();
    return 0;
}

// L<n>_{q,k,v}.f32 (q [B][H][D]; K, V [B][Hkv][L][D]) and L<n>_ref_{f32,f16}.f32 ([B][H][D]), raw
// little-endian fp32, as bench/vs_mlx.py reads them.
int mode_dump(const Options& o) {
    auto save = [&](const std::string& file, const void* p, size_t bytes) {
        const std::string path = o.dump + "/" + file;
        FILE* f = std::fopen(path.c_str(), "wb");
        const bool ok = f && std::fwrite(p, 1, bytes, f) == bytes;
        if (f) std::fclose(f);
        if (!ok) std::fprintf(stderr, "cannot write %s\n", path.c_str());
        return ok;
    };
    for (int L : o.lens) {
        const std::string stem = "L" + std::to_string(L) + "_";
        for (KvType type : {KvType::f32, KvType::f16}) {
            const Workload w = workload(o, type, L);
            const std::vector<float> ref = gpu_fp64(w);
            if (!save(stem + "ref_" + name(type) + ".f32", ref.data(), ref.size() * sizeof(float))) return 1;
            if (type != KvType::f32) continue;  // the f16 workload holds the same values rounded
            if (!save(stem + "q.f32", w.q->host(), w.q->size()) || !save(stem + "k.f32", w.k->host(), w.k->size()) ||
                !save(stem + "v.f32", w.v->host(), w.v->size()))
                return 1;
        }
    }
    return 0;
}

// --chain=N: N warm decode steps in one submission (run_paged_steps), wall clock until they complete
// divided by N, for the contiguous layout (one block per sequence) and the paged one (page 16). With
// --graph, the paged chain is also captured once into a HIP graph and replayed (impl ours-graph).
// max_err is against fp64 on the stored values (f32/f16) or the unquantised data (i8).
int mode_chain(const Options& o) {
    const Table t(kChainSchema);
    for (int L : o.lens)
        for (KvType type : o.types) {
            const Workload w = workload(o, type, L);
            const std::vector<float> ref = gpu_fp64(w);
            for (const bool contiguous : {true, false}) {
                const PagedCache cache(w, 16, uint64_t(L) * 131 + 16, contiguous, contiguous ? 1.0 : o.pool, false);
                Buffer out(ref.size() * sizeof(float));
                const PagedArgs args = cache.args(w, o.parts[0], out);
                run_paged(args);
                const double err = max_abs_diff(out.as<float>(), ref.data(), ref.size());
                std::vector<double> wall, gpu;
                for (int i = 0; i < o.warmup + o.reps; ++i) {
                    const auto t0 = Clock::now();
                    const double g = run_paged_steps(args, o.chain);
                    const double ms = std::chrono::duration<double, std::milli>(Clock::now() - t0).count();
                    if (i >= o.warmup) wall.push_back(ms / o.chain), gpu.push_back(g / o.chain);
                }
                const double bytes = double(cache.bytes()) + double(w.out_floats()) * 2 * sizeof(float);
                auto emit = [&](const char* impl, const std::vector<double>& wl, const std::vector<double>& gp,
                                double e) {
                    const Sample s = summarise(wl);
                    t.row()
                        .text("impl", impl)
                        .text("layout", contiguous ? "contiguous" : "paged16")
                        .text("dtype", name(type))
                        .count("batch", w.shape.batch)
                        .count("seq_len", L)
                        .count("chain", o.chain)
                        .count("reps", o.reps)
                        .fixed("median_us", s.median_us(), 2)
                        .fixed("min_us", s.min * 1e3, 2)
                        .fixed("max_us", s.max * 1e3, 2)
                        .fixed("gbps", gbps(bytes, s), 1)
                        .general("max_err", e)
                        .text("err_vs", type == KvType::i8 ? "fp32_data" : "stored")
                        .fixed("gpu_us", summarise(gp).median_us(), 2)
                        .emit();
                };
                emit("ours", wall, gpu, err);
                if (o.graph && !contiguous) {  // the same chain, captured once and replayed
                    PagedGraph graph(args, o.chain);
                    std::vector<double> gwall, ggpu;
                    for (int i = 0; i < o.warmup + o.reps; ++i) {
                        const auto t0 = Clock::now();
                        const double g = graph.launch();
                        const double ms = std::chrono::duration<double, std::milli>(Clock::now() - t0).count();
                        if (i >= o.warmup) gwall.push_back(ms / o.chain), ggpu.push_back(g / o.chain);
                    }
                    emit("ours-graph", gwall, ggpu, max_abs_diff(out.as<float>(), ref.data(), ref.size()));
                }
            }
        }
    return 0;
}

// --accuracy: the paged kernel's error for each storage type against fp64 on the unrounded fp32
// data. The same seed gives every type the same q and fp32 K/V; f16 rounds them, i8 quantises them
// per (block, KV head).
int mode_accuracy(const Options& o) {
    const Table t(kAccuracySchema);
    for (const bool varied : {false, true})
        for (int L : o.lens) {
            const std::vector<float> ref = gpu_fp64(workload(o, KvType::f32, L, varied));
            for (KvType type : o.types)
                for (int page : o.pages) {
                    const Workload w = workload(o, type, L, varied);
                    const PagedCache cache(w, page, uint64_t(L) * 131 + page, false, o.pool, false);
                    Buffer out(ref.size() * sizeof(float));
                    run_paged(cache.args(w, o.parts[0], out));
                    const float* got = out.as<float>();
                    double worst = 0, sq = 0;
                    for (size_t i = 0; i < ref.size(); ++i) {
                        const double e = std::fabs(double(got[i]) - double(ref[i]));
                        worst = std::max(worst, e);
                        sq += e * e;
                    }
                    t.row()
                        .text("data", varied ? "varied" : "uniform")
                        .text("dtype", name(type))
                        .count("seq_len", L)
                        .count("page", page)
                        .general("max_abs_err", worst)
                        .general("rms_err", std::sqrt(sq / double(ref.size())))
                        .emit();
                }
        }
    return 0;
}

// The sweep: per (length, type), the naive kernels and the reference's CPU path on the contiguous
// cache, then the paged step per (page, partition). gbps is min_bytes (live K/V, q and out) over the
// median; max_diff_vs_naive compares outputs with the naive kernels'; kv_bytes is the cache read.
// decode_us and reduce_us time the two-kernel form of the same step (run_paged_split, cold).
int mode_sweep(const Options& o, const GpuTimer& timer, const CpuReference& cpu_ref, int threads) {
    const Table t(kSweepSchema);
    auto timed = [&](const char* impl, const Workload& w, int page, int part, int n, const Sample& s) {
        Table::Row r = t.row();
        r.text("impl", impl)
            .text("dtype", name(w.type))
            .count("batch", w.shape.batch)
            .count("seq_len", w.max_len)
            .count("page", page)
            .count("part", part)
            .count("reps", n)
            .fixed("median_us", s.median_us(), 2)
            .fixed("min_us", s.min * 1e3, 2)
            .fixed("max_us", s.max * 1e3, 2)
            .fixed("gbps", gbps(w.min_bytes(), s), 1);
        return r;
    };
    if (o.cpu && !cpu_ref.available())
        std::printf("# cpu_ref_fp64: no rows (name the reference's kvref shared library with --cpu-ref=LIB)\n");
    for (int L : o.lens)
        for (KvType type : o.types) {
            const Workload w = workload(o, type, L);
            const size_t n = w.out_floats();
            const bool i8 = type == KvType::i8;  // the naive kernels and the CPU rows take f32/f16
            const size_t contig_bytes = w.k->size() + w.v->size();
            Buffer out_naive(n * sizeof(float)), out_paged(n * sizeof(float));
            const bool have_naive = o.naive && !i8;
            if (have_naive)
                timed("gpu_naive", w, 0, 0, o.reps, timer([&] { return run_naive(w.naive_args(out_naive)); }))
                    .general("max_diff_vs_naive", 0)
                    .count("kv_bytes", (long long)contig_bytes)
                    .emit();
            if (o.cpu && cpu_ref.available() && !i8) {
                std::vector<float> out(n);
                std::vector<double> ms;
                for (int i = 0; i <= o.cpu_reps; ++i) {  // the first run warms up
                    const auto t0 = Clock::now();
                    cpu_ref.run(w, out.data(), threads);
                    if (i) ms.push_back(std::chrono::duration<double, std::milli>(Clock::now() - t0).count());
                }
                timed("cpu_ref_fp64", w, 0, 0, o.cpu_reps, summarise(ms))
                    .general("max_diff_vs_naive", have_naive ? max_abs_diff(out.data(), out_naive.as<float>(), n) : NAN)
                    .count("kv_bytes", (long long)contig_bytes)
                    .emit();
            }
            for (int page : o.pages) {
                const PagedCache cache(w, page, uint64_t(L) * 131 + page, false, o.pool, false);
                for (int part : o.parts) {
                    const int p = resolved_part(w, part);
                    const PagedArgs args = cache.args(w, part, out_paged);
                    const Sample s = timer([&] { return run_paged(args); });
                    const double diff = have_naive ? max_abs_diff(out_paged.as<float>(), out_naive.as<float>(), n) : NAN;
                    if (o.flush) flush_gpu_caches();
                    const KernelTimes split = run_paged_split(args);
                    timed("gpu_paged", w, page, p, o.reps, s)
                        .general("max_diff_vs_naive", diff)
                        .count("kv_bytes", (long long)cache.bytes())
                        .fixed("decode_us", split.decode_ms * 1e3, 2)
                        .fixed("reduce_us", split.reduce_ms * 1e3, 2)
                        .emit();
                    if (o.per_head) {
                        PagedArgs one = args;
                        one.share_kv = false;
                        const Sample sp = timer([&] { return run_paged(one); });
                        timed("gpu_paged_per_head", w, page, p, o.reps, sp)
                            .general("max_diff_vs_naive",
                                     have_naive ? max_abs_diff(out_paged.as<float>(), out_naive.as<float>(), n) : NAN)
                            .count("kv_bytes", (long long)cache.bytes())
                            .emit();
                    }
                    if (o.loads && page % 16 == 0 && p % 16 == 0)
                        timed("gpu_paged_loads", w, page, p, o.reps, timer([&] { return run_paged_loads(args); }))
                            .general("max_diff_vs_naive", NAN)
                            .count("kv_bytes", (long long)cache.bytes())
                            .emit();
                }
            }
        }
    return 0;
}

// ---- environment record --------------------------------------------------------------------
// The "# env" header line: the build (build_info.json beside this program, written by the package
// Makefile: commit, dirty flag), the HIP runtime and driver, the ROCm release, the device, the CPU
// and the load average before the run (the reference's scripts/env.sh records the same beside its
// results).

std::string read_file(const std::string& path) {
    std::string out;
    if (FILE* f = std::fopen(path.c_str(), "r")) {
        char buf[4096];
        size_t n;
        while ((n = std::fread(buf, 1, sizeof buf, f)) > 0) out.append(buf, n);
        std::fclose(f);
    }
    return out;
}

// The value of "key" in a flat JSON object as text: a string's contents, or the literal.
std::string json_field(const std::string& text, const std::string& key) {
    const size_t k = text.find("\"" + key + "\"");
    if (k == std::string::npos) return "unknown";
    size_t i = text.find(':', k);
    if (i == std::string::npos) return "unknown";
    i = text.find_first_not_of(" \t\n", i + 1);
    if (i == std::string::npos) return "unknown";
    if (text[i] == '"') {
        const size_t e = text.find('"', i + 1);
        return e == std::string::npos ? "unknown" : text.substr(i + 1, e - i - 1);
    }
    const size_t e = text.find_first_of(",}\n", i);
    return text.substr(i, e == std::string::npos ? std::string::npos : e - i);
}

std::string trim(std::string s) {
    while (!s.empty() && (s.back() == '\n' || s.back() == ' ')) s.pop_back();
    return s;
}

void print_env(const std::string& loadavg, int threads) {
    char exe[4096] = {0};
    const ssize_t n = readlink("/proc/self/exe", exe, sizeof exe - 1);
    std::string dir = n > 0 ? std::string(exe, size_t(n)) : std::string();
    dir = dir.substr(0, dir.find_last_of('/') + 1);
    const std::string built = read_file(dir + "build_info.json");
    std::string cpu = "unknown";
    const std::string info = read_file("/proc/cpuinfo");
    if (const size_t m = info.find("model name"); m != std::string::npos) {
        const size_t c = info.find(':', m), e = info.find('\n', m);
        if (c != std::string::npos && c < e) cpu = info.substr(c + 2, e - c - 2);
    }
    kvb_device_info_t d{};
    const bool dev = kvb_device_info(&d) == KVB_OK;
    std::printf("# env commit=%s dirty=%s built_at=%s hipcc=%s hip_runtime=%d hip_driver=%d rocm=%s device=\"%s\" "
                "arch=%s pci=%s cus=%d sclk_mhz=%d mclk_mhz=%d hbm_gib=%.1f cpu=\"%s\" cpu_threads=%d loadavg=%s\n",
                json_field(built, "commit").c_str(), json_field(built, "dirty").c_str(),
                json_field(built, "built_at").c_str(), json_field(built, "hipcc").c_str(), dev ? d.runtime_version : 0,
                dev ? d.driver_version : 0, trim(read_file("/opt/rocm/.info/version")).c_str(), d.name, d.arch,
                d.pci_bus_id, d.compute_units, d.clock_khz / 1000, d.memory_clock_khz / 1000,
                double(d.total_memory) / double(1ull << 30), cpu.c_str(), threads, loadavg.c_str());
}

}  // namespace

int main(int argc, char** argv) {
    std::string loadavg = trim(read_file("/proc/loadavg"));  // before this run adds its own load
    loadavg = loadavg.substr(0, loadavg.find(' ', loadavg.find(' ', loadavg.find(' ') + 1) + 1));
    for (char& ch : loadavg)
        if (ch == ' ') ch = ',';
    Options o;
    if (!parse(argc, argv, o) || !apply_config(o)) return 2;
    if (o.parts.empty() || o.reps < 1 || o.warmup < 0 || o.cpu_reps < 1 || o.merge < 0) {
        std::fprintf(stderr, "--parts needs a value; --reps and --cpu-reps at least 1, --warmup at least 0; "
                             "--merge is auto, fused or separate\n");
        return 2;
    }
    if (o.schema) {  // each mode's CSV header, "mode:header" (needs no GPU)
        for (const Schema* s : {&kSweepSchema, &kBwSchema, &kChainSchema, &kAccuracySchema})
            std::printf("%s:%s\n", s->mode, s->header().c_str());
        return 0;
    }
    if (!gpu_available()) {
        std::fprintf(stderr, "no GPU\n");
        return 1;
    }
    const int threads = int(std::max(1u, std::thread::hardware_concurrency()));
    std::printf("# device=%s batch=%d heads=%d kv_heads=%d head_dim=%d reps=%d warmup=%d cpu_reps=%d cpu_threads=%d "
                "flush=%d simdgroups=%d timing=%s dist=%s pool=%.2f merge=%s\n",
                device_name().c_str(), o.shape.batch, o.shape.num_heads, o.shape.num_kv_heads, o.shape.head_dim,
                o.reps, o.warmup, o.cpu_reps, threads, o.flush, kSimdGroups, o.sync ? "sync" : "pipelined",
                o.dist == Dist::normal ? "normal" : "uniform", o.pool,
                o.merge == KVB_MERGE_FUSED ? "fused" : o.merge == KVB_MERGE_SEPARATE ? "separate" : "auto");
    print_env(loadavg, threads);
    kvb_set_merge_mode(o.merge);
    const GpuTimer timer(o);
    if (o.bw) return mode_bw(o, timer);
    if (!o.dump.empty()) return mode_dump(o);
    if (o.chain > 0) return mode_chain(o);
    if (o.accuracy) return mode_accuracy(o);
    const CpuReference cpu_ref(o.cpu ? o.cpu_ref : std::string());
    return mode_sweep(o, timer, cpu_ref, threads);
}
