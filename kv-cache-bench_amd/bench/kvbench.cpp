// Decode-step benchmark on MI355X: the paged fused kernels vs the naive 3-pass kernels, CSV on
// stdout (the reference's bench/bench.cpp, GPU side). GPU time is a hipEvent pair around each
// step; caches are flushed (1 GiB streaming read) before every timed run unless --no-flush; runs are
// queued back to back (pipelined) unless --sync; the median of --reps runs is reported.
// --chain=N times N back-to-back steps per submission with warm caches (run_paged_steps).
// --loads adds a gpu_paged_loads row: the decode's loads alone, no arithmetic (run_paged_loads).
// --bw runs the read-bandwidth probe. --config=c1..c4 selects a BASELINE configuration (N(0,1)
// data, its page, partition and pool). --accuracy instead prints the error of the paged kernel for
// each storage type against the fp64 attention of the unrounded fp32 data; --dump=DIR writes the
// inputs and fp64 outputs as raw little-endian fp32 files (the reference's bench/bench.cpp:126-215).
// The fp64 outputs come from the GPU fp64 reference (run_attention_fp64). The fp64 CPU leg is timed
// by bench.py's cpu_baseline.
#include <algorithm>
#include <cmath>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <string>

#include "kvb/workload.hpp"

using namespace kvb;

namespace {

std::vector<int> parse_ints(const char* s) {
    std::vector<int> v;
    for (const char* p = s; *p;) {
        v.push_back(std::atoi(p));
        p = std::strchr(p, ',');
        if (!p) break;
        ++p;
    }
    return v;
}

struct Stats {
    double median, min, max;
};

Stats stats(std::vector<double> t) {
    if (t.empty()) return {0, 0, 0};
    std::sort(t.begin(), t.end());
    const size_t n = t.size();
    return {n % 2 ? t[n / 2] : (t[n / 2 - 1] + t[n / 2]) / 2, t.front(), t.back()};
}

}  // namespace

int main(int argc, char** argv) {
    Shape shape{2, 32, 8, 128};
    std::vector<int> lens{512, 1024, 2048, 4096, 8192, 16384, 32768}, pages{16, 32, 64, 128}, parts{0};
    std::vector<KvType> types{KvType::f32, KvType::f16, KvType::i8};
    int reps = 30, warmup = 3, chain = 0;
    bool naive = true, flush = true, per_head = false, bw = false, sync = false, accuracy = false, loads = false;
    std::string dump;
    Dist dist = Dist::uniform;
    double pool = 1.0;
    std::string config;
    size_t bw_bytes = size_t(4) << 30;
    for (int i = 1; i < argc; ++i) {
        const char* a = argv[i];
        auto val = [&](const char* key) -> const char* {
            const size_t n = std::strlen(key);
            return std::strncmp(a, key, n) == 0 && a[n] == '=' ? a + n + 1 : nullptr;
        };
        if (auto v = val("--batch")) shape.batch = std::atoi(v);
        else if (auto v = val("--heads")) shape.num_heads = std::atoi(v);
        else if (auto v = val("--kv-heads")) shape.num_kv_heads = std::atoi(v);
        else if (auto v = val("--dim")) shape.head_dim = std::atoi(v);
        else if (auto v = val("--lens")) lens = parse_ints(v);
        else if (auto v = val("--pages")) pages = parse_ints(v);
        else if (auto v = val("--parts")) parts = parse_ints(v);
        else if (auto v = val("--reps")) reps = std::atoi(v);
        else if (auto v = val("--warmup")) warmup = std::atoi(v);
        else if (auto v = val("--chain")) chain = std::atoi(v);
        else if (auto v = val("--pool")) pool = std::atof(v);
        else if (auto v = val("--bw-bytes")) bw_bytes = size_t(std::atof(v));
        else if (auto v = val("--dist")) dist = std::strcmp(v, "normal") == 0 ? Dist::normal : Dist::uniform;
        else if (auto v = val("--config")) config = v;
        else if (auto v = val("--types")) {
            types.clear();
            for (KvType t : {KvType::f32, KvType::f16, KvType::i8})
                if (std::strstr(v, name(t))) types.push_back(t);
        } else if (!std::strcmp(a, "--no-naive")) naive = false;
        else if (!std::strcmp(a, "--no-flush")) flush = false;
        else if (!std::strcmp(a, "--per-head")) per_head = true;
        else if (!std::strcmp(a, "--loads")) loads = true;
        else if (!std::strcmp(a, "--bw")) bw = true;
        else if (!std::strcmp(a, "--sync")) sync = true;
        else if (!std::strcmp(a, "--accuracy")) accuracy = true;
        else if (auto v = val("--dump")) dump = v;
        else {
            std::fprintf(stderr, "unknown argument %s\n", a);
            return 2;
        }
    }
    // The BASELINE configurations (fixed lengths; c5's ragged batch is bench.py's).
    if (config == "c1") shape = {1, 32, 8, 128}, lens = {512}, pages = {16}, parts = {128}, types = {KvType::f32}, pool = 2.0, dist = Dist::normal;
    else if (config == "c2") shape = {8, 32, 8, 128}, lens = {4096}, pages = {16}, parts = {512}, types = {KvType::f16}, pool = 1.5, dist = Dist::normal;
    else if (config == "c3") shape = {16, 32, 8, 128}, lens = {8192}, pages = {64}, parts = {mi355x_part_tokens({16, 32, 8, 128}, 8192, mi355x_min_groups(KvType::i8, 128))}, types = {KvType::i8}, pool = 1.0, dist = Dist::normal;
    else if (config == "c4") shape = {4, 64, 8, 128}, lens = {32768}, pages = {128}, parts = {mi355x_part_tokens({4, 64, 8, 128}, 32768)}, types = {KvType::f16}, pool = 1.25, dist = Dist::normal;
    else if (!config.empty()) {
        std::fprintf(stderr, "unknown config %s (c1..c4)\n", config.c_str());
        return 2;
    }
    if (!gpu_available()) {
        std::fprintf(stderr, "no GPU\n");
        return 1;
    }
    std::printf("# device=%s batch=%d heads=%d kv_heads=%d head_dim=%d reps=%d warmup=%d flush=%d waves=%d timing=%s dist=%s pool=%.2f\n",
                device_name().c_str(), shape.batch, shape.num_heads, shape.num_kv_heads, shape.head_dim, reps, warmup,
                flush, kSimdGroups, sync ? "sync" : "pipelined", dist == Dist::normal ? "normal" : "uniform", pool);

    auto time_gpu = [&](const std::function<double()>& run) {
        if (sync) {
            for (int i = 0; i < warmup; ++i) run();
            std::vector<double> t;
            for (int i = 0; i < reps; ++i) {
                if (flush) flush_gpu_caches();
                t.push_back(run());
            }
            return stats(t);
        }
        begin_pipelined();
        for (int i = 0; i < warmup; ++i) run();
        for (int i = 0; i < reps; ++i) {
            if (flush) flush_gpu_caches();
            run();
        }
        std::vector<double> t = end_pipelined();
        t.erase(t.begin(), t.begin() + std::min<size_t>(t.size(), size_t(warmup)));
        return stats(t);
    };
    if (bw) {
        Buffer src(bw_bytes);
        std::fill_n(src.as<float>(), src.size() / 4, 1.0f);
        std::printf("impl,bytes,reps,median_us,min_us,max_us,gbps\n");
        const Stats s = time_gpu([&] { return run_read_bandwidth(src); });
        std::printf("read_bw,%zu,%d,%.2f,%.2f,%.2f,%.1f\n", src.size(), reps, s.median * 1e3, s.min * 1e3, s.max * 1e3,
                    double(src.size()) / (s.median * 1e-3) / 1e9);
        return 0;
    }
    // fp64 attention of a workload's contiguous cache (f32/f16 values as stored)
    auto reference = [&](const Workload& w) {
        Buffer out(w.out_floats() * sizeof(float));
        run_attention_fp64(w.naive_args(out));
        return std::vector<float>(out.as<float>(), out.as<float>() + w.out_floats());
    };
    if (!dump.empty()) {  // L<n>_{q,k,v}.f32: q [B][H][D], K, V [B][Hkv][L][D]; L<n>_ref_{f32,f16}.f32: [B][H][D]
        auto write = [&](const std::string& file, const void* p, size_t bytes) {
            FILE* f = std::fopen((dump + "/" + file).c_str(), "wb");
            const bool ok = f && std::fwrite(p, 1, bytes, f) == bytes;
            if (f) std::fclose(f);
            if (!ok) {
                std::fprintf(stderr, "cannot write %s/%s\n", dump.c_str(), file.c_str());
                std::exit(1);
            }
        };
        for (int L : lens) {
            const std::string pre = "L" + std::to_string(L) + "_";
            for (KvType type : {KvType::f32, KvType::f16}) {
                const Workload w(shape, type, std::vector<int>(size_t(shape.batch), L), uint64_t(L), 3.0f, false, false, dist);
                const std::vector<float> ref = reference(w);
                write(pre + "ref_" + name(type) + ".f32", ref.data(), ref.size() * sizeof(float));
                if (type == KvType::f32) {  // the f16 workload holds these values rounded to fp16
                    write(pre + "q.f32", w.q->host(), w.q->size());
                    write(pre + "k.f32", w.k->host(), w.k->size());
                    write(pre + "v.f32", w.v->host(), w.v->size());
                }
            }
        }
        return 0;
    }
    if (accuracy) {  // same seed = same q and fp32 K/V for every type; f16 rounds them, i8 quantizes per block
        std::printf("data,dtype,seq_len,page,max_abs_err,rms_err\n");
        for (bool varied : {false, true})
            for (int L : lens) {
                const std::vector<int> ls(size_t(shape.batch), L);
                const Workload exact(shape, KvType::f32, ls, uint64_t(L), 3.0f, false, varied, dist);
                const std::vector<float> ref = reference(exact);
                for (KvType type : types)
                    for (int page : pages) {
                        const Workload w(shape, type, ls, uint64_t(L), 3.0f, false, varied, dist);
                        const PagedCache cache(w, page, uint64_t(L) * 131 + page, false, pool, false);
                        Buffer out(ref.size() * sizeof(float));
                        run_paged(cache.args(w, parts[0], out));
                        double mx = 0, sq = 0;
                        for (size_t i = 0; i < ref.size(); ++i) {
                            const double e = std::fabs(double(out.as<float>()[i]) - ref[i]);
                            mx = std::max(mx, e), sq += e * e;
                        }
                        std::printf("%s,%s,%d,%d,%.3g,%.3g\n", varied ? "varied" : "uniform", name(type), L, page, mx,
                                    std::sqrt(sq / double(ref.size())));
                        std::fflush(stdout);
                    }
            }
        return 0;
    }
    if (chain) {  // warm, back-to-back steps in one submission
        std::printf("impl,layout,dtype,batch,seq_len,page,part,chain,reps,median_us,min_us,max_us,gbps\n");
        for (int L : lens)
            for (KvType type : types)
                for (int page : pages)
                    for (int part : parts) {
                        const Workload w(shape, type, std::vector<int>(size_t(shape.batch), L), uint64_t(L), 3.0f, false, false, dist);
                        const PagedCache cache(w, page, uint64_t(L) * 131 + page, false, pool, false);
                        Buffer out(w.out_floats() * sizeof(float));
                        run_paged(cache.args(w, part, out));
                        std::vector<double> t;
                        for (int i = 0; i < warmup + reps; ++i) {
                            const double ms = run_paged_steps(cache.args(w, part, out), chain) / chain;
                            if (i >= warmup) t.push_back(ms);
                        }
                        const Stats st = stats(t);
                        std::printf("gpu_paged_chain,paged%d,%s,%d,%d,%d,%d,%d,%d,%.2f,%.2f,%.2f,%.1f\n", page, name(type),
                                    shape.batch, L, page, part ? part : auto_part_tokens(w.shape, w.max_len), chain, reps,
                                    st.median * 1e3, st.min * 1e3, st.max * 1e3, w.min_bytes() / (st.median * 1e-3) / 1e9);
                        std::fflush(stdout);
                    }
        return 0;
    }
    std::printf("impl,dtype,batch,seq_len,page,part,reps,median_us,min_us,max_us,gbps,decode_us,reduce_us,max_diff_vs_naive,kv_bytes\n");
    auto row = [&](const char* impl, const Workload& w, int page, int part, Stats s, KernelTimes kt, double diff,
                   size_t kv_bytes) {
        std::printf("%s,%s,%d,%d,%d,%d,%d,%.2f,%.2f,%.2f,%.1f,%.2f,%.2f,%.3g,%zu\n", impl, name(w.type), w.shape.batch,
                    w.max_len, page, part, reps, s.median * 1e3, s.min * 1e3, s.max * 1e3,
                    w.min_bytes() / (s.median * 1e-3) / 1e9, kt.decode_ms * 1e3, kt.reduce_ms * 1e3, diff, kv_bytes);
        std::fflush(stdout);
    };
    for (int L : lens)
        for (KvType type : types) {
            const Workload w(shape, type, std::vector<int>(size_t(shape.batch), L), uint64_t(L), 3.0f, false, false, dist);
            const size_t n = w.out_floats();
            Buffer out_naive(n * sizeof(float)), out_paged(n * sizeof(float));
            const bool i8 = type == KvType::i8;
            const size_t contig_bytes = w.k->size() + w.v->size();
            if (naive && !i8)
                row("gpu_naive", w, 0, 0, time_gpu([&] { return run_naive(w.naive_args(out_naive)); }), {}, 0, contig_bytes);
            for (int page : pages) {
                const PagedCache cache(w, page, uint64_t(L) * 131 + page, false, pool, false);
                for (int part : parts) {
                    const Stats s = time_gpu([&] { return run_paged(cache.args(w, part, out_paged)); });
                    if (flush) flush_gpu_caches();
                    const KernelTimes kt = run_paged_split(cache.args(w, part, out_paged));
                    const double diff = naive && !i8 ? max_abs_diff(out_paged.as<float>(), out_naive.as<float>(), n) : NAN;
                    const int p = part ? part : auto_part_tokens(w.shape, w.max_len);
                    row("gpu_paged", w, page, p, s, kt, diff, cache.bytes());
                    if (loads && page % 16 == 0 && p % 16 == 0)
                        row("gpu_paged_loads", w, page, p, time_gpu([&] { return run_paged_loads(cache.args(w, part, out_paged)); }),
                            {}, NAN, cache.bytes());
                    if (per_head) {
                        PagedArgs args = cache.args(w, part, out_paged);
                        args.share_kv = false;
                        row("gpu_paged_per_head", w, page, p, time_gpu([&] { return run_paged(args); }), {}, NAN,
                            cache.bytes());
                    }
                }
            }
        }
    return 0;
}
