// GPU kernels against the fp64 oracle over a grid of shapes, lengths, page sizes, storage types
// and seeds (the reference's tests/gpu_tests.cpp:66-166), widened with GQA groups 2 and 8, N(0,1)
// data, and oversized, poisoned pools. Exit code 77 (skipped) when there is no GPU.
#include <cmath>
#include <cstdio>

#include "test_util.hpp"

using namespace kvbt;

namespace {

constexpr double kHalfUnit = 1.0 / 2048;  // fp16 unit roundoff

// The derived storage-error bounds of the reference (tests/gpu_tests.cpp:19-62), from the oracle.
double fp16_storage_bound(const Workload& w) {
    const kvbo_shape s = oshape(w.shape);
    return kvbo_fp16_storage_bound(&s, w.lens.data(), w.max_len, static_cast<const float*>(w.q->host()), w.k32.data(),
                                   w.v32.data());
}

double i8_storage_bound(const Workload& w, const PagedCache& c) {
    const kvbo_shape s = oshape(w.shape);
    return kvbo_i8_storage_bound(&s, w.lens.data(), c.layout.page_size, c.layout.max_blocks,
                                 static_cast<const int32_t*>(c.table->host()), static_cast<const float*>(w.q->host()),
                                 static_cast<const float*>(c.k_scale->host()), static_cast<const float*>(c.v_scale->host()));
}

}  // namespace

int main() {
    if (!gpu_available()) {
        std::puts("SKIP: no GPU on this machine, GPU correctness tests not run");
        return 77;
    }
    std::printf("device: %s\n", device_name().c_str());
    const int threads = hw_threads();
    (void)kHalfUnit;

    // GQA 4 (D 128), MHA with D 64, GQA 8 (D 128), GQA 2 (D 64)
    const Shape shapes[] = {{1, 8, 2, 128}, {1, 4, 4, 64}, {1, 16, 2, 128}, {1, 8, 4, 64}};
    const int lengths[] = {1, 7, 100, 513, 2049, 4097};
    const int pages[] = {16, 32, 64, 128};
    struct SeedCfg {
        uint64_t seed;
        int part_tokens;
        float q_amp;
        Dist dist;
        double pool;
    };
    const SeedCfg seeds[] = {{1, 64, 1.0f, Dist::uniform, 1.0},
                             {2, 256, 8.0f, Dist::uniform, 1.5},
                             {3, 512, 3.0f, Dist::uniform, 2.0},
                             {4, 128, 1.0f, Dist::normal, 3.0}};

    int checks = 0, failed = 0;
    double worst[3] = {0, 0, 0}, worst_storage_ratio = 0, worst_i8_ratio = 0, worst_i8_err = 0;
    auto check = [&](bool ok, const char* what, const Shape& s, int L, KvType t, int page, uint64_t seed, double err,
                     double tol) {
        ++checks;
        if (ok) return;
        ++failed;
        std::printf("FAIL %s H=%d Hkv=%d D=%d L=%d %s page=%d seed=%llu: err %.3g > tol %.3g\n", what, s.num_heads,
                    s.num_kv_heads, s.head_dim, L, name(t), page, (unsigned long long)seed, err, tol);
        std::fflush(stdout);
    };

    for (const Shape& shape : shapes)
        for (int L : lengths) {
            for (KvType type : {KvType::f32, KvType::f16, KvType::i8})
                for (const SeedCfg& sc : seeds) {
                    const bool i8 = type == KvType::i8;
                    const int ti = int(type);
                    // Three sequences of different lengths, none a multiple of every page size. int8 gets
                    // magnitudes that differ per block and head, so a misapplied scale shows.
                    Workload w(shape, type, {L, L / 3 + 1, L + 5}, sc.seed, sc.q_amp, type == KvType::f16, i8, sc.dist);
                    const size_t n = w.out_floats();
                    std::vector<float> ref(n);  // f32, f16: on the stored values; i8: on the fp32 data
                    reference(w, ref.data(), threads);
                    Buffer out(n * sizeof(float));
                    const double tol0 = kernel_tol(w);

                    if (!i8) {  // the naive kernels have no int8 path
                        run_naive(w.naive_args(out));
                        const double err = max_abs_diff(out.as<float>(), ref.data(), n);
                        check(err <= tol0, "naive", w.shape, L, type, 0, sc.seed, err, tol0);
                    }

                    std::vector<float> ref32;
                    double storage_tol = 0;
                    if (type == KvType::f16) {  // oracle on the unrounded fp32 data
                        ref32.resize(n);
                        const kvbo_shape os = oshape(w.shape);
                        kvbo_attention_f32(&os, w.lens.data(), w.max_len, static_cast<const float*>(w.q->host()),
                                           w.k32.data(), w.v32.data(), ref32.data(), softmax_scale(w.shape), threads);
                        storage_tol = fp16_storage_bound(w);
                    }

                    for (int page : pages) {
                        PagedCache cache(w, page, sc.seed * 1000 + page, false, sc.pool, true);
                        std::vector<float> deq;  // i8: oracle on the dequantised values the kernel reads
                        if (i8) deq.resize(n), paged_reference(w, cache, deq.data(), threads);
                        const std::vector<float>& kref = i8 ? deq : ref;
                        const double tol = i8 ? kernel_tol(w, &cache) : tol0;
                        std::fill_n(out.as<float>(), n, NAN);
                        run_paged(cache.args(w, sc.part_tokens, out));
                        double err = max_abs_diff(out.as<float>(), kref.data(), n);
                        check(err <= tol, "paged", w.shape, L, type, page, sc.seed, err, tol);
                        worst[ti] = std::max(worst[ti], err / std::max(1.0, tol / kTolKernel));
                        if (page == 16 && shape.group() > 1) {  // one workgroup per query head
                            PagedArgs args = cache.args(w, sc.part_tokens, out);
                            args.share_kv = false;
                            std::fill_n(out.as<float>(), n, NAN);
                            run_paged(args);
                            const double e = max_abs_diff(out.as<float>(), kref.data(), n);
                            check(e <= tol, "paged-per-head", w.shape, L, type, page, sc.seed, e, tol);
                            std::fill_n(out.as<float>(), n, NAN);
                            run_paged(cache.args(w, sc.part_tokens, out));
                        }
                        if (type == KvType::f16) {
                            const double e32 = max_abs_diff(out.as<float>(), ref32.data(), n);
                            check(e32 <= storage_tol, "paged-f16-vs-f32-data", w.shape, L, type, page, sc.seed, e32,
                                  storage_tol);
                            worst_storage_ratio = std::max(worst_storage_ratio, e32 / storage_tol);
                        }
                        if (i8) {
                            const double e32 = max_abs_diff(out.as<float>(), ref.data(), n);
                            const double b = i8_storage_bound(w, cache) + (tol - kTolKernel);
                            check(e32 <= b, "paged-i8-vs-f32-data", w.shape, L, type, page, sc.seed, e32, b);
                            worst_i8_ratio = std::max(worst_i8_ratio, e32 / b);
                            worst_i8_err = std::max(worst_i8_err, e32);
                        }
                    }
                }
            std::printf("shape H=%d Hkv=%d D=%d L=%d done: %d checks, %d failed\n", shape.num_heads, shape.num_kv_heads,
                        shape.head_dim, L, checks, failed);
            std::fflush(stdout);
        }

    std::printf("max |gpu - ref| / max(1, max|v|): f32 storage %.3g, f16 storage %.3g, i8 storage %.3g (tolerance %.0e)\n",
                worst[0], worst[1], worst[2], kTolKernel);
    std::printf("f16 storage vs fp32 data: worst error / derived bound = %.3f\n", worst_storage_ratio);
    std::printf("i8 storage vs fp32 data: worst error %.3g, worst error / derived bound = %.3f\n", worst_i8_err,
                worst_i8_ratio);
    std::printf("%d checks, %d failed\n", checks, failed);
    return failed ? 1 : 0;
}
