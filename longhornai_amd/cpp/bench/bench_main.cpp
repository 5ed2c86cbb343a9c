// bench_main.cpp -- benchmark driver for the quantized-GEMM family on MI355X.
//
// The reference's driver (bench/bench_main.cpp) registers named specs with
// their FLOP and byte counts in a BenchSuite, runs them with a host clock,
// prints a table and a roofline view and optionally writes CSVs (--csv,
// --roofline).  This driver does the same for the quantized path, with a
// HIP timing mode:
//   --timing hip  (default) device-resident buffers through the C ABI
//                 (include/longhorn_hip.h), timed with HIP events on the
//                 launch stream; the BASELINE configurations, with weight
//                 sets rotated so that every launch streams its weights from
//                 HBM (more than twice the 256 MB Infinity Cache in flight).
//   --timing host the synchronous lh:: drop-in (kernels/gemm_quant.hpp,
//                 quant.hpp, gemm.hpp) timed with steady_clock, as the
//                 reference times its kernels; every call includes the
//                 host<->device copies and the weight prepack.
// Other options: --filter SUBSTR, --iters N, --warmup N, --csv PATH,
// --roofline PATH.  Inputs are synthetic (seeded mt19937): random int4 /
// int8 codes and scales, N(0,1) activations.
#include <hip/hip_runtime_api.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <iostream>
#include <memory>
#include <random>
#include <string>
#include <vector>

#include "bench_util.hpp"
#include "kernels/dtypes.hpp"
#include "kernels/gemm.hpp"
#include "kernels/gemm_quant.hpp"
#include "kernels/quant.hpp"
#include "longhorn_hip.h"

namespace {

constexpr double kRotateBytes = 2.0 * 256e6 + 64e6;  // > 2 x Infinity Cache

[[noreturn]] void die(const std::string& what) {
    std::fprintf(stderr, "lh_bench: %s\n", what.c_str());
    std::exit(1);
}

void check(int st, const char* what) {
    if (st != LHQ_OK) die(std::string(what) + ": " + lhq_status_string(st) + ": " + lhq_last_error());
}

// Device allocation owned by the benchmark (freed at exit).
struct DevBuf {
    void* p = nullptr;
    explicit DevBuf(size_t bytes) {
        if (hipMalloc(&p, bytes ? bytes : 1) != hipSuccess) die("hipMalloc of " + std::to_string(bytes) + " bytes");
    }
    ~DevBuf() { (void)hipFree(p); }
    DevBuf(const DevBuf&) = delete;
    DevBuf& operator=(const DevBuf&) = delete;
    template <class T> T* as() const { return static_cast<T*>(p); }
};
using Dev = std::shared_ptr<DevBuf>;

Dev upload(const void* host, size_t bytes) {
    auto d = std::make_shared<DevBuf>(bytes);
    if (hipMemcpy(d->p, host, bytes, hipMemcpyHostToDevice) != hipSuccess) die("hipMemcpy H2D");
    return d;
}

std::vector<uint8_t> rand_bytes(size_t n, uint32_t seed, uint8_t mask = 0xFF) {
    std::mt19937 rng(seed);
    std::vector<uint8_t> v(n);
    size_t i = 0;
    for (; i + 4 <= n; i += 4) {
        const uint32_t r = rng();
        for (int b = 0; b < 4; ++b) v[i + b] = static_cast<uint8_t>(r >> (8 * b)) & mask;
    }
    for (; i < n; ++i) v[i] = static_cast<uint8_t>(rng()) & mask;
    return v;
}

std::vector<uint16_t> rand_bf16(size_t n, uint32_t seed) {
    std::mt19937 rng(seed);
    std::normal_distribution<float> d(0.0f, 1.0f);
    std::vector<uint16_t> v(n);
    for (auto& x : v) x = lh::bfloat16(d(rng)).bits;
    return v;
}

std::vector<float> rand_f32(size_t n, uint32_t seed, float lo = -1.0f, float hi = 1.0f) {
    std::mt19937 rng(seed);
    std::uniform_real_distribution<float> d(lo, hi);
    std::vector<float> v(n);
    for (auto& x : v) x = d(rng);
    return v;
}

// ---- W4A16 (asymmetric int4, fp16 scale + u4 zero per group) --------------
struct W4Set {
    Dev qw, sc, zs;
};

double w4_bytes(int M, int K, int N, int G) {
    return double(K) * N / 2 + double(K / G) * N * 2 + double(K / G) * N / 2 + 2.0 * M * K + 2.0 * M * N;
}

// `n` prepacked weight sets of one shape (same random codes, separate
// buffers: the rotation is about where the bytes live, not their values).
std::vector<W4Set> make_w4_sets(int K, int N, int G, int n, uint32_t seed) {
    const size_t ng = size_t(K / G) * N;
    const auto packed = rand_bytes(size_t(K / 2) * N, seed);
    std::vector<uint16_t> sc(ng);
    std::mt19937 rng(seed + 1);
    std::uniform_real_distribution<float> d(0.002f, 0.01f);
    for (auto& s : sc) s = lh::half(d(rng)).bits;
    const auto zeros = rand_bytes(ng, seed + 2, 0x0F);
    auto dp = upload(packed.data(), packed.size());
    auto ds = upload(sc.data(), sc.size() * 2);
    auto dz = upload(zeros.data(), zeros.size());
    std::vector<W4Set> sets;
    for (int i = 0; i < n; ++i) {
        W4Set w{std::make_shared<DevBuf>(lhq_w4_qweight_bytes(K, N)),
                std::make_shared<DevBuf>(lhq_w4_scales_bytes(K, N, G, 1)),
                std::make_shared<DevBuf>(lhq_w4_zeros_bytes(K, N, G))};
        check(lhq_w4_prepack_asym(dp->as<uint8_t>(), ds->as<uint16_t>(), dz->as<uint8_t>(), K, N, G,
                                  w.qw->as<uint8_t>(), w.sc->as<uint16_t>(), w.zs->as<uint32_t>(), nullptr),
              "lhq_w4_prepack_asym");
        sets.push_back(std::move(w));
    }
    if (hipDeviceSynchronize() != hipSuccess) die("prepack");
    return sets;
}

void add_w4(lh_bench::BenchSuite& suite, const std::string& tag, int M, int K, int N, int G, int iters) {
    const double per = w4_bytes(M, K, N, G);
    const int nsets = std::max(2, int(std::ceil(kRotateBytes / per)));
    auto sets = std::make_shared<std::vector<W4Set>>(make_w4_sets(K, N, G, nsets, 1000 + K + N));
    auto A = upload(rand_bf16(size_t(M) * K, 7).data(), size_t(M) * K * 2);
    auto C = std::make_shared<DevBuf>(size_t(M) * N * 2);
    lh_bench::BenchSpec s;
    s.name = tag + "[" + std::to_string(M) + "x" + std::to_string(K) + "x" + std::to_string(N) + "]";
    s.flops = 2.0 * M * K * N;
    s.bytes = per;
    s.peak_flops = lh_bench::kBf16PeakFlops;
    s.iters = iters;
    s.dev_fn = [=](hipStream_t st, int i) {
        const W4Set& w = (*sets)[i % sets->size()];
        check(lhq_gemm_w4a16_bf16(A->as<uint16_t>(), w.qw->as<uint8_t>(), w.sc->as<uint16_t>(),
                                  w.zs->as<uint32_t>(), C->as<uint16_t>(), M, N, K, G, st),
              "lhq_gemm_w4a16_bf16");
    };
    suite.add(std::move(s));
}

// Config 4: 512 tokens, top-2 distinct of 8 experts, one grouped launch.
void add_moe(lh_bench::BenchSuite& suite) {
    const int T = 512, E = 8, K = 4096, N = 14336, G = 128;  // top-2 routing below
    std::mt19937 rng(4);
    std::vector<int> counts(E, 0);
    for (int t = 0; t < T; ++t) {
        int a = rng() % E, b = rng() % (E - 1);
        if (b >= a) ++b;  // distinct second expert
        ++counts[a];
        ++counts[b];
    }
    std::vector<int32_t> off(E + 1, 0);
    for (int e = 0; e < E; ++e) off[e + 1] = off[e] + counts[e];
    const int rows = off[E];
    auto sets = std::make_shared<std::vector<W4Set>>(make_w4_sets(K, N, G, E, 44));
    std::vector<const void*> q(E), sc(E), zs(E);
    for (int e = 0; e < E; ++e) {
        q[e] = (*sets)[e].qw->p;
        sc[e] = (*sets)[e].sc->p;
        zs[e] = (*sets)[e].zs->p;
    }
    auto dq = upload(q.data(), E * sizeof(void*));
    auto dsc = upload(sc.data(), E * sizeof(void*));
    auto dzs = upload(zs.data(), E * sizeof(void*));
    auto doff = upload(off.data(), off.size() * 4);
    auto A = upload(rand_bf16(size_t(rows) * K, 8).data(), size_t(rows) * K * 2);
    auto C = std::make_shared<DevBuf>(size_t(rows) * N * 2);
    lh_bench::BenchSpec s;
    s.name = "moe_grouped_w4a16[512tok top2 of 8, 4096x14336]";
    s.flops = 2.0 * rows * K * N;
    s.bytes = E * (w4_bytes(0, K, N, G)) + 2.0 * rows * K + 2.0 * rows * N;
    s.peak_flops = lh_bench::kBf16PeakFlops;
    s.iters = 50;
    // the launch only sees the weights through the device pointer tables:
    // `keep` holds the buffers they point to for as long as the spec lives
    s.dev_fn = [=, keep = sets](hipStream_t st, int) {
        check(lhq_gemm_w4a16_bf16_grouped(A->as<uint16_t>(), doff->as<int32_t>(),
                                          dq->as<const uint8_t* const>(), dsc->as<const uint16_t* const>(),
                                          dzs->as<const uint32_t* const>(), C->as<uint16_t>(), E, rows, N, K, G, st),
              "lhq_gemm_w4a16_bf16_grouped");
    };
    suite.add(std::move(s));
}

// ---- W8A8 ------------------------------------------------------------------
// Config 3 (bf16 out, activations already quantized) and config 1 (M = 1
// GEMV through the reference path: per-row quantization of fp32 A, then
// gemm_w8a8 with fp32 C; one step = both launches).
void add_w8(lh_bench::BenchSuite& suite, int M, int K, int N, bool gemv_c1, int iters) {
    const auto bq = rand_bytes(size_t(K) * N, 300 + M);
    std::vector<int8_t> b8(bq.size());
    for (size_t i = 0; i < bq.size(); ++i) b8[i] = static_cast<int8_t>(int(bq[i] % 255) - 127);
    auto Bq = upload(b8.data(), b8.size());
    const int64_t btb = lhq_b8_prepacked_bytes(K, N);
    const int nsets = gemv_c1 ? std::max(2, int(std::ceil(kRotateBytes / double(btb)))) : 1;
    auto Bt = std::make_shared<std::vector<Dev>>();
    for (int i = 0; i < nsets; ++i) {
        Bt->push_back(std::make_shared<DevBuf>(btb));
        check(lhq_b8_prepack(Bq->as<uint8_t>(), K, N, Bt->back()->as<uint8_t>(), nullptr), "lhq_b8_prepack");
    }
    if (hipDeviceSynchronize() != hipSuccess) die("b8 prepack");  // Bq is freed on return
    auto Bs = upload(rand_f32(N, 301, 0.001f, 0.01f).data(), size_t(N) * 4);
    auto As = std::make_shared<DevBuf>(size_t(M) * 4);
    auto Aq = std::make_shared<DevBuf>(size_t(M) * K);
    lh_bench::BenchSpec s;
    s.flops = 2.0 * M * K * N;
    s.peak_flops = lh_bench::kInt8PeakOps;
    s.iters = iters;
    if (gemv_c1) {
        auto A = upload(rand_f32(size_t(M) * K, 302).data(), size_t(M) * K * 4);
        auto C = std::make_shared<DevBuf>(size_t(M) * N * 4);
        s.name = "w8a8/c1_gemv_f32[" + std::to_string(M) + "x" + std::to_string(K) + "x" + std::to_string(N) + "]";
        s.bytes = double(K) * N + 4.0 * N + 4.0 * M * K + 4.0 * M * N;
        s.dev_fn = [=](hipStream_t st, int i) {
            check(lhq_q8_quantize_per_row(A->as<float>(), Aq->as<int8_t>(), As->as<float>(), M, K, st),
                  "lhq_q8_quantize_per_row");
            check(lhq_gemm_w8a8(Aq->as<int8_t>(), (*Bt)[i % Bt->size()]->as<int8_t>(), As->as<float>(),
                                Bs->as<float>(), C->as<float>(), M, N, K, 1.0f, 0.0f, st),
                  "lhq_gemm_w8a8");
        };
    } else {
        auto Ab = upload(rand_bf16(size_t(M) * K, 303).data(), size_t(M) * K * 2);
        check(lhq_q8_quantize_per_row_bf16(Ab->as<uint16_t>(), Aq->as<int8_t>(), As->as<float>(), M, K, nullptr),
              "lhq_q8_quantize_per_row_bf16");
        if (hipDeviceSynchronize() != hipSuccess) die("activation quantization");  // Ab is freed on return
        auto C = std::make_shared<DevBuf>(size_t(M) * N * 2);
        s.name = "w8a8/prefill_bf16[" + std::to_string(M) + "x" + std::to_string(K) + "x" + std::to_string(N) + "]";
        s.bytes = double(M) * K + double(K) * N + 4.0 * (M + N) + 2.0 * M * N;
        s.dev_fn = [=](hipStream_t st, int) {
            check(lhq_gemm_w8a8_bf16(Aq->as<int8_t>(), (*Bt)[0]->as<int8_t>(), As->as<float>(), Bs->as<float>(),
                                     C->as<uint16_t>(), M, N, K, st),
                  "lhq_gemm_w8a8_bf16");
        };
    }
    suite.add(std::move(s));
}

// FP8 e4m3 GEMM (gemm_quant.cpp:87-104) at config 3's shape: random e4m3
// codes below the NaN code, per-tensor scales, fp32 C.
void add_fp8(lh_bench::BenchSuite& suite, int M, int K, int N) {
    auto codes = [](size_t n, uint32_t seed) {
        auto v = rand_bytes(n, seed);
        for (auto& b : v)
            if ((b & 0x7F) == 0x7F) b ^= 1;  // 0x7f / 0xff are NaN in e4m3
        return v;
    };
    auto B = upload(codes(size_t(K) * N, 500).data(), size_t(K) * N);
    auto Bt = std::make_shared<DevBuf>(lhq_b8_prepacked_bytes(K, N));
    check(lhq_b8_prepack(B->as<uint8_t>(), K, N, Bt->as<uint8_t>(), nullptr), "lhq_b8_prepack");
    if (hipDeviceSynchronize() != hipSuccess) die("fp8 prepack");  // B is freed on return
    auto A = upload(codes(size_t(M) * K, 501).data(), size_t(M) * K);
    const float sc[2] = {0.01f, 0.02f};
    auto S = upload(sc, sizeof(sc));
    auto C = std::make_shared<DevBuf>(size_t(M) * N * 4);
    lh_bench::BenchSpec s;
    s.name = "fp8/gemm_e4m3[" + std::to_string(M) + "x" + std::to_string(K) + "x" + std::to_string(N) + "]";
    s.flops = 2.0 * M * K * N;
    s.bytes = double(M) * K + double(K) * N + 4.0 * M * N;
    s.peak_flops = lh_bench::kFp8PeakFlops;
    s.iters = 50;
    s.dev_fn = [=](hipStream_t st, int) {
        check(lhq_gemm_fp8_e4m3(A->as<uint8_t>(), Bt->as<uint8_t>(), S->as<float>(), S->as<float>() + 1,
                                C->as<float>(), M, N, K, 1.0f, 0.0f, st),
              "lhq_gemm_fp8_e4m3");
    };
    suite.add(std::move(s));
}

void add_act_quant(lh_bench::BenchSuite& suite, int M, int K) {
    auto Ab = upload(rand_bf16(size_t(M) * K, 400).data(), size_t(M) * K * 2);
    auto Aq = std::make_shared<DevBuf>(size_t(M) * K);
    auto As = std::make_shared<DevBuf>(size_t(M) * 4);
    lh_bench::BenchSpec s;
    s.name = "quant/q8_per_row_bf16[" + std::to_string(M) + "x" + std::to_string(K) + "]";
    s.bytes = 2.0 * M * K + double(M) * K + 4.0 * M;
    s.iters = 100;
    s.dev_fn = [=](hipStream_t st, int) {
        check(lhq_q8_quantize_per_row_bf16(Ab->as<uint16_t>(), Aq->as<int8_t>(), As->as<float>(), M, K, st),
              "lhq_q8_quantize_per_row_bf16");
    };
    suite.add(std::move(s));
}

// ---- host timing: the synchronous lh:: drop-in ------------------------------
void add_host(lh_bench::BenchSuite& suite) {
    // the reference driver's fp32 GEMM shapes (bench_main.cpp:42-46)
    const int shapes[3][3] = {{128, 768, 768}, {128, 2048, 768}, {128, 768, 2048}};
    const char* tags[3] = {"lh/gemm/qkv_small", "lh/gemm/mlp_up", "lh/gemm/mlp_down"};
    for (int t = 0; t < 3; ++t) {
        const int M = shapes[t][0], N = shapes[t][1], K = shapes[t][2];
        auto A = std::make_shared<std::vector<float>>(rand_f32(size_t(M) * K, 1));
        auto B = std::make_shared<std::vector<float>>(rand_f32(size_t(K) * N, 2));
        auto C = std::make_shared<std::vector<float>>(size_t(M) * N);
        lh_bench::BenchSpec s;
        s.name = std::string(tags[t]) + "[" + std::to_string(M) + "x" + std::to_string(N) + "x" + std::to_string(K) + "]";
        s.flops = 2.0 * M * N * K;
        s.bytes = 4.0 * (double(M) * K + double(K) * N + double(M) * N);
        s.host_fn = [=] { lh::gemm(A->data(), B->data(), C->data(), M, N, K); };
        suite.add(std::move(s));
    }
    {
        const int M = 1, K = 4096, N = 4096;
        auto A = std::make_shared<std::vector<float>>(rand_f32(size_t(M) * K, 3));
        auto W = rand_f32(size_t(K) * N, 4);
        auto Bq = std::make_shared<std::vector<int8_t>>(size_t(K) * N);
        auto Bs = std::make_shared<std::vector<float>>(N);
        lh::q8_quantize_per_col(W.data(), Bq->data(), Bs->data(), K, N);
        auto Aq = std::make_shared<std::vector<int8_t>>(size_t(M) * K);
        auto As = std::make_shared<std::vector<float>>(M);
        auto C = std::make_shared<std::vector<float>>(size_t(M) * N);
        lh_bench::BenchSpec s;
        s.name = "lh/c1_w8_gemv[1x4096x4096]";
        s.flops = 2.0 * M * K * N;
        s.bytes = double(K) * N + 4.0 * N + 4.0 * K + 4.0 * N;
        s.peak_flops = lh_bench::kInt8PeakOps;
        s.host_fn = [=] {
            lh::q8_quantize_per_row(A->data(), Aq->data(), As->data(), M, K);
            lh::gemm_w8a8(Aq->data(), Bq->data(), As->data(), Bs->data(), C->data(), M, N, K);
        };
        suite.add(std::move(s));
    }
    {
        const int M = 1, K = 4096, N = 4096, G = 128;
        auto A = std::make_shared<std::vector<float>>(rand_f32(size_t(M) * K, 5));
        auto W = rand_f32(size_t(K) * N, 6, -0.05f, 0.05f);
        auto P = std::make_shared<std::vector<uint8_t>>(size_t(K / 2) * N);
        auto S = std::make_shared<std::vector<float>>(size_t(K / G) * N);
        lh::q4_quantize_groupwise(W.data(), P->data(), S->data(), K, N, G);
        auto C = std::make_shared<std::vector<float>>(size_t(M) * N);
        lh_bench::BenchSpec s;
        s.name = "lh/gemm_w4a16_groupwise[1x4096x4096 G128]";
        s.flops = 2.0 * M * K * N;
        s.bytes = double(K) * N / 2 + 4.0 * (K / G) * N + 4.0 * K + 4.0 * N;
        s.host_fn = [=] { lh::gemm_w4a16_groupwise(A->data(), P->data(), S->data(), C->data(), M, N, K, G); };
        suite.add(std::move(s));
    }
}

}  // namespace

int main(int argc, char** argv) {
    lh_bench::Timing timing = lh_bench::Timing::Hip;
    std::string filter, csv_path, roofline_path;
    int iters = -1, warmup = -1;
    for (int i = 1; i < argc; ++i) {
        const std::string a = argv[i];
        auto next = [&]() -> std::string {
            if (i + 1 >= argc) die("missing value after " + a);
            return argv[++i];
        };
        if (a == "--timing") {
            const std::string v = next();
            if (v == "hip") timing = lh_bench::Timing::Hip;
            else if (v == "host") timing = lh_bench::Timing::Host;
            else die("--timing takes hip or host");
        } else if (a == "--filter") filter = next();
        else if (a == "--iters") iters = std::atoi(next().c_str());
        else if (a == "--warmup") warmup = std::atoi(next().c_str());
        else if (a == "--csv") csv_path = next();
        else if (a == "--roofline") roofline_path = next();
        else die("unknown option " + a);
    }

    lh_bench::BenchSuite suite;
    auto want = [&](const std::string& name) { return filter.empty() || name.find(filter) != std::string::npos; };
    if (timing == lh_bench::Timing::Hip) {
        // Registration builds device data; skip what the filter excludes.
        if (want("w4a16/decode")) add_w4(suite, "w4a16/decode", 1, 8192, 28672, 128, 200);
        for (int M : {1, 4, 16})
            for (auto kn : {std::pair<int, int>{4096, 4096}, {4096, 11008}, {11008, 4096}})
                if (want("w4a16/c2")) add_w4(suite, "w4a16/c2", M, kn.first, kn.second, 128, 200);
        for (auto kn : {std::pair<int, int>{8192, 10240}, {8192, 8192}, {28672, 8192}})
            if (want("w4a16/c5")) add_w4(suite, "w4a16/c5", 8, kn.first, kn.second, 128, 200);
        if (want("w4a16/c5_prefill")) {
            add_w4(suite, "w4a16/c5_prefill", 64, 8192, 28672, 128, 100);
            add_w4(suite, "w4a16/c5_prefill", 4096, 8192, 28672, 128, 10);
        }
        if (want("moe")) add_moe(suite);
        if (want("w8a8/c1")) add_w8(suite, 1, 4096, 4096, true, 200);
        if (want("w8a8/prefill")) {
            add_w8(suite, 2048, 4096, 14336, false, 50);
            add_w8(suite, 4096, 4096, 14336, false, 50);
        }
        if (want("fp8/")) add_fp8(suite, 4096, 4096, 14336);
        if (want("quant/")) add_act_quant(suite, 4096, 4096);
    } else {
        add_host(suite);
    }
    if (suite.size() == 0) die("no benchmark matches the filter");

    const auto results = suite.run(std::cout, timing, filter, iters, warmup);
    std::cout << "\n";
    lh_bench::print_roofline(std::cout, results);
    if (!csv_path.empty()) std::cout << (lh_bench::write_csv(csv_path, results) ? "wrote " : "failed to write ") << csv_path << "\n";
    if (!roofline_path.empty())
        std::cout << (lh_bench::write_roofline_csv(roofline_path, results) ? "wrote " : "failed to write ")
                  << roofline_path << "\n";
    return results.empty() ? 1 : 0;
}
