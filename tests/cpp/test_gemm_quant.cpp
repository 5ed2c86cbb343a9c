// Quantized GEMMs through the lh:: drop-in (GPU): the reference suite's
// checks (tests/test_gemm_quant.cpp:31-138, same names, seeds and bounds) and
// parity with the CPU oracle's restatement of gemm_quant.cpp: W8A8 bit-exact,
// W4A16 within relative Frobenius 1e-4, FP8 within 1e-5.
#include <gtest/gtest.h>

#include <cmath>
#include <cstdint>
#include <vector>

#include "kernels/gemm.hpp"
#include "kernels/gemm_quant.hpp"
#include "kernels/quant.hpp"
#include "oracle.hpp"
#include "test_util.hpp"

namespace {

double rms(const std::vector<float>& a, const std::vector<float>& b) {
    double s = 0.0;
    for (size_t i = 0; i < a.size(); ++i) {
        const double d = static_cast<double>(a[i]) - b[i];
        s += d * d;
    }
    return std::sqrt(s / a.size());
}
double rms(const std::vector<float>& a) {
    double s = 0.0;
    for (double x : a) s += x * x;
    return std::sqrt(s / a.size());
}

}  // namespace

TEST(GemmQuant, W8A8MatchesFp32WithinTolerance) {
    constexpr int M = 32, N = 48, K = 64;
    auto A = lh_test::random_vector(M * K, 5000, -1.0f, 1.0f);
    auto B = lh_test::random_vector(K * N, 5001, -1.0f, 1.0f);
    std::vector<float> C_fp32(M * N, 0.0f);
    lh::gemm(A.data(), B.data(), C_fp32.data(), M, N, K);
    std::vector<int8_t> Aq(M * K), Bq(K * N);
    std::vector<float> A_s(M), B_s(N);
    lh::q8_quantize_per_row(A.data(), Aq.data(), A_s.data(), M, K);
    lh::q8_quantize_per_col(B.data(), Bq.data(), B_s.data(), K, N);
    std::vector<float> C_q(M * N, 0.0f);
    lh::gemm_w8a8(Aq.data(), Bq.data(), A_s.data(), B_s.data(), C_q.data(), M, N, K);
    const double rel = rms(C_q, C_fp32) / rms(C_fp32);
    EXPECT_LT(rel, 0.05) << "rel RMS = " << rel;
}

TEST(GemmQuant, W4A16MatchesFp32WithinTolerance) {
    constexpr int M = 16, N = 32, K = 64, G = 32;
    auto A = lh_test::random_vector(M * K, 5100, -1.0f, 1.0f);
    auto B = lh_test::random_vector(K * N, 5101, -1.0f, 1.0f);
    std::vector<float> C_fp32(M * N, 0.0f);
    lh::gemm(A.data(), B.data(), C_fp32.data(), M, N, K);
    std::vector<uint8_t> Bp(K * N / 2);
    std::vector<float> B_s((K / G) * N);
    lh::q4_quantize_groupwise(B.data(), Bp.data(), B_s.data(), K, N, G);
    std::vector<float> C_q(M * N, 0.0f);
    lh::gemm_w4a16_groupwise(A.data(), Bp.data(), B_s.data(), C_q.data(), M, N, K, G);
    const double rel = rms(C_q, C_fp32) / rms(C_fp32);
    EXPECT_LT(rel, 0.10) << "rel RMS = " << rel;
}

TEST(GemmQuant, Fp8MatchesFp32WithinTolerance) {
    constexpr int M = 16, N = 32, K = 64;
    auto A = lh_test::random_vector(M * K, 5200, -1.0f, 1.0f);
    auto B = lh_test::random_vector(K * N, 5201, -1.0f, 1.0f);
    std::vector<float> C_fp32(M * N, 0.0f);
    lh::gemm(A.data(), B.data(), C_fp32.data(), M, N, K);
    std::vector<lh::fp8_e4m3> A8(M * K), B8(K * N);
    float sa = 0.0f, sb = 0.0f;
    lh::fp8_quantize_per_tensor(A.data(), A8.data(), &sa, M * K);
    lh::fp8_quantize_per_tensor(B.data(), B8.data(), &sb, K * N);
    std::vector<float> C_q(M * N, 0.0f);
    lh::gemm_fp8_e4m3(A8.data(), B8.data(), sa, sb, C_q.data(), M, N, K);
    const double rel = rms(C_q, C_fp32) / rms(C_fp32);
    EXPECT_LT(rel, 0.10) << "rel RMS = " << rel;
}

TEST(GemmQuant, W8A8RespectsBeta) {
    constexpr int M = 4, N = 4, K = 4;
    auto A = lh_test::random_vector(M * K, 5300, -1.0f, 1.0f);
    auto B = lh_test::random_vector(K * N, 5301, -1.0f, 1.0f);
    std::vector<float> C0(M * N, 1.5f);
    auto C_fp32 = C0;
    lh::gemm(A.data(), B.data(), C_fp32.data(), M, N, K, 0.5f, 2.0f);
    std::vector<int8_t> Aq(M * K), Bq(K * N);
    std::vector<float> A_s(M), B_s(N);
    lh::q8_quantize_per_row(A.data(), Aq.data(), A_s.data(), M, K);
    lh::q8_quantize_per_col(B.data(), Bq.data(), B_s.data(), K, N);
    auto C_q = C0;
    lh::gemm_w8a8(Aq.data(), Bq.data(), A_s.data(), B_s.data(), C_q.data(), M, N, K, 0.5f, 2.0f);
    EXPECT_LT(rms(C_q, C_fp32) / rms(C_fp32), 0.05);
}

TEST(GemmQuant, W4A16BandwidthBeatsFp16ByMoreThan3x) {
    constexpr int K = 4096, N = 4096;
    for (int G : {32, 64, 128}) {
        const int64_t packed = static_cast<int64_t>(K) * N / 2;
        const int64_t scales = static_cast<int64_t>(K) / G * N * sizeof(float);
        const int64_t fp16 = static_cast<int64_t>(K) * N * 2;
        const double ratio = static_cast<double>(fp16) / (packed + scales);
        EXPECT_GT(ratio, 3.0) << "G=" << G << " ratio=" << ratio;
    }
}

// ---- parity with the oracle ----------------------------------------------

TEST(GemmQuantParity, W8A8BitExactAcrossShapes) {
    struct S { int M, N, K; float alpha, beta; };
    for (const S s : {S{1, 4096, 4096, 1.0f, 0.0f}, S{33, 300, 100, 1.0f, 0.0f}, S{257, 129, 512, 0.5f, 2.0f},
                      S{4, 4, 4, -1.25f, 1.0f}, S{70, 520, 1000, 1.0f, -0.5f}}) {
        auto A = lh_test::random_vector(static_cast<int64_t>(s.M) * s.K, 6000 + s.M, -1.0f, 1.0f);
        auto B = lh_test::random_vector(static_cast<int64_t>(s.K) * s.N, 6001 + s.N, -0.05f, 0.05f);
        std::vector<int8_t> Aq(A.size()), Bq(B.size());
        std::vector<float> As(s.M), Bs(s.N);
        lho_q8_quantize_per_row(A.data(), Aq.data(), As.data(), s.M, s.K);
        lho_q8_quantize_per_col(B.data(), Bq.data(), Bs.data(), s.K, s.N);
        auto C = lh_test::random_vector(static_cast<int64_t>(s.M) * s.N, 6002, -1.0f, 1.0f);
        auto Co = C;
        lh::gemm_w8a8(Aq.data(), Bq.data(), As.data(), Bs.data(), C.data(), s.M, s.N, s.K, s.alpha, s.beta);
        lho_gemm_w8a8(Aq.data(), Bq.data(), As.data(), Bs.data(), Co.data(), s.M, s.N, s.K, s.alpha, s.beta);
        EXPECT_TRUE(lh_test::BitEqual(C, Co)) << "M=" << s.M << " N=" << s.N << " K=" << s.K;
    }
}

TEST(GemmQuantParity, W8A8BetaZeroIgnoresNaN) {
    constexpr int M = 8, N = 16, K = 32;
    auto A = lh_test::random_vector(M * K, 7, -1.0f, 1.0f);
    auto B = lh_test::random_vector(K * N, 8, -1.0f, 1.0f);
    std::vector<int8_t> Aq(A.size()), Bq(B.size());
    std::vector<float> As(M), Bs(N);
    lho_q8_quantize_per_row(A.data(), Aq.data(), As.data(), M, K);
    lho_q8_quantize_per_col(B.data(), Bq.data(), Bs.data(), K, N);
    std::vector<float> C(M * N, std::nanf("")), Co(M * N, 0.0f);
    lh::gemm_w8a8(Aq.data(), Bq.data(), As.data(), Bs.data(), C.data(), M, N, K);
    lho_gemm_w8a8(Aq.data(), Bq.data(), As.data(), Bs.data(), Co.data(), M, N, K, 1.0f, 0.0f);
    EXPECT_TRUE(lh_test::BitEqual(C, Co));
}

TEST(GemmQuantParity, W4A16WithinFrobenius1e4) {
    struct S { int M, N, K, G; float alpha, beta; };
    // G = 16 and 96 are served by the dequantize + fp32 GEMM path
    for (const S s : {S{1, 4096, 4096, 128, 1.0f, 0.0f}, S{16, 96, 256, 32, 1.0f, 0.0f}, S{5, 200, 384, 64, 0.5f, 2.0f},
                      S{40, 64, 1024, 256, -1.0f, 1.0f}, S{3, 48, 64, 16, 1.0f, 0.0f}, S{9, 40, 192, 96, 1.0f, 0.5f},
                      S{2, 24, 96, 32, 2.0f, 0.0f}}) {
        auto A = lh_test::random_vector(static_cast<int64_t>(s.M) * s.K, 7000 + s.M, -1.0f, 1.0f);
        auto W = lh_test::random_vector(static_cast<int64_t>(s.K) * s.N, 7001 + s.K, -0.05f, 0.05f);
        std::vector<uint8_t> Bp(W.size() / 2);
        std::vector<float> Bs(static_cast<size_t>(s.K / s.G) * s.N);
        lho_q4_quantize_groupwise(W.data(), Bp.data(), Bs.data(), s.K, s.N, s.G);
        auto C = lh_test::random_vector(static_cast<int64_t>(s.M) * s.N, 7002, -1.0f, 1.0f);
        auto Co = C;
        lh::gemm_w4a16_groupwise(A.data(), Bp.data(), Bs.data(), C.data(), s.M, s.N, s.K, s.G, s.alpha, s.beta);
        lho_gemm_w4a16_groupwise(A.data(), Bp.data(), Bs.data(), Co.data(), s.M, s.N, s.K, s.G, s.alpha, s.beta);
        const double err = lh_test::rel_frobenius(C, Co);
        EXPECT_LE(err, 1e-4) << "M=" << s.M << " N=" << s.N << " K=" << s.K << " G=" << s.G << " err=" << err;
    }
}

TEST(GemmQuantParity, Fp8WithinFrobenius1e5) {
    struct S { int M, N, K; float alpha, beta; };
    for (const S s : {S{16, 32, 64, 1.0f, 0.0f}, S{100, 300, 512, 0.5f, 2.0f}, S{7, 9, 5, 1.0f, 1.0f}}) {
        auto A = lh_test::random_vector(static_cast<int64_t>(s.M) * s.K, 8000 + s.M, -2.0f, 2.0f);
        auto B = lh_test::random_vector(static_cast<int64_t>(s.K) * s.N, 8001 + s.N, -2.0f, 2.0f);
        std::vector<uint8_t> A8(A.size()), B8(B.size());
        float sa = 0, sb = 0;
        lho_fp8_quantize_per_tensor(A.data(), A8.data(), &sa, A.size());
        lho_fp8_quantize_per_tensor(B.data(), B8.data(), &sb, B.size());
        std::vector<lh::fp8_e4m3> Ae(A8.size()), Be(B8.size());
        for (size_t i = 0; i < A8.size(); ++i) Ae[i] = lh::fp8_e4m3::from_bits(A8[i]);
        for (size_t i = 0; i < B8.size(); ++i) Be[i] = lh::fp8_e4m3::from_bits(B8[i]);
        auto C = lh_test::random_vector(static_cast<int64_t>(s.M) * s.N, 8002, -1.0f, 1.0f);
        auto Co = C;
        lh::gemm_fp8_e4m3(Ae.data(), Be.data(), sa, sb, C.data(), s.M, s.N, s.K, s.alpha, s.beta);
        lho_gemm_fp8_e4m3(A8.data(), B8.data(), sa, sb, Co.data(), s.M, s.N, s.K, s.alpha, s.beta);
        const double err = lh_test::rel_frobenius(C, Co);
        EXPECT_LE(err, 1e-5) << "M=" << s.M << " N=" << s.N << " K=" << s.K << " err=" << err;
    }
}
