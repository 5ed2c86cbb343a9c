// Quantized GEMMs through the lh:: drop-in (GPU) against the CPU oracle's
// restatement of gemm_quant.cpp:29-104: W8A8 bit-exact, W4A16 within
// relative Frobenius 1e-4, FP8 within 1e-5.
#include <gtest/gtest.h>

#include <cmath>
#include <cstdint>
#include <vector>

#include "kernels/gemm.hpp"
#include "kernels/gemm_quant.hpp"
#include "kernels/quant.hpp"
#include "oracle.hpp"
#include "test_util.hpp"

TEST(GemmQuantParity, W8A8BitExactAcrossShapes) {
    struct S { int M, N, K; float alpha, beta; };
    for (const S s : {S{1, 4096, 4096, 1.0f, 0.0f}, S{33, 300, 100, 1.0f, 0.0f}, S{257, 129, 512, 0.5f, 2.0f},
                      S{4, 4, 4, -1.25f, 1.0f}, S{70, 520, 1000, 1.0f, -0.5f}}) {
        auto A = lh_test::uniform(static_cast<int64_t>(s.M) * s.K, 6000 + s.M, -1.0f, 1.0f);
        auto B = lh_test::uniform(static_cast<int64_t>(s.K) * s.N, 6001 + s.N, -0.05f, 0.05f);
        std::vector<int8_t> Aq(A.size()), Bq(B.size());
        std::vector<float> As(s.M), Bs(s.N);
        lho_q8_quantize_per_row(A.data(), Aq.data(), As.data(), s.M, s.K);
        lho_q8_quantize_per_col(B.data(), Bq.data(), Bs.data(), s.K, s.N);
        auto C = lh_test::uniform(static_cast<int64_t>(s.M) * s.N, 6002, -1.0f, 1.0f);
        auto Co = C;
        lh::gemm_w8a8(Aq.data(), Bq.data(), As.data(), Bs.data(), C.data(), s.M, s.N, s.K, s.alpha, s.beta);
        lho_gemm_w8a8(Aq.data(), Bq.data(), As.data(), Bs.data(), Co.data(), s.M, s.N, s.K, s.alpha, s.beta);
        EXPECT_TRUE(lh_test::BitEqual(C, Co)) << "M=" << s.M << " N=" << s.N << " K=" << s.K;
    }
}

TEST(GemmQuantParity, W8A8BetaZeroIgnoresNaN) {
    constexpr int M = 8, N = 16, K = 32;
    auto A = lh_test::uniform(M * K, 7, -1.0f, 1.0f);
    auto B = lh_test::uniform(K * N, 8, -1.0f, 1.0f);
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
        auto A = lh_test::uniform(static_cast<int64_t>(s.M) * s.K, 7000 + s.M, -1.0f, 1.0f);
        auto W = lh_test::uniform(static_cast<int64_t>(s.K) * s.N, 7001 + s.K, -0.05f, 0.05f);
        std::vector<uint8_t> Bp(W.size() / 2);
        std::vector<float> Bs(static_cast<size_t>(s.K / s.G) * s.N);
        lho_q4_quantize_groupwise(W.data(), Bp.data(), Bs.data(), s.K, s.N, s.G);
        auto C = lh_test::uniform(static_cast<int64_t>(s.M) * s.N, 7002, -1.0f, 1.0f);
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
        auto A = lh_test::uniform(static_cast<int64_t>(s.M) * s.K, 8000 + s.M, -2.0f, 2.0f);
        auto B = lh_test::uniform(static_cast<int64_t>(s.K) * s.N, 8001 + s.N, -2.0f, 2.0f);
        std::vector<uint8_t> A8(A.size()), B8(B.size());
        float sa = 0, sb = 0;
        lho_fp8_quantize_per_tensor(A.data(), A8.data(), &sa, A.size());
        lho_fp8_quantize_per_tensor(B.data(), B8.data(), &sb, B.size());
        std::vector<lh::fp8_e4m3> Ae(A8.size()), Be(B8.size());
        for (size_t i = 0; i < A8.size(); ++i) Ae[i] = lh::fp8_e4m3::from_bits(A8[i]);
        for (size_t i = 0; i < B8.size(); ++i) Be[i] = lh::fp8_e4m3::from_bits(B8[i]);
        auto C = lh_test::uniform(static_cast<int64_t>(s.M) * s.N, 8002, -1.0f, 1.0f);
        auto Co = C;
        lh::gemm_fp8_e4m3(Ae.data(), Be.data(), sa, sb, C.data(), s.M, s.N, s.K, s.alpha, s.beta);
        lho_gemm_fp8_e4m3(A8.data(), B8.data(), sa, sb, Co.data(), s.M, s.N, s.K, s.alpha, s.beta);
        const double err = lh_test::rel_frobenius(C, Co);
        EXPECT_LE(err, 1e-5) << "M=" << s.M << " N=" << s.N << " K=" << s.K << " err=" << err;
    }
}
