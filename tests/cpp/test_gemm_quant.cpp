// Quantized GEMMs through the lh:: drop-in (GPU) against the CPU oracle's
// restatement of gemm_quant.cpp:29-104: W8A8 bit-exact, W4A16 within
// relative Frobenius 1e-4, FP8 within 1e-5.
#include <gtest/gtest.h>

#include <cmath>
#include <cstdint>
#include <limits>
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

// Non-finite activations (+Inf, -Inf, NaN, and +Inf with -Inf in one row)
// give the reference's pattern: +-Inf where the row's infinite products
// agree in sign, NaN where an infinity meets a zero weight or the other
// sign, NaN for a NaN activation; every other row within 1e-4.
TEST(GemmQuantParity, W4A16NonFiniteActivationsFollowReference) {
    const int M = 6, N = 96, K = 256, G = 128;
    auto A = lh_test::uniform(static_cast<int64_t>(M) * K, 7100, -1.0f, 1.0f);
    const float inf = std::numeric_limits<float>::infinity();
    A[1 * K + 3] = inf;
    A[2 * K + 200] = -inf;
    A[3 * K + 17] = std::numeric_limits<float>::quiet_NaN();
    A[4 * K + 5] = inf;
    A[4 * K + 250] = -inf;
    auto W = lh_test::uniform(static_cast<int64_t>(K) * N, 7101, -0.05f, 0.05f);
    std::vector<uint8_t> Bp(W.size() / 2);
    std::vector<float> Bs(static_cast<size_t>(K / G) * N);
    lho_q4_quantize_groupwise(W.data(), Bp.data(), Bs.data(), K, N, G);
    // a zero code under row 1's infinity in some columns: Inf * 0 = NaN there
    for (int n = 0; n < N; n += 7) {
        uint8_t& byte = Bp[static_cast<size_t>(3 / 2) * N + n];
        byte = static_cast<uint8_t>(byte & 0x0f);  // k = 3 is the high nibble: code 0
    }
    std::vector<float> C(static_cast<size_t>(M) * N, 0.0f), Co(C);
    lh::gemm_w4a16_groupwise(A.data(), Bp.data(), Bs.data(), C.data(), M, N, K, G, 1.0f, 0.0f);
    lho_gemm_w4a16_groupwise(A.data(), Bp.data(), Bs.data(), Co.data(), M, N, K, G, 1.0f, 0.0f);
    int nan_seen = 0, inf_seen = 0;
    for (int m = 0; m < M; ++m) {
        std::vector<float> row(C.begin() + m * N, C.begin() + (m + 1) * N), rowo(Co.begin() + m * N, Co.begin() + (m + 1) * N);
        bool finite_row = true;
        for (int n = 0; n < N; ++n) {
            const float g = row[n], w = rowo[n];
            if (std::isnan(w) || std::isinf(w)) finite_row = false;
            if (std::isnan(w)) {
                ++nan_seen;
                EXPECT_TRUE(std::isnan(g)) << "m=" << m << " n=" << n << " got " << g;
            } else if (std::isinf(w)) {
                ++inf_seen;
                EXPECT_EQ(g, w) << "m=" << m << " n=" << n;
            }
        }
        if (finite_row) {
            const double err = lh_test::rel_frobenius(row, rowo);
            EXPECT_LE(err, 1e-4) << "row " << m << " err=" << err;
        }
    }
    EXPECT_GT(nan_seen, 0);
    EXPECT_GT(inf_seen, 0);
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
