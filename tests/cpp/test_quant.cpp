// Quantizers through the lh:: drop-in (GPU): bit-exact parity with the CPU
// oracle's restatement of quant.cpp (quant.cpp:34-249) at every scope.
#include <gtest/gtest.h>

#include <cmath>
#include <cstdint>
#include <vector>

#include "kernels/quant.hpp"
#include "oracle.hpp"
#include "test_util.hpp"

using lh_test::BitEqual;

namespace {
std::vector<float> spiky(int rows, int cols, uint32_t seed) {
    // wide magnitudes, exact zeros, a zero row and +-127 ties (x*inv = k+0.5)
    auto x = lh_test::uniform(static_cast<int64_t>(rows) * cols, seed, -4.0f, 4.0f);
    for (int c = 0; c < cols; ++c) x[c] = 0.0f;                       // all-zero first row
    for (size_t i = 7; i < x.size(); i += 13) x[i] *= 1000.0f;        // outliers
    for (size_t i = 5; i < x.size(); i += 17) x[i] = 0.0f;
    for (size_t i = 3; i < x.size(); i += 29) x[i] = 2.5f;
    return x;
}
}  // namespace

TEST(QuantParity, Q8AllScopesBitExact) {
    const int rows = 37, cols = 129;
    auto x = spiky(rows, cols, 77);
    const size_t n = x.size();
    std::vector<int8_t> q(n), qo(n);
    float s = 0, so = 0;
    lh::q8_quantize_per_tensor(x.data(), q.data(), &s, n);
    lho_q8_quantize_per_tensor(x.data(), qo.data(), &so, n);
    EXPECT_TRUE(BitEqual(q, qo));
    EXPECT_EQ(s, so);
    std::vector<float> sr(rows), sro(rows), sc(cols), sco(cols);
    lh::q8_quantize_per_row(x.data(), q.data(), sr.data(), rows, cols);
    lho_q8_quantize_per_row(x.data(), qo.data(), sro.data(), rows, cols);
    EXPECT_TRUE(BitEqual(q, qo));
    EXPECT_TRUE(BitEqual(sr, sro));
    lh::q8_quantize_per_col(x.data(), q.data(), sc.data(), rows, cols);
    lho_q8_quantize_per_col(x.data(), qo.data(), sco.data(), rows, cols);
    EXPECT_TRUE(BitEqual(q, qo));
    EXPECT_TRUE(BitEqual(sc, sco));
    std::vector<float> d(n), dox(n);
    lh::q8_dequantize_per_col(q.data(), sc.data(), d.data(), rows, cols);
    lho_q8_dequantize_per_col(q.data(), sc.data(), dox.data(), rows, cols);
    EXPECT_TRUE(BitEqual(d, dox));
}

TEST(QuantParity, Q4GroupwiseBitExact) {
    for (int G : {2, 8, 32, 64, 128}) {
        const int K = 256, N = 24;
        auto x = spiky(K, N, 100 + G);
        std::vector<uint8_t> p(K * N / 2), po(K * N / 2);
        std::vector<float> s((K / G) * N), so((K / G) * N);
        lh::q4_quantize_groupwise(x.data(), p.data(), s.data(), K, N, G);
        lho_q4_quantize_groupwise(x.data(), po.data(), so.data(), K, N, G);
        EXPECT_TRUE(BitEqual(p, po)) << "G=" << G;
        EXPECT_TRUE(BitEqual(s, so)) << "G=" << G;
        std::vector<float> d(K * N), dox(K * N);
        lh::q4_dequantize_groupwise(p.data(), s.data(), d.data(), K, N, G);
        lho_q4_dequantize_groupwise(p.data(), s.data(), dox.data(), K, N, G);
        EXPECT_TRUE(BitEqual(d, dox)) << "G=" << G;
    }
}

TEST(QuantParity, Fp8AllScopesBitExact) {
    const int rows = 19, cols = 70;
    auto x = spiky(rows, cols, 99);
    const size_t n = x.size();
    std::vector<lh::fp8_e4m3> q(n);
    std::vector<uint8_t> qo(n), qb(n);
    float s = 0, so = 0;
    auto bits = [&]() { for (size_t i = 0; i < n; ++i) qb[i] = q[i].bits; return qb; };
    lh::fp8_quantize_per_tensor(x.data(), q.data(), &s, n);
    lho_fp8_quantize_per_tensor(x.data(), qo.data(), &so, n);
    EXPECT_TRUE(BitEqual(bits(), qo));
    EXPECT_EQ(s, so);
    std::vector<float> sr(rows), sro(rows), sc(cols), sco(cols);
    lh::fp8_quantize_per_row(x.data(), q.data(), sr.data(), rows, cols);
    lho_fp8_quantize_per_row(x.data(), qo.data(), sro.data(), rows, cols);
    EXPECT_TRUE(BitEqual(bits(), qo));
    EXPECT_TRUE(BitEqual(sr, sro));
    lh::fp8_quantize_per_col(x.data(), q.data(), sc.data(), rows, cols);
    lho_fp8_quantize_per_col(x.data(), qo.data(), sco.data(), rows, cols);
    EXPECT_TRUE(BitEqual(bits(), qo));
    EXPECT_TRUE(BitEqual(sc, sco));
}

TEST(QuantParity, Q4GetAllBytes) {
    // every byte value, both nibbles: the inline unpack matches the oracle
    std::vector<uint8_t> packed(256);
    for (int b = 0; b < 256; ++b) packed[b] = static_cast<uint8_t>(b);
    for (int k = 0; k < 2; ++k)
        for (int n = 0; n < 256; ++n) EXPECT_EQ(+lh::q4_get(packed.data(), k, n, 256), +lho_q4_get(packed.data(), k, n, 256));
}
