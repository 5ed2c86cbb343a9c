// fp32 GEMM drivers through the lh:: drop-in (GPU) against the oracle's
// restatement of gemm.cpp:5-75: single, batched and ragged grouped calls.
#include <gtest/gtest.h>

#include <vector>

#include "kernels/gemm.hpp"
#include "oracle.hpp"
#include "test_util.hpp"

TEST(GemmParity, MatchesOracleWithinFrobenius1e6) {
    struct S { int M, N, K; float alpha, beta; };
    for (const S s : {S{64, 80, 300, 1.0f, 0.0f}, S{1, 513, 700, 0.5f, 2.0f}, S{129, 33, 17, -1.0f, 1.0f}}) {
        auto A = lh_test::uniform(static_cast<int64_t>(s.M) * s.K, 91);
        auto B = lh_test::uniform(static_cast<int64_t>(s.K) * s.N, 92);
        auto C = lh_test::uniform(static_cast<int64_t>(s.M) * s.N, 93);
        auto Co = C, Cr = C, Cro = C;
        lh::gemm(A.data(), B.data(), C.data(), s.M, s.N, s.K, s.alpha, s.beta);
        lho_gemm(A.data(), B.data(), Co.data(), s.M, s.N, s.K, s.alpha, s.beta);
        lh::gemm_ref(A.data(), B.data(), Cr.data(), s.M, s.N, s.K, s.alpha, s.beta);
        lho_gemm_ref(A.data(), B.data(), Cro.data(), s.M, s.N, s.K, s.alpha, s.beta);
        EXPECT_LE(lh_test::rel_frobenius(C, Co), 1e-6) << "M=" << s.M;
        EXPECT_LE(lh_test::rel_frobenius(Cr, Cro), 1e-6) << "M=" << s.M;
    }
}

TEST(GemmParity, BatchedAndGroupedMatchOracle) {
    const int batch = 3, M = 17, K = 45, N = 22;
    auto A = lh_test::uniform(batch * M * K, 94);
    auto B = lh_test::uniform(batch * K * N, 95);
    auto C = lh_test::uniform(batch * M * N, 96);
    auto Co = C;
    lh::gemm_batched(A.data(), B.data(), C.data(), batch, M, N, K, 0.75f, 1.5f);
    lho_gemm_batched(A.data(), B.data(), Co.data(), batch, M, N, K, 0.75f, 1.5f);
    EXPECT_LE(lh_test::rel_frobenius(C, Co), 1e-6);
    // ragged groups, one of them empty in M and one in K (C = beta * C)
    const int Mg[4] = {9, 0, 3, 6}, Kg[4] = {31, 8, 0, 70}, Ng[4] = {5, 7, 4, 33};
    std::vector<std::vector<float>> As, Bs, Cs, Cos;
    for (int g = 0; g < 4; ++g) {
        As.push_back(lh_test::uniform(Mg[g] * Kg[g], 100 + g));
        Bs.push_back(lh_test::uniform(Kg[g] * Ng[g], 110 + g));
        Cs.push_back(lh_test::uniform(Mg[g] * Ng[g], 120 + g));
        Cos.push_back(Cs.back());
    }
    const float *pa[4], *pb[4];
    float *pc[4], *pco[4];
    for (int g = 0; g < 4; ++g) {
        pa[g] = As[g].data();
        pb[g] = Bs[g].data();
        pc[g] = Cs[g].data();
        pco[g] = Cos[g].data();
    }
    lh::gemm_grouped(pa, pb, pc, Mg, Ng, Kg, 4, -1.0f, 0.5f);
    lho_gemm_grouped(pa, pb, pco, Mg, Ng, Kg, 4, -1.0f, 0.5f);
    for (int g = 0; g < 4; ++g) EXPECT_LE(lh_test::rel_frobenius(Cs[g], Cos[g]), 1e-6) << "group " << g;
}
