// test_moe.cpp -- lh::moe_dispatch / lh::moe_combine (the drop-in, on the GPU)
// bit for bit against the oracle's restatement of moe.cpp:102-221.
#include <gtest/gtest.h>

#include <cstdint>
#include <numeric>
#include <random>
#include <vector>

#include "kernels/moe.hpp"
#include "oracle.hpp"
#include "test_util.hpp"

namespace {

lh::MoEConfig config(int T, int H, int E, int K) {
    lh::MoEConfig c;
    c.n_tokens = T;
    c.hidden_dim = H;
    c.n_experts = E;
    c.top_k = K;
    return c;
}

// top-k distinct experts per token, uniformly
std::vector<int32_t> routing(int T, int E, int K, uint32_t seed) {
    std::mt19937 rng(seed);
    std::vector<int32_t> ids(static_cast<size_t>(T) * K);
    std::vector<int32_t> perm(E);
    for (int t = 0; t < T; ++t) {
        std::iota(perm.begin(), perm.end(), 0);
        std::shuffle(perm.begin(), perm.end(), rng);
        for (int k = 0; k < K; ++k) ids[static_cast<size_t>(t) * K + k] = perm[k];
    }
    return ids;
}

}  // namespace

TEST(MoEParity, DispatchBitExactVsOracle) {
    const int shapes[][4] = {{100, 64, 8, 2}, {37, 5, 16, 4}, {1, 8, 4, 1}, {513, 128, 64, 6}};
    for (const auto& sh : shapes) {
        const int T = sh[0], H = sh[1], E = sh[2], K = sh[3];
        auto hidden = lh_test::uniform(T * H, 7000 + T);
        auto ids = routing(T, E, K, 7100 + T);
        std::vector<int32_t> off(E + 1), tok(T * K), slot(T * K), woff(E + 1), wtok(T * K), wslot(T * K), wpos(T * K);
        std::vector<float> out(static_cast<size_t>(T) * K * H), want(out.size());
        lh::moe_dispatch(hidden.data(), ids.data(), off.data(), tok.data(), slot.data(), out.data(),
                         config(T, H, E, K));
        lho_moe_dispatch(hidden.data(), int64_t{H} * 4, ids.data(), T, K, E, woff.data(), wtok.data(),
                         wslot.data(), wpos.data(), want.data());
        EXPECT_TRUE(lh_test::BitEqual(off, woff)) << "T=" << T;
        EXPECT_TRUE(lh_test::BitEqual(tok, wtok)) << "T=" << T;
        EXPECT_TRUE(lh_test::BitEqual(slot, wslot)) << "T=" << T;
        EXPECT_TRUE(lh_test::BitEqual(out, want)) << "T=" << T;
    }
}

TEST(MoEParity, CombineBitExactVsOracle) {
    const int shapes[][4] = {{100, 64, 8, 2}, {41, 7, 16, 4}, {1, 5000, 2, 2}, {300, 96, 16, 3}};
    for (const auto& sh : shapes) {
        const int T = sh[0], H = sh[1], E = sh[2], K = sh[3];
        auto ids = routing(T, E, K, 8000 + T);
        std::vector<int32_t> off(E + 1), tok(T * K), slot(T * K), pos(T * K);
        lho_moe_dispatch(nullptr, 0, ids.data(), T, K, E, off.data(), tok.data(), slot.data(), pos.data(), nullptr);
        auto y = lh_test::uniform(T * K * H, 8100 + T);
        auto gates = lh_test::uniform(T * K, 8200 + T);
        std::vector<float> got(static_cast<size_t>(T) * H), want(got.size());
        lh::moe_combine(y.data(), off.data(), tok.data(), slot.data(), gates.data(), got.data(), config(T, H, E, K));
        lho_moe_combine_f32(y.data(), tok.data(), slot.data(), gates.data(), want.data(), T, H, K);
        EXPECT_TRUE(lh_test::BitEqual(got, want)) << "T=" << T << " H=" << H;
    }
}

// dispatch -> identity experts -> combine: each token gets sum_k gate_k * x
TEST(MoE, DispatchThenCombineRestoresWeightedTokens) {
    constexpr int T = 64, H = 32, E = 8, K = 2;
    auto hidden = lh_test::uniform(T * H, 9000);
    auto ids = routing(T, E, K, 9001);
    std::vector<float> gates(T * K, 0.5f);  // 0.5 x + 0.5 x == x exactly
    const auto cfg = config(T, H, E, K);
    std::vector<int32_t> off(E + 1), tok(T * K), slot(T * K);
    std::vector<float> xs(static_cast<size_t>(T) * K * H), out(static_cast<size_t>(T) * H);
    lh::moe_dispatch(hidden.data(), ids.data(), off.data(), tok.data(), slot.data(), xs.data(), cfg);
    lh::moe_combine(xs.data(), off.data(), tok.data(), slot.data(), gates.data(), out.data(), cfg);
    EXPECT_TRUE(lh_test::BitEqual(out, hidden));
}
