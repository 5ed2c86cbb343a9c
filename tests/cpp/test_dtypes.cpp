// lh:: storage types (host-side conversions of the drop-in dtypes.hpp):
// bit-exact agreement with the oracle -- exhaustive for every 16- and 8-bit
// decode, and for encodes over every fp32 bit pattern with a stride, plus all
// fp32 values near each format's rounding boundaries.
#include <gtest/gtest.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <vector>

#include "kernels/dtypes.hpp"
#include "oracle.hpp"
#include "test_util.hpp"

using lh::bfloat16;
using lh::fp8_e4m3;
using lh::fp8_e5m2;
using lh::half;

namespace {
uint32_t fbits(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    return u;
}
float bitsf(uint32_t u) {
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}
// fp32 patterns worth checking exhaustively for a format with `man` mantissa
// bits: for every fp32 exponent, all patterns whose dropped mantissa bits are
// near 0, the halfway point or the top (ties, carries, saturation edges).
template <typename F>
void boundary_sweep(int man, F&& check) {
    const int drop = 23 - man;
    const uint32_t half = 1u << (drop - 1), full = 1u << drop;
    for (uint32_t sign = 0; sign < 2; ++sign)
        for (uint32_t e = 0; e < 256; ++e)
            for (uint32_t keep = 0; keep < (1u << man); ++keep)
                for (uint32_t low : {0u, 1u, half - 1, half, half + 1, full - 1})
                    check(bitsf((sign << 31) | (e << 23) | (keep << drop) | low));
}
}  // namespace

TEST(DtypesParity, DecodeExhaustive) {
    for (uint32_t h = 0; h < 65536; ++h) {
        EXPECT_EQ(fbits(lh::detail::half_bits_to_float(static_cast<uint16_t>(h))),
                  fbits(lho_f16_to_f32(static_cast<uint16_t>(h))))
            << "half " << h;
        EXPECT_EQ(fbits(lh::detail::bf16_bits_to_float(static_cast<uint16_t>(h))),
                  fbits(lho_bf16_to_f32(static_cast<uint16_t>(h))))
            << "bf16 " << h;
    }
    for (uint32_t b = 0; b < 256; ++b) {
        EXPECT_EQ(fbits(lh::detail::e4m3_bits_to_float(static_cast<uint8_t>(b))),
                  fbits(lho_e4m3_to_f32(static_cast<uint8_t>(b))))
            << "e4m3 " << b;
        EXPECT_EQ(fbits(lh::detail::e5m2_bits_to_float(static_cast<uint8_t>(b))),
                  fbits(lho_e5m2_to_f32(static_cast<uint8_t>(b))))
            << "e5m2 " << b;
    }
}

TEST(DtypesParity, EncodeStrided) {
    // every 4099th fp32 bit pattern (~1M values over all signs, exponents,
    // NaNs and infinities), each through all four encoders
    int bad = 0;
    for (uint64_t u = 0; u < (1ull << 32) && bad < 10; u += 4099) {
        const float f = bitsf(static_cast<uint32_t>(u));
        if (lh::detail::float_to_half_bits(f) != lho_f32_to_f16(f) ||
            lh::detail::float_to_bf16_bits(f) != lho_f32_to_bf16(f) ||
            lh::detail::float_to_e4m3_bits(f) != lho_f32_to_e4m3(f) ||
            lh::detail::float_to_e5m2_bits(f) != lho_f32_to_e5m2(f)) {
            ++bad;
            std::printf("encode mismatch at fp32 bits 0x%08x\n", static_cast<unsigned>(u));
        }
    }
    EXPECT_EQ(bad, 0);
}

TEST(DtypesParity, EncodeRoundingBoundaries) {
    int bad = 0;
    boundary_sweep(10, [&](float f) { bad += lh::detail::float_to_half_bits(f) != lho_f32_to_f16(f); });
    boundary_sweep(7, [&](float f) { bad += lh::detail::float_to_bf16_bits(f) != lho_f32_to_bf16(f); });
    boundary_sweep(3, [&](float f) { bad += lh::detail::float_to_e4m3_bits(f) != lho_f32_to_e4m3(f); });
    boundary_sweep(2, [&](float f) { bad += lh::detail::float_to_e5m2_bits(f) != lho_f32_to_e5m2(f); });
    EXPECT_EQ(bad, 0);
}
