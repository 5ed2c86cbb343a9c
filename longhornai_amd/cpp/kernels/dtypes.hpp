// kernels/dtypes.hpp -- the 16- and 8-bit storage types of LonghornAI's
// kernel headers, for the MI355X drop-in backend.
//
// Same types and functions as the reference (src/kernels/dtypes.hpp:13-336):
// lh::half, lh::bfloat16, lh::fp8_e4m3, lh::fp8_e5m2, each a bit container
// that converts from and to float, and lh::detail::float_to_*_bits /
// *_bits_to_float.  They are host-side value types here (the GPU kernels
// convert on the device with the same rules).
//
// Conversion rules (the reference's, dtypes.hpp:17-269):
//   fp32 -> fp16 / bf16 / e5m2 / e4m3: round to nearest, ties to even.
//   fp16: overflow -> inf, NaN -> 0x7e00 | sign.
//   bf16: NaN keeps its payload with the quiet bit set.
//   e5m2: overflow -> inf (0x7c | sign), NaN -> 0x7f | sign.
//   e4m3 (no infinities): NaN and inf -> 0x7f | sign; |x| > 448 -> 0x7e | sign
//     (448); |x| < 2^-9 -> signed zero, including the interval where
//     round-to-nearest would give the smallest subnormal 2^-9.
//
// Implementation: one narrowing routine parameterised by the target format
// (exponent bits, mantissa bits, overflow policy) instead of one hand-written
// routine per type.
#ifndef LONGHORN_MI355X_KERNELS_DTYPES_HPP
#define LONGHORN_MI355X_KERNELS_DTYPES_HPP

#include <cstdint>
#include <cstring>

namespace lh {

namespace detail {

inline uint32_t f32_bits(float f) {
    uint32_t u;
    std::memcpy(&u, &f, sizeof(u));
    return u;
}
inline float bits_f32(uint32_t u) {
    float f;
    std::memcpy(&f, &u, sizeof(f));
    return f;
}

// Target format description for the narrowing conversion.
struct NarrowFormat {
    int exp_bits;          // exponent field width
    int man_bits;          // stored mantissa width
    uint32_t inf_code;     // code (without sign) for overflow
    uint32_t nan_code;     // code (without sign) for NaN (and inf when !has_inf)
    bool has_inf;          // inf input maps to inf_code (else nan_code)
    uint32_t max_finite;   // largest code (without sign) a rounding may reach
    int min_keep_exp;      // biased target exponents below this flush to zero
};

// fp32 -> a narrower binary float, round to nearest even on the magnitude.
inline uint32_t narrow(float value, const NarrowFormat& f) {
    const uint32_t x = f32_bits(value);
    const uint32_t sign = (x >> 31) << (f.exp_bits + f.man_bits);
    const uint32_t e32 = (x >> 23) & 0xffu;
    const uint32_t m32 = x & 0x7fffffu;
    if (e32 == 0xffu) {
        if (m32 != 0 || !f.has_inf) return sign | f.nan_code;
        return sign | f.inf_code;
    }
    const int bias = (1 << (f.exp_bits - 1)) - 1;
    const int e = static_cast<int>(e32) - 127 + bias;  // target biased exponent
    if (e < f.min_keep_exp) return sign;                // flushes (and fp32 zero / tiny)
    // Significand with the hidden bit (fp32 subnormals are far below every
    // target format's range and flushed above).
    const uint64_t sig = static_cast<uint64_t>(m32) | 0x800000u;
    // Number of fp32 significand bits dropped: normal targets keep man_bits,
    // subnormal targets (e <= 0) lose 1 - e more.
    const int drop = (23 - f.man_bits) + (e <= 0 ? 1 - e : 0);
    if (drop > 24) return sign;  // below half of the smallest subnormal
    uint64_t kept = sig >> drop;
    const uint64_t rem = sig & ((uint64_t{1} << drop) - 1);
    const uint64_t halfway = uint64_t{1} << (drop - 1);
    if (rem > halfway || (rem == halfway && (kept & 1u))) ++kept;
    // Reassemble: for normal targets the hidden bit of `kept` lands on the
    // exponent field's lowest bit, so adding the exponent folds a mantissa
    // carry into the exponent; subnormal results keep exponent field 0.
    uint64_t code = (e <= 0) ? kept : ((static_cast<uint64_t>(e - 1) << f.man_bits) + kept);
    if (code > f.max_finite) return sign | f.inf_code;
    return sign | static_cast<uint32_t>(code);
}

// A narrower binary float -> fp32 (exact).
inline float widen(uint32_t code, int exp_bits, int man_bits, bool has_inf, uint32_t nan_code) {
    const int width = exp_bits + man_bits;
    const uint32_t sign = ((code >> width) & 1u) << 31;
    const uint32_t mag = code & ((1u << width) - 1u);
    const uint32_t e = mag >> man_bits;
    const uint32_t m = mag & ((1u << man_bits) - 1u);
    const int bias = (1 << (exp_bits - 1)) - 1;
    // IEEE-like formats: inf, or NaN with the payload moved up (quiet bit
    // not forced); formats without infinities have one NaN code -> qNaN
    if (has_inf && e == (1u << exp_bits) - 1u) return bits_f32(sign | 0x7f800000u | (m << (23 - man_bits)));
    if (!has_inf && mag == nan_code) return bits_f32(sign | 0x7fc00000u);
    if (e == 0) {
        // subnormal: m * 2^(1 - bias - man_bits), exact in fp32
        const float v = static_cast<float>(m) * bits_f32(static_cast<uint32_t>(127 + 1 - bias - man_bits) << 23);
        return bits_f32(sign | f32_bits(v));
    }
    return bits_f32(sign | ((e - bias + 127) << 23) | (m << (23 - man_bits)));
}

// binary16: 5 exponent bits, 10 mantissa bits, IEEE infinities.
constexpr NarrowFormat kHalf{5, 10, 0x7c00u, 0x7e00u, true, 0x7bffu, -10};
// OCP E5M2: IEEE-like, infinities at 0x7c.
constexpr NarrowFormat kE5M2{5, 2, 0x7cu, 0x7fu, true, 0x7bu, -1};
// OCP E4M3 as the reference defines it: no infinities, 0x7e (448) is the
// largest finite value and every overflow saturates to it; exponents that
// would give |x| < 2^-9 flush to zero.
constexpr NarrowFormat kE4M3{4, 3, 0x7eu, 0x7fu, false, 0x7eu, -2};

inline uint16_t float_to_half_bits(float value) {
    // values that round above 65504 become inf (IEEE binary16 overflow)
    return static_cast<uint16_t>(narrow(value, kHalf));
}
inline float half_bits_to_float(uint16_t h) { return widen(h, 5, 10, true, 0x7e00u); }

inline uint16_t float_to_bf16_bits(float value) {
    const uint32_t x = f32_bits(value);
    if ((x & 0x7f800000u) == 0x7f800000u && (x & 0x7fffffu) != 0)
        return static_cast<uint16_t>((x >> 16) | 0x40u);  // quiet NaN, payload kept
    const uint32_t rounded = x + 0x7fffu + ((x >> 16) & 1u);
    return static_cast<uint16_t>(rounded >> 16);
}
inline float bf16_bits_to_float(uint16_t b) { return bits_f32(static_cast<uint32_t>(b) << 16); }

inline uint8_t float_to_e4m3_bits(float value) { return static_cast<uint8_t>(narrow(value, kE4M3)); }
inline float e4m3_bits_to_float(uint8_t b) { return widen(b, 4, 3, false, 0x7fu); }

inline uint8_t float_to_e5m2_bits(float value) { return static_cast<uint8_t>(narrow(value, kE5M2)); }
inline float e5m2_bits_to_float(uint8_t b) { return widen(b, 5, 2, true, 0x7fu); }

}  // namespace detail

// IEEE-754 binary16.
struct half {
    uint16_t bits = 0;
    half() = default;
    half(float v) : bits(detail::float_to_half_bits(v)) {}  // NOLINT(runtime/explicit)
    float to_float() const { return detail::half_bits_to_float(bits); }
    operator float() const { return to_float(); }
    static half from_bits(uint16_t b) {
        half h;
        h.bits = b;
        return h;
    }
};

// Brain floating point: the upper 16 bits of an fp32, rounded.
struct bfloat16 {
    uint16_t bits = 0;
    bfloat16() = default;
    bfloat16(float v) : bits(detail::float_to_bf16_bits(v)) {}  // NOLINT(runtime/explicit)
    float to_float() const { return detail::bf16_bits_to_float(bits); }
    operator float() const { return to_float(); }
    static bfloat16 from_bits(uint16_t b) {
        bfloat16 v;
        v.bits = b;
        return v;
    }
};

// FP8 E4M3 (no infinities, saturating).
struct fp8_e4m3 {
    uint8_t bits = 0;
    fp8_e4m3() = default;
    fp8_e4m3(float v) : bits(detail::float_to_e4m3_bits(v)) {}  // NOLINT(runtime/explicit)
    float to_float() const { return detail::e4m3_bits_to_float(bits); }
    operator float() const { return to_float(); }
    static fp8_e4m3 from_bits(uint8_t b) {
        fp8_e4m3 v;
        v.bits = b;
        return v;
    }
};

// FP8 E5M2 (IEEE-like, with infinities).
struct fp8_e5m2 {
    uint8_t bits = 0;
    fp8_e5m2() = default;
    fp8_e5m2(float v) : bits(detail::float_to_e5m2_bits(v)) {}  // NOLINT(runtime/explicit)
    float to_float() const { return detail::e5m2_bits_to_float(bits); }
    operator float() const { return to_float(); }
    static fp8_e5m2 from_bits(uint8_t b) {
        fp8_e5m2 v;
        v.bits = b;
        return v;
    }
};

}  // namespace lh

#endif  // LONGHORN_MI355X_KERNELS_DTYPES_HPP
