// common.hpp -- shared device helpers for the gfx950 quantized-GEMM kernels.
//
// Everything here is written for CDNA4 (gfx950) wave64 execution: MFMA
// operand vector types, bit-exact bf16/fp16/e4m3 conversions that reproduce
// the reference's software dtypes (dtypes.hpp:17-196), and the status
// plumbing of the C ABI (include/longhorn_hip.h).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdlib>

#include "longhorn_hip.h"
#include "w4layout.hpp"

namespace lhq {

// ---------------------------------------------------------------------------
// MFMA operand types (verified lane layouts, gfx950):
//   16x16xK: lane l holds row/col (l & 15), K-slice (l >> 4);
//            D element j of lane l is D[4*(l>>4) + j][l & 15].
//   32x32xK: lane l holds row/col (l & 31), K-slice (l >> 5);
//            D element j of lane l is D[8*(j>>2) + 4*(l>>5) + (j&3)][l & 31].
// ---------------------------------------------------------------------------
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;
typedef __attribute__((ext_vector_type(16))) float f32x16_t;
typedef __attribute__((ext_vector_type(4))) int i32x4_t;
typedef __attribute__((ext_vector_type(16))) int i32x16_t;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4_t;
typedef __attribute__((ext_vector_type(2))) uint32_t u32x2_t;

__device__ __forceinline__ f32x4_t mfma_bf16_16x16x32(u32x4_t a, u32x4_t b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}
__device__ __forceinline__ f32x16_t mfma_bf16_32x32x16(u32x4_t a, u32x4_t b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}
__device__ __forceinline__ i32x16_t mfma_i8_32x32x32(u32x4_t a, u32x4_t b, i32x16_t c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(i32x4_t, a),
                                                 __builtin_bit_cast(i32x4_t, b), c, 0, 0, 0);
}
__device__ __forceinline__ i32x4_t mfma_i8_16x16x64(u32x4_t a, u32x4_t b, i32x4_t c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(i32x4_t, a),
                                                 __builtin_bit_cast(i32x4_t, b), c, 0, 0, 0);
}
// gfx950's 32x32x64 MFMA of the f8f6f4 family with both operands e4m3
// (format 0) and unit block scales (E8M0 127 = 2^0): 32 bytes of k per lane,
// given here as two 16-byte halves.
typedef __attribute__((ext_vector_type(8))) int i32x8_t;
__device__ __forceinline__ f32x16_t mfma_fp8_32x32x64(u32x4_t a_lo, u32x4_t a_hi, u32x4_t b_lo, u32x4_t b_hi,
                                                      f32x16_t c) {
    const i32x8_t a = __builtin_bit_cast(i32x8_t, __builtin_shufflevector(a_lo, a_hi, 0, 1, 2, 3, 4, 5, 6, 7));
    const i32x8_t b = __builtin_bit_cast(i32x8_t, __builtin_shufflevector(b_lo, b_hi, 0, 1, 2, 3, 4, 5, 6, 7));
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 127, 0, 127);
}
__device__ __forceinline__ f32x4_t mfma_fp8_16x16x32(u32x2_t a, u32x2_t b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_fp8_fp8(__builtin_bit_cast(long, a),
                                                      __builtin_bit_cast(long, b), c, 0, 0, 0);
}

// ---------------------------------------------------------------------------
// Bit-exact conversions (same results as the reference software dtypes).
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
    return __uint_as_float(static_cast<uint32_t>(b) << 16);
}
// The reference's fp32 -> bf16 rule (dtypes.hpp:87-98): round to nearest
// even on the dropped 16 bits; NaN keeps its payload with the quiet bit set.
__device__ __forceinline__ uint32_t bf16_rule(uint32_t x) {
    const uint32_t rounded = (x + 0x7fffu + ((x >> 16) & 1u)) >> 16;
    const uint32_t quiet = (x >> 16) | 0x40u;
    return ((x & 0x7fffffffu) > 0x7f800000u) ? quiet : rounded;
}
// The same conversion on gfx950's v_cvt_pk_bf16_f32, which gives the rule's
// result for every one of the 2^32 fp32 inputs (lhq_selftest_bf16 checks
// this exhaustively on the device): one instruction per pair instead of
// seven per element.
typedef float lhq_f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 lhq_bf16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(lhq_f32x2{a, b}, lhq_bf16x2));
}
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}
// binary16 -> fp32 (exact for every encoding; dtypes.hpp:57-85).
__device__ __forceinline__ float f16_to_f32(uint16_t h) {
    return static_cast<float>(__builtin_bit_cast(_Float16, h));
}

// fp32 -> E4M3 with the reference's rules (dtypes.hpp:111-158): NaN/inf ->
// 0x7f, saturation to 0x7e above 448, flush to zero below 2^-9.
__device__ __forceinline__ uint32_t rne_shift_u32(uint32_t v, int sh) {
    uint32_t kept = v >> sh;
    uint32_t dropped = v & ((1u << sh) - 1u);
    uint32_t half = 1u << (sh - 1);
    if (dropped > half || (dropped == half && (kept & 1u))) kept += 1u;
    return kept;
}
__device__ __forceinline__ uint8_t f32_to_e4m3(float value) {
    uint32_t x = __float_as_uint(value);
    uint32_t s = (x >> 24) & 0x80u;
    uint32_t e8 = (x >> 23) & 0xffu;
    uint32_t m = x & 0x7fffffu;
    if (e8 == 0xffu) return static_cast<uint8_t>(s | 0x7fu);
    int e = static_cast<int>(e8) - 120;
    if (e > 15 || (e == 15 && m > 0x600000u)) return static_cast<uint8_t>(s | 0x7eu);
    if (e >= 1) {
        uint32_t code = (static_cast<uint32_t>(e) << 3) | (m >> 20);
        uint32_t low = m & 0xfffffu;
        if (low > 0x80000u || (low == 0x80000u && (code & 1u))) {
            code += 1u;
            if (code >= 0x80u && (code >> 3) > 15u) return static_cast<uint8_t>(s | 0x7eu);
        }
        return static_cast<uint8_t>(s | (code & 0x7fu));
    }
    if (e < -2) return static_cast<uint8_t>(s);
    return static_cast<uint8_t>(s | (rne_shift_u32(m | 0x800000u, 21 - e) & 0x7fu));
}
// E4M3 -> fp32 (dtypes.hpp:160-196).
__device__ __forceinline__ float e4m3_to_f32(uint8_t b) {
    uint32_t s = (b & 0x80u) ? 0x80000000u : 0u;
    uint32_t e = (b >> 3) & 0xfu;
    uint32_t m = b & 7u;
    if (e == 0xfu && m == 7u) return __uint_as_float(s | 0x7fc00000u);
    if (e == 0) return __uint_as_float(s | __float_as_uint(static_cast<float>(m) * 0x1p-9f));
    return __uint_as_float(s | ((e + 120u) << 23) | (m << 20));
}

// Saturating round to a symmetric integer range (quant.cpp:12-19, 117-124):
// clamp first, then round-to-nearest-even; NaN converts to 0 on both sides.
__device__ __forceinline__ int sat_rint(float v, int lim) {
    if (v >= static_cast<float>(lim)) return lim;
    if (v <= static_cast<float>(-lim)) return -lim;
    return static_cast<int>(__builtin_rintf(v));
}

// ---------------------------------------------------------------------------
// Prepacked W4 layout (shared by prepack and GEMM kernels).
//
//   qweight  [Nt][Kt][64 lanes][16 B]       Nt = ceil(N/16), Kt = ceil(K/128)
//     A 1 KiB tile covers 16 columns x 128 k.  Lane l owns column
//     16*nt + (l & 15) and, in dword j (0..3), the eight k values
//     128*kt + 32*j + 8*(l >> 4) + e (e = 0..7): exactly the B operand of one
//     16x16x32 MFMA.  Element e sits in nibble w4_slot(e): elements 0..3 in
//     the low nibbles of bytes 0..3, elements 4..7 in their high nibbles, so
//     one mask exposes four codes as whole bytes (see w4_operand).
//   scales   [Nt][NG][16]  fp32 (symmetric) or fp16 (asymmetric), NG = K/G
//   zeros    [Nt][ceil(NG/8)][16] u32, group g in nibble g % 8 (asymmetric)
// Codes are unsigned: symmetric int4 q in [-7,7] is stored as q + 8 with an
// implied zero point of 8.
// ---------------------------------------------------------------------------
__host__ __device__ inline int ceil_div(int a, int b) { return (a + b - 1) / b; }
__host__ __device__ inline int64_t ceil_div64(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Nibble index (bits 4*slot .. 4*slot+3 of the lane's dword) of operand
// element e of a prepacked W4 dword.
__host__ __device__ constexpr int w4_slot(int e) { return e < 4 ? 2 * e : 2 * (e - 4) + 1; }

// The codes enter the MFMA as the exact bf16 integers 128 + u: high byte
// 0x43 (exponent 2^7), code in mantissa bits 0..3.
constexpr float kW4Bias = 128.0f;

// One prepacked dword (eight 4-bit codes) -> the four bf16 pairs of a
// 16x16x32 MFMA B operand: 2 masks, 1 shift and 4 byte permutes.
// __builtin_amdgcn_perm(hi, lo, sel) picks result byte i from the eight
// bytes {lo: 0..3, hi: 4..7} named by byte i of sel.
__device__ __forceinline__ u32x4_t w4_operand(uint32_t d) {
    const uint32_t lo = d & 0x0F0F0F0Fu;         // codes of elements 0..3
    const uint32_t hi = (d >> 4) & 0x0F0F0F0Fu;  // codes of elements 4..7
    constexpr uint32_t kExp = 0x43434343u;
    u32x4_t b;
    b[0] = __builtin_amdgcn_perm(kExp, lo, 0x04010400u);  // {e0, e1}
    b[1] = __builtin_amdgcn_perm(kExp, lo, 0x04030402u);  // {e2, e3}
    b[2] = __builtin_amdgcn_perm(kExp, hi, 0x04010400u);  // {e4, e5}
    b[3] = __builtin_amdgcn_perm(kExp, hi, 0x04030402u);  // {e6, e7}
    return b;
}

// The same with the zero point folded in: zb holds 16 - z in each byte, so
// every code byte becomes u + 16 - z (1..31, no carry between bytes) and the
// operands are the exact bf16 integers 144 + u - z.
__device__ __forceinline__ u32x4_t w4_operand_z(uint32_t d, uint32_t zb) {
    const uint32_t lo = (d & 0x0F0F0F0Fu) + zb;
    const uint32_t hi = ((d >> 4) & 0x0F0F0F0Fu) + zb;
    constexpr uint32_t kExp = 0x43434343u;
    u32x4_t b;
    b[0] = __builtin_amdgcn_perm(kExp, lo, 0x04010400u);
    b[1] = __builtin_amdgcn_perm(kExp, lo, 0x04030402u);
    b[2] = __builtin_amdgcn_perm(kExp, hi, 0x04010400u);
    b[3] = __builtin_amdgcn_perm(kExp, hi, 0x04030402u);
    return b;
}

}  // namespace lhq

// ---------------------------------------------------------------------------
// Host-side status plumbing (defined in capi.cpp).
// ---------------------------------------------------------------------------
namespace lhq {
// Tuning knobs (kernel choice and launch shape overrides, LHQ_W4_* and
// LHQ_GEMM8_*) are read from the environment only in a build made with
// -DLHQ_TUNING_KNOBS (make TUNING=1), for sweeps.  The product library
// ignores the environment and always runs the tested heuristic.
inline int tuning_knob(const char* name, int dflt) {
#ifdef LHQ_TUNING_KNOBS
    const char* v = std::getenv(name);
    return v ? std::atoi(v) : dflt;
#else
    (void)name;
    return dflt;
#endif
}
int set_error(int code, const char* fmt, ...);
int check_launch(const char* what);
inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }
}  // namespace lhq

#define LHQ_REQUIRE(cond, ...)                                              \
    do {                                                                    \
        if (!(cond)) return ::lhq::set_error(LHQ_ERR_INVALID, __VA_ARGS__); \
    } while (0)
#define LHQ_SUPPORTED(cond, ...)                                                \
    do {                                                                        \
        if (!(cond)) return ::lhq::set_error(LHQ_ERR_UNSUPPORTED, __VA_ARGS__); \
    } while (0)
