// kernels/quant.hpp -- quantizers of LonghornAI's quantized-GEMM path, on
// the MI355X backend.
//
// Drop-in for the reference header (src/kernels/quant.hpp:28-94): the same
// functions with the same signatures, host pointers and semantics.  Each
// call copies its inputs to the GPU, runs the gfx950 kernel behind the C ABI
// (include/longhorn_hip.h), copies the result back and returns when it is
// complete.  A HIP failure prints the library's message and aborts; there is
// no CPU code path.
//
// Semantics (bit-exact with the reference, quant.cpp:12-249):
//   int8 symmetric: scale = max|x| / 127 (1 when max|x| == 0);
//     per-tensor and per-row multiply by 1/scale, per-column divides;
//     q = lrintf of the clamped value, in [-127, 127].
//   int4 group-wise: scale = max|w| / 7 per (group of G rows, column) (1 when
//     zero); q = lrintf(w / scale) clamped to [-7, 7]; rows 2i / 2i+1 of
//     column n share byte packed[i*N + n] (low / high nibble).
//   fp8 E4M3: scale = max|x| / 448, then the E4M3 conversion of dtypes.hpp.
#ifndef LONGHORN_MI355X_KERNELS_QUANT_HPP
#define LONGHORN_MI355X_KERNELS_QUANT_HPP

#include <cstddef>
#include <cstdint>

#include "kernels/dtypes.hpp"

namespace lh {

// --- INT8 symmetric (quant.hpp:28-48) --------------------------------------
void q8_quantize_per_tensor(const float* src, int8_t* dst, float* scale_out,
                            int64_t n);
void q8_dequantize_per_tensor(const int8_t* src, float scale, float* dst,
                              int64_t n);

void q8_quantize_per_row(const float* src, int8_t* dst, float* scales_out,
                         int rows, int dim);
void q8_dequantize_per_row(const int8_t* src, const float* scales, float* dst,
                           int rows, int dim);

void q8_quantize_per_col(const float* src, int8_t* dst, float* scales_out,
                         int rows, int cols);
void q8_dequantize_per_col(const int8_t* src, const float* scales, float* dst,
                           int rows, int cols);

// --- INT4 group (packed) (quant.hpp:50-63) ----------------------------------
void q4_quantize_groupwise(const float* src, uint8_t* packed,
                           float* scales_out, int K, int N, int group_size);
void q4_dequantize_groupwise(const uint8_t* packed, const float* scales,
                             float* dst, int K, int N, int group_size);

// The int4 value of row k, column n of a packed [K, N] tensor (quant.hpp:
// 65-75): byte (k/2)*N + n, low nibble for even k, sign-extended from 4 bits.
inline int8_t q4_get(const uint8_t* packed, int k, int n, int N) {
    const uint8_t byte = packed[static_cast<int64_t>(k / 2) * N + n];
    const int nib = (k & 1) ? (byte >> 4) : (byte & 0x0f);
    return static_cast<int8_t>(nib >= 8 ? nib - 16 : nib);
}

// --- FP8 E4M3 (quant.hpp:77-94) ---------------------------------------------
void fp8_quantize_per_tensor(const float* src, fp8_e4m3* dst,
                             float* scale_out, int64_t n);
void fp8_dequantize_per_tensor(const fp8_e4m3* src, float scale, float* dst,
                               int64_t n);

void fp8_quantize_per_row(const float* src, fp8_e4m3* dst, float* scales_out,
                          int rows, int dim);
void fp8_dequantize_per_row(const fp8_e4m3* src, const float* scales,
                            float* dst, int rows, int dim);

void fp8_quantize_per_col(const float* src, fp8_e4m3* dst, float* scales_out,
                          int rows, int cols);
void fp8_dequantize_per_col(const fp8_e4m3* src, const float* scales,
                            float* dst, int rows, int cols);

}  // namespace lh

#endif  // LONGHORN_MI355X_KERNELS_QUANT_HPP
