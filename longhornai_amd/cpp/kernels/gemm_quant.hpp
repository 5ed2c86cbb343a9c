// kernels/gemm_quant.hpp -- quantized GEMMs of LonghornAI, on the MI355X
// backend.
//
// Drop-in for the reference header (src/kernels/gemm_quant.hpp:34-70): the
// same three functions, signatures and results, computed by the gfx950
// kernels behind the C ABI (include/longhorn_hip.h).  Calls are synchronous
// on host memory like the reference's; a HIP failure prints the library's
// message and aborts (no CPU code path).
//
//   gemm_w8a8             C = beta*C + alpha*A_s[m]*B_s[n]*sum_k Aq*Bq; the
//                         int32 accumulation and the fp32 epilogue
//                         ((alpha*A_s)*B_s)*float(acc) are bit-exact.
//   gemm_w4a16_groupwise  C = beta*C + alpha*A @ dequant(B); MFMA over the
//                         exact int4 codes, fp32 accumulation (relative
//                         Frobenius error vs the reference well below 1e-4).
//   gemm_fp8_e4m3         C = beta*C + ((alpha*sA)*sB)*sum_k A*B, fp32 acc.
// beta == 0 writes C without reading it (gemm_quant.cpp:12-21).
#ifndef LONGHORN_MI355X_KERNELS_GEMM_QUANT_HPP
#define LONGHORN_MI355X_KERNELS_GEMM_QUANT_HPP

#include <cstdint>

#include "kernels/dtypes.hpp"

namespace lh {

void gemm_w8a8(const int8_t* A_q, const int8_t* B_q,
               const float* A_scales, const float* B_scales,
               float* C, int M, int N, int K,
               float alpha = 1.0f, float beta = 0.0f);

void gemm_w4a16_groupwise(const float* A, const uint8_t* B_packed,
                          const float* B_scales, float* C,
                          int M, int N, int K, int group_size,
                          float alpha = 1.0f, float beta = 0.0f);

void gemm_fp8_e4m3(const fp8_e4m3* A, const fp8_e4m3* B,
                   float A_scale, float B_scale,
                   float* C, int M, int N, int K,
                   float alpha = 1.0f, float beta = 0.0f);

}  // namespace lh

#endif  // LONGHORN_MI355X_KERNELS_GEMM_QUANT_HPP
