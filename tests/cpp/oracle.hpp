// oracle.hpp -- the CPU parity checker (oracle/lhq_oracle.c, built into
// oracle/liboracle.so) as seen from the C++ suites.  TEST INFRASTRUCTURE
// ONLY: the suites compare the lh:: drop-in (GPU) against these functions;
// the drop-in library itself never links them.
#ifndef LONGHORN_TESTS_ORACLE_HPP
#define LONGHORN_TESTS_ORACLE_HPP

#include <cstdint>

extern "C" {
uint16_t lho_f32_to_f16(float);
float lho_f16_to_f32(uint16_t);
uint16_t lho_f32_to_bf16(float);
float lho_bf16_to_f32(uint16_t);
uint8_t lho_f32_to_e4m3(float);
float lho_e4m3_to_f32(uint8_t);
uint8_t lho_f32_to_e5m2(float);
float lho_e5m2_to_f32(uint8_t);
int8_t lho_q4_get(const uint8_t*, int, int, int);
void lho_q8_quantize_per_tensor(const float*, int8_t*, float*, int64_t);
void lho_q8_quantize_per_row(const float*, int8_t*, float*, int, int);
void lho_q8_quantize_per_col(const float*, int8_t*, float*, int, int);
void lho_q8_dequantize_per_row(const int8_t*, const float*, float*, int, int);
void lho_q8_dequantize_per_col(const int8_t*, const float*, float*, int, int);
void lho_q4_quantize_groupwise(const float*, uint8_t*, float*, int, int, int);
void lho_q4_dequantize_groupwise(const uint8_t*, const float*, float*, int, int, int);
void lho_fp8_quantize_per_tensor(const float*, uint8_t*, float*, int64_t);
void lho_fp8_quantize_per_row(const float*, uint8_t*, float*, int, int);
void lho_fp8_quantize_per_col(const float*, uint8_t*, float*, int, int);
void lho_gemm_w8a8(const int8_t*, const int8_t*, const float*, const float*, float*, int, int, int, float, float);
void lho_gemm_w4a16_groupwise(const float*, const uint8_t*, const float*, float*, int, int, int, int, float, float);
void lho_gemm_fp8_e4m3(const uint8_t*, const uint8_t*, float, float, float*, int, int, int, float, float);
void lho_gemm_ref(const float*, const float*, float*, int, int, int, float, float);
void lho_gemm(const float*, const float*, float*, int, int, int, float, float);
void lho_gemm_batched(const float*, const float*, float*, int, int, int, int, float, float);
void lho_gemm_grouped(const float* const*, const float* const*, float* const*, const int*, const int*, const int*, int,
                      float, float);
void lho_moe_dispatch(const void*, int64_t, const int32_t*, int, int, int, int32_t*, int32_t*, int32_t*, int32_t*,
                      void*);
void lho_moe_combine_f32(const float*, const int32_t*, const int32_t*, const float*, float*, int, int, int);
}

#endif  // LONGHORN_TESTS_ORACLE_HPP
