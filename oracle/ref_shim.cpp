// ref_shim.cpp -- C entry points over the reference's own quantized-GEMM
// sources, compiled from /root/reference/src by oracle/Makefile into
// oracle/_ref/libref.so.  TEST INFRASTRUCTURE ONLY: it lets the CPU tests pin
// the C restatement (lhq_oracle.c) bit-for-bit against the real reference,
// and lets bench.py time the reference CPU path.  Nothing here is shipped.
//
// Each wrapper forwards to one lh:: function with unchanged arguments:
//   quant.hpp:31-94, gemm_quant.hpp:42-70, gemm.hpp:14-29, dtypes.hpp:17-269,
//   moe.hpp:75-102 (dispatch, expert MLP, combine; MoEConfig moe.hpp:39-49).
#include <cstdint>

#include "kernels/dtypes.hpp"
#include "kernels/gemm.hpp"
#include "kernels/gemm_quant.hpp"
#include "kernels/moe.hpp"
#include "kernels/quant.hpp"

static_assert(sizeof(lh::fp8_e4m3) == 1, "fp8_e4m3 must be one byte");

extern "C" {

uint16_t ref_f32_to_f16(float v) { return lh::detail::float_to_half_bits(v); }
float ref_f16_to_f32(uint16_t h) { return lh::detail::half_bits_to_float(h); }
uint16_t ref_f32_to_bf16(float v) { return lh::detail::float_to_bf16_bits(v); }
float ref_bf16_to_f32(uint16_t b) { return lh::detail::bf16_bits_to_float(b); }
uint8_t ref_f32_to_e4m3(float v) { return lh::detail::float_to_e4m3_bits(v); }
float ref_e4m3_to_f32(uint8_t b) { return lh::detail::e4m3_bits_to_float(b); }
uint8_t ref_f32_to_e5m2(float v) { return lh::detail::float_to_e5m2_bits(v); }
float ref_e5m2_to_f32(uint8_t b) { return lh::detail::e5m2_bits_to_float(b); }

// Array forms: values never pass through a host double, so NaN payloads
// (signaling ones included) arrive bit for bit.
void ref_f16_to_f32_n(const uint16_t* x, float* y, int64_t n) { for (int64_t i = 0; i < n; ++i) y[i] = lh::detail::half_bits_to_float(x[i]); }
void ref_e4m3_to_f32_n(const uint8_t* x, float* y, int64_t n) { for (int64_t i = 0; i < n; ++i) y[i] = lh::detail::e4m3_bits_to_float(x[i]); }
void ref_e5m2_to_f32_n(const uint8_t* x, float* y, int64_t n) { for (int64_t i = 0; i < n; ++i) y[i] = lh::detail::e5m2_bits_to_float(x[i]); }
void ref_f32_to_f16_n(const float* x, uint16_t* y, int64_t n) { for (int64_t i = 0; i < n; ++i) y[i] = lh::detail::float_to_half_bits(x[i]); }
void ref_f32_to_bf16_n(const float* x, uint16_t* y, int64_t n) { for (int64_t i = 0; i < n; ++i) y[i] = lh::detail::float_to_bf16_bits(x[i]); }
void ref_f32_to_e4m3_n(const float* x, uint8_t* y, int64_t n) { for (int64_t i = 0; i < n; ++i) y[i] = lh::detail::float_to_e4m3_bits(x[i]); }
void ref_f32_to_e5m2_n(const float* x, uint8_t* y, int64_t n) { for (int64_t i = 0; i < n; ++i) y[i] = lh::detail::float_to_e5m2_bits(x[i]); }

void ref_q8_quantize_per_tensor(const float* s, int8_t* d, float* sc, int64_t n) { lh::q8_quantize_per_tensor(s, d, sc, n); }
void ref_q8_dequantize_per_tensor(const int8_t* s, float sc, float* d, int64_t n) { lh::q8_dequantize_per_tensor(s, sc, d, n); }
void ref_q8_quantize_per_row(const float* s, int8_t* d, float* sc, int r, int c) { lh::q8_quantize_per_row(s, d, sc, r, c); }
void ref_q8_dequantize_per_row(const int8_t* s, const float* sc, float* d, int r, int c) { lh::q8_dequantize_per_row(s, sc, d, r, c); }
void ref_q8_quantize_per_col(const float* s, int8_t* d, float* sc, int r, int c) { lh::q8_quantize_per_col(s, d, sc, r, c); }
void ref_q8_dequantize_per_col(const int8_t* s, const float* sc, float* d, int r, int c) { lh::q8_dequantize_per_col(s, sc, d, r, c); }
void ref_q4_quantize_groupwise(const float* s, uint8_t* p, float* sc, int K, int N, int G) { lh::q4_quantize_groupwise(s, p, sc, K, N, G); }
void ref_q4_dequantize_groupwise(const uint8_t* p, const float* sc, float* d, int K, int N, int G) { lh::q4_dequantize_groupwise(p, sc, d, K, N, G); }
int8_t ref_q4_get(const uint8_t* p, int k, int n, int N) { return lh::q4_get(p, k, n, N); }

void ref_fp8_quantize_per_tensor(const float* s, uint8_t* d, float* sc, int64_t n) {
    lh::fp8_quantize_per_tensor(s, reinterpret_cast<lh::fp8_e4m3*>(d), sc, n);
}
void ref_fp8_dequantize_per_tensor(const uint8_t* s, float sc, float* d, int64_t n) {
    lh::fp8_dequantize_per_tensor(reinterpret_cast<const lh::fp8_e4m3*>(s), sc, d, n);
}
void ref_fp8_quantize_per_row(const float* s, uint8_t* d, float* sc, int r, int c) {
    lh::fp8_quantize_per_row(s, reinterpret_cast<lh::fp8_e4m3*>(d), sc, r, c);
}
void ref_fp8_dequantize_per_row(const uint8_t* s, const float* sc, float* d, int r, int c) {
    lh::fp8_dequantize_per_row(reinterpret_cast<const lh::fp8_e4m3*>(s), sc, d, r, c);
}
void ref_fp8_quantize_per_col(const float* s, uint8_t* d, float* sc, int r, int c) {
    lh::fp8_quantize_per_col(s, reinterpret_cast<lh::fp8_e4m3*>(d), sc, r, c);
}
void ref_fp8_dequantize_per_col(const uint8_t* s, const float* sc, float* d, int r, int c) {
    lh::fp8_dequantize_per_col(reinterpret_cast<const lh::fp8_e4m3*>(s), sc, d, r, c);
}

void ref_gemm_w8a8(const int8_t* A, const int8_t* B, const float* As, const float* Bs,
                   float* C, int M, int N, int K, float alpha, float beta) {
    lh::gemm_w8a8(A, B, As, Bs, C, M, N, K, alpha, beta);
}
void ref_gemm_w4a16_groupwise(const float* A, const uint8_t* Bp, const float* Bs, float* C,
                              int M, int N, int K, int G, float alpha, float beta) {
    lh::gemm_w4a16_groupwise(A, Bp, Bs, C, M, N, K, G, alpha, beta);
}
void ref_gemm_fp8_e4m3(const uint8_t* A, const uint8_t* B, float sa, float sb, float* C,
                       int M, int N, int K, float alpha, float beta) {
    lh::gemm_fp8_e4m3(reinterpret_cast<const lh::fp8_e4m3*>(A),
                      reinterpret_cast<const lh::fp8_e4m3*>(B), sa, sb, C, M, N, K, alpha, beta);
}
void ref_gemm_ref(const float* A, const float* B, float* C, int M, int N, int K, float alpha, float beta) {
    lh::gemm_ref(A, B, C, M, N, K, alpha, beta);
}
void ref_gemm(const float* A, const float* B, float* C, int M, int N, int K, float alpha, float beta) {
    lh::gemm(A, B, C, M, N, K, alpha, beta);
}
void ref_gemm_batched(const float* A, const float* B, float* C, int batch, int M, int N, int K,
                      float alpha, float beta) {
    lh::gemm_batched(A, B, C, batch, M, N, K, alpha, beta);
}
void ref_gemm_grouped(const float* const* A, const float* const* B, float* const* C, const int* M,
                      const int* N, const int* K, int groups, float alpha, float beta) {
    lh::gemm_grouped(A, B, C, M, N, K, groups, alpha, beta);
}

static lh::MoEConfig moe_cfg(int T, int H, int I, int E, int K) {
    lh::MoEConfig c;
    c.n_tokens = T;
    c.hidden_dim = H;
    c.intermediate_dim = I;
    c.n_experts = E;
    c.top_k = K;
    return c;
}
void ref_moe_dispatch(const float* hidden, const int32_t* ids, int32_t* offsets, int32_t* tok,
                      int32_t* slot, float* out, int T, int H, int E, int K) {
    lh::moe_dispatch(hidden, ids, offsets, tok, slot, out, moe_cfg(T, H, 0, E, K));
}
void ref_moe_expert_mlp(const float* x, const int32_t* offsets, const float* Wg, const float* Wu,
                        const float* Wd, float* y, int H, int I, int E) {
    lh::moe_expert_mlp(x, offsets, Wg, Wu, Wd, y, moe_cfg(0, H, I, E, 1));
}
void ref_moe_combine(const float* y, const int32_t* offsets, const int32_t* tok, const int32_t* slot,
                     const float* gates, float* out, int T, int H, int E, int K) {
    lh::moe_combine(y, offsets, tok, slot, gates, out, moe_cfg(T, H, 0, E, K));
}

}  // extern "C"
