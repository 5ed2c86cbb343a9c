// kernels/gemm.hpp -- fp32 GEMM and its batched / grouped drivers, on the
// MI355X backend.
//
// Drop-in for the reference header (src/kernels/gemm.hpp:13-29), row-major,
// fp32 accumulation:
//   gemm_ref      C = alpha*A@B + beta*C (C always read);
//   gemm          beta applied first, beta == 0 never reads C;
//   gemm_batched  uniform batch, A [batch,M,K], B [batch,K,N], C [batch,M,N];
//   gemm_grouped  ragged pointer-array groups (A[g], B[g], C[g], M[g], N[g],
//                 K[g]).
// Synchronous on host memory; a HIP failure aborts with the library's message.
#ifndef LONGHORN_MI355X_KERNELS_GEMM_HPP
#define LONGHORN_MI355X_KERNELS_GEMM_HPP

#include <cstdint>

namespace lh {

void gemm_ref(const float* A, const float* B, float* C,
              int M, int N, int K, float alpha = 1.0f, float beta = 0.0f);

void gemm(const float* A, const float* B, float* C,
          int M, int N, int K, float alpha = 1.0f, float beta = 0.0f);

void gemm_batched(const float* A, const float* B, float* C,
                  int batch, int M, int N, int K,
                  float alpha = 1.0f, float beta = 0.0f);

void gemm_grouped(const float* const* A, const float* const* B,
                  float* const* C, const int* M, const int* N, const int* K,
                  int groups, float alpha = 1.0f, float beta = 0.0f);

}  // namespace lh

#endif  // LONGHORN_MI355X_KERNELS_GEMM_HPP
