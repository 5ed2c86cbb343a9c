// gemm.cpp -- lh:: fp32 GEMM drivers (reference gemm.cpp:5-75) on the MI355X
// backend.
#include "kernels/gemm.hpp"

#include "kernels/device.hpp"
#include "longhorn_hip.h"

namespace lh {

namespace {

using dev::Buffer;

size_t nonneg(int v) { return v > 0 ? static_cast<size_t>(v) : 0; }

// One fp32 GEMM of `batch` uniform problems on the GPU.  `read_c` uploads C
// (gemm_ref always reads C; gemm reads it only for beta != 0).
template <typename Launch>
void run(const float* A, const float* B, float* C, int batch, int M, int N, int K, bool read_c, Launch launch,
         const char* what) {
    if (batch <= 0 || M <= 0 || N <= 0) return;
    const size_t a = nonneg(batch) * nonneg(M) * nonneg(K), b = nonneg(batch) * nonneg(K) * nonneg(N);
    const size_t c = nonneg(batch) * nonneg(M) * nonneg(N);
    Buffer dA(a * sizeof(float)), dB(b * sizeof(float)), dC(c * sizeof(float));
    dA.upload(A, a * sizeof(float));
    dB.upload(B, b * sizeof(float));
    if (read_c) dC.upload(C, c * sizeof(float));
    dev::check(launch(dA.as<float>(), dB.as<float>(), dC.as<float>()), what);
    dC.download(C, c * sizeof(float));
}

}  // namespace

void gemm_ref(const float* A, const float* B, float* C, int M, int N, int K, float alpha, float beta) {
    run(A, B, C, 1, M, N, K, true, [&](const float* a, const float* b, float* c) {
        return lhq_gemm_f32_ref(a, b, c, M, N, K, alpha, beta, dev::stream());
    }, "gemm_ref");
}

void gemm(const float* A, const float* B, float* C, int M, int N, int K, float alpha, float beta) {
    run(A, B, C, 1, M, N, K, beta != 0.0f, [&](const float* a, const float* b, float* c) {
        return lhq_gemm_f32(a, b, c, M, N, K, alpha, beta, dev::stream());
    }, "gemm");
}

void gemm_batched(const float* A, const float* B, float* C, int batch, int M, int N, int K, float alpha, float beta) {
    run(A, B, C, batch, M, N, K, beta != 0.0f, [&](const float* a, const float* b, float* c) {
        return lhq_gemm_f32_batched(a, b, c, batch, M, N, K, alpha, beta, dev::stream());
    }, "gemm_batched");
}

void gemm_grouped(const float* const* A, const float* const* B, float* const* C, const int* M, const int* N,
                  const int* K, int groups, float alpha, float beta) {
    // Each group is an independent problem of its own shape (gemm.cpp:69-75);
    // they run one after another on the GPU.
    for (int g = 0; g < groups; ++g) gemm(A[g], B[g], C[g], M[g], N[g], K[g], alpha, beta);
}

}  // namespace lh
