// gemm_f32.hip -- fp32 GEMM behind the gemm.hpp drop-in (gemm.hpp:13-29).
//
// The reference's fp32 GEMM is the baseline every quantized-GEMM test
// compares against (test_gemm_quant.cpp:38,62,83,106).  It is not a hot path
// here, so this is a plain LDS-tiled VALU kernel: a 256-thread workgroup owns
// a 64x64 output tile, each thread a 4x4 block, K staged 16 at a time.
// Semantics follow gemm.cpp: lh::gemm applies beta first and never reads C
// when beta == 0 (gemm.cpp:60-68); lh::gemm_ref always reads C and returns
// alpha*acc + beta*C (gemm.cpp:5-16).  grid.z walks a uniform batch
// (gemm.cpp:59-67).
#include "common.hpp"

namespace lhq {
namespace {

constexpr int T = 64, TK = 16;

template <bool REF>
__global__ __launch_bounds__(256) void gemm_f32_kernel(const float* __restrict__ A, const float* __restrict__ B,
                                                       float* __restrict__ C, int M, int N, int K, float alpha,
                                                       float beta) {
    __shared__ float sa[TK][T + 4];
    __shared__ float sb[TK][T + 4];
    const int64_t z = blockIdx.z;
    A += z * M * static_cast<int64_t>(K);
    B += z * K * static_cast<int64_t>(N);
    C += z * M * static_cast<int64_t>(N);
    const int m0 = blockIdx.y * T, n0 = blockIdx.x * T;
    const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
    float acc[4][4] = {};
    for (int k0 = 0; k0 < K; k0 += TK) {
        for (int i = threadIdx.x; i < T * TK; i += 256) {
            const int r = i / TK, c = i % TK;  // A tile: 64 rows x 16 k
            const int gm = m0 + r, gk = k0 + c;
            sa[c][r] = (gm < M && gk < K) ? A[static_cast<int64_t>(gm) * K + gk] : 0.0f;
            const int kr = i / T, nc = i % T;  // B tile: 16 k x 64 cols
            const int gk2 = k0 + kr, gn = n0 + nc;
            sb[kr][nc] = (gk2 < K && gn < N) ? B[static_cast<int64_t>(gk2) * N + gn] : 0.0f;
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < TK; ++kk) {
            float a[4], b[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) a[i] = sa[kk][ty * 4 + i];
#pragma unroll
            for (int j = 0; j < 4; ++j) b[j] = sb[kk][tx * 4 + j];
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_fmaf(a[i], b[j], acc[i][j]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int m = m0 + ty * 4 + i;
        if (m >= M) continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int n = n0 + tx * 4 + j;
            if (n >= N) continue;
            float* c = C + static_cast<int64_t>(m) * N + n;
            if (REF) {
                *c = alpha * acc[i][j] + beta * *c;
            } else {
                const float base = (beta == 0.0f) ? 0.0f : (beta == 1.0f) ? *c : *c * beta;
                *c = base + alpha * acc[i][j];
            }
        }
    }
}

template <bool REF>
int launch(const float* A, const float* B, float* C, int batch, int M, int N, int K, float alpha, float beta,
           void* stream, const char* who) {
    LHQ_REQUIRE(batch >= 0 && M >= 0 && N >= 0 && K >= 0, "%s: negative dims", who);
    LHQ_REQUIRE(batch <= 65535, "%s: batch %d too large", who, batch);
    if (batch == 0 || M == 0 || N == 0) return LHQ_OK;
    LHQ_REQUIRE(C && ((A && B) || K == 0), "%s: null pointer", who);
    dim3 grid(ceil_div(N, T), ceil_div(M, T), batch);
    gemm_f32_kernel<REF><<<grid, 256, 0, as_stream(stream)>>>(A, B, C, M, N, K, alpha, beta);
    return check_launch(who);
}

}  // namespace
}  // namespace lhq

extern "C" {

int lhq_gemm_f32(const float* A, const float* B, float* C, int M, int N, int K, float alpha, float beta,
                 void* stream) {
    return lhq::launch<false>(A, B, C, 1, M, N, K, alpha, beta, stream, "gemm_f32");
}

int lhq_gemm_f32_ref(const float* A, const float* B, float* C, int M, int N, int K, float alpha, float beta,
                     void* stream) {
    return lhq::launch<true>(A, B, C, 1, M, N, K, alpha, beta, stream, "gemm_f32_ref");
}

int lhq_gemm_f32_batched(const float* A, const float* B, float* C, int batch, int M, int N, int K, float alpha,
                         float beta, void* stream) {
    return lhq::launch<false>(A, B, C, batch, M, N, K, alpha, beta, stream, "gemm_f32_batched");
}

}  // extern "C"
