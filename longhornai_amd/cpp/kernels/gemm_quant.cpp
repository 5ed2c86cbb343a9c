// gemm_quant.cpp -- lh:: quantized GEMMs (reference gemm_quant.cpp:29-104) on
// the MI355X backend.
//
// Each call stages host operands in device memory, converts the weights to
// the layout the gfx950 kernels stream (lhq_b8_prepack / lhq_w4_prepack_sym,
// once per call: the reference's interface has no persistent weight handle),
// launches the kernel and copies C back.
#include "kernels/gemm_quant.hpp"

#include <algorithm>
#include <cmath>

#include "kernels/device.hpp"
#include "longhorn_hip.h"

namespace lh {

namespace {

using dev::Buffer;

size_t nonneg(int v) { return v > 0 ? static_cast<size_t>(v) : 0; }

// The 8-bit MFMA kernels take K in multiples of 16: pad the activation rows
// with zero codes (a zero code contributes nothing: int8 0 and e4m3 0x00 are
// both exactly zero) and let the weight prepack zero-pad the weights.
constexpr int kK8Align = 16;
int pad_k8(int K) { return (K + kK8Align - 1) / kK8Align * kK8Align; }

// A [M, K] bytes -> device [M, Kp] with zero padding.
void stage_a8(Buffer& dst, const void* A, int M, int K, int Kp) {
    dst.zero();
    dev::upload_pitched(dst, nonneg(Kp), A, nonneg(K), nonneg(M));
}

// C staging: only read when beta != 0 (beta == 0 never reads C).
void stage_c(Buffer& dC, const float* C, size_t count, float beta) {
    if (beta != 0.0f) dC.upload(C, count * sizeof(float));
}

bool all_finite(const float* x, size_t count) {
    for (size_t i = 0; i < count; ++i)
        if (!std::isfinite(x[i])) return false;
    return true;
}

}  // namespace

void gemm_w8a8(const int8_t* A_q, const int8_t* B_q, const float* A_scales, const float* B_scales, float* C,
               int M, int N, int K, float alpha, float beta) {
    if (M <= 0 || N <= 0) return;
    const size_t mn = nonneg(M) * nonneg(N);
    if (K <= 0) {
        // empty reduction: C = beta-applied C (gemm_quant.cpp:12-21 with no terms)
        Buffer dC(mn * sizeof(float));
        stage_c(dC, C, mn, beta);
        Buffer dA(nonneg(M) * kK8Align), dB(static_cast<size_t>(lhq_b8_prepacked_bytes(kK8Align, N)));
        dA.zero();
        dB.zero();
        Buffer as(nonneg(M) * sizeof(float)), bs(nonneg(N) * sizeof(float));
        as.upload(A_scales, nonneg(M) * sizeof(float));
        bs.upload(B_scales, nonneg(N) * sizeof(float));
        dev::check(lhq_gemm_w8a8(dA.as<int8_t>(), dB.as<int8_t>(), as.as<float>(), bs.as<float>(), dC.as<float>(),
                                 M, N, kK8Align, alpha, beta, dev::stream()),
                   "gemm_w8a8");
        dC.download(C, mn * sizeof(float));
        return;
    }
    const int Kp = pad_k8(K);
    Buffer dA(nonneg(M) * nonneg(Kp)), dB(nonneg(K) * nonneg(N));
    Buffer dBt(static_cast<size_t>(lhq_b8_prepacked_bytes(Kp, N)));
    Buffer as(nonneg(M) * sizeof(float)), bs(nonneg(N) * sizeof(float)), dC(mn * sizeof(float));
    stage_a8(dA, A_q, M, K, Kp);
    dB.upload(B_q, nonneg(K) * nonneg(N));
    as.upload(A_scales, nonneg(M) * sizeof(float));
    bs.upload(B_scales, nonneg(N) * sizeof(float));
    stage_c(dC, C, mn, beta);
    dev::check(lhq_b8_prepack(dB.as<uint8_t>(), K, N, dBt.as<uint8_t>(), dev::stream()), "gemm_w8a8 (prepack)");
    dev::check(lhq_gemm_w8a8(dA.as<int8_t>(), dBt.as<int8_t>(), as.as<float>(), bs.as<float>(), dC.as<float>(), M, N,
                             Kp, alpha, beta, dev::stream()),
               "gemm_w8a8");
    dC.download(C, mn * sizeof(float));
}

void gemm_w4a16_groupwise(const float* A, const uint8_t* B_packed, const float* B_scales, float* C, int M, int N,
                          int K, int group_size, float alpha, float beta) {
    if (M <= 0 || N <= 0) return;
    const int G = group_size;
    if (K <= 0 || G <= 0 || K % G != 0 || K % 2 != 0)
        dev::fail("gemm_w4a16_groupwise", "need K > 0 even and group_size | K (quant.hpp:50-61)");
    const size_t mn = nonneg(M) * nonneg(N);
    const size_t kn = nonneg(K) * nonneg(N);
    const size_t ns = nonneg(K / G) * nonneg(N);
    Buffer dA(nonneg(M) * nonneg(K) * sizeof(float)), dP(kn / 2), dS(ns * sizeof(float)), dC(mn * sizeof(float));
    dA.upload(A, nonneg(M) * nonneg(K) * sizeof(float));
    dP.upload(B_packed, kn / 2);
    dS.upload(B_scales, ns * sizeof(float));
    stage_c(dC, C, mn, beta);
    // The MFMA kernels sum x * (q - z) through exact group sums that
    // subtract an activation sum, so a non-finite activation turns its
    // whole output row into NaN (Inf - Inf).  The reference adds
    // a * (q * s) term by term (gemm_quant.cpp:74-79): +-Inf where the
    // weight is nonzero, NaN where it is zero or infinities of both signs
    // meet.  Host activations holding a non-finite value therefore take the
    // dequantize + fp32 GEMM path, which adds products the same way.
    const bool mfma_groups = (G == 32 || G == 64 || G % 128 == 0) && all_finite(A, nonneg(M) * nonneg(K));
    if (mfma_groups) {
        // int4 codes straight into the MFMA, group scales in fp32
        Buffer qw(static_cast<size_t>(lhq_w4_qweight_bytes(K, N)));
        Buffer qs(static_cast<size_t>(lhq_w4_scales_bytes(K, N, G, 0)));
        dev::check(lhq_w4_prepack_sym(dP.as<uint8_t>(), dS.as<float>(), K, N, G, qw.as<uint8_t>(), qs.as<float>(),
                                      dev::stream()),
                   "gemm_w4a16_groupwise (prepack)");
        // thin grids split K across workgroups over a workspace
        // (a zero-byte Buffer holds no allocation: the call then runs unsplit)
        const int64_t ws_bytes = std::max<int64_t>(0, lhq_gemm_w4a16_workspace_bytes(M, N, K, G));
        Buffer ws(static_cast<size_t>(ws_bytes));
        dev::check(lhq_gemm_w4a16_ws(dA.as<float>(), qw.as<uint8_t>(), qs.as<float>(), dC.as<float>(), M, N, K, G,
                                     alpha, beta, ws.get(), ws_bytes, dev::stream()),
                   "gemm_w4a16_groupwise");
    } else {
        // group sizes the MFMA segmentation cannot express (not 32, 64 or a
        // multiple of 128), or non-finite activations: dequantize on the GPU
        // (exact: float(q) * s, as gemm_quant.cpp:64-70 does) and run the
        // fp32 GEMM on the GPU
        Buffer dW(kn * sizeof(float));
        dev::check(lhq_q4_dequantize_groupwise(dP.as<uint8_t>(), dS.as<float>(), dW.as<float>(), K, N, G,
                                               dev::stream()),
                   "gemm_w4a16_groupwise (dequantize)");
        dev::check(lhq_gemm_f32(dA.as<float>(), dW.as<float>(), dC.as<float>(), M, N, K, alpha, beta, dev::stream()),
                   "gemm_w4a16_groupwise (fp32 gemm)");
    }
    dC.download(C, mn * sizeof(float));
}

void gemm_fp8_e4m3(const fp8_e4m3* A, const fp8_e4m3* B, float A_scale, float B_scale, float* C, int M, int N, int K,
                   float alpha, float beta) {
    if (M <= 0 || N <= 0) return;
    const size_t mn = nonneg(M) * nonneg(N);
    const int Kq = K > 0 ? K : 0;
    const int Kp = pad_k8(Kq > 0 ? Kq : 1);
    Buffer dA(nonneg(M) * nonneg(Kp)), dB(nonneg(Kp) * nonneg(N));
    Buffer dBt(static_cast<size_t>(lhq_b8_prepacked_bytes(Kp, N)));
    Buffer sa(sizeof(float)), sb(sizeof(float)), dC(mn * sizeof(float));
    stage_a8(dA, A, M, Kq, Kp);
    dB.zero();
    dB.upload(B, nonneg(Kq) * nonneg(N));
    sa.upload(&A_scale, sizeof(float));
    sb.upload(&B_scale, sizeof(float));
    stage_c(dC, C, mn, beta);
    dev::check(lhq_b8_prepack(dB.as<uint8_t>(), Kp, N, dBt.as<uint8_t>(), dev::stream()), "gemm_fp8_e4m3 (prepack)");
    dev::check(lhq_gemm_fp8_e4m3(dA.as<uint8_t>(), dBt.as<uint8_t>(), sa.as<float>(), sb.as<float>(), dC.as<float>(),
                                 M, N, Kp, alpha, beta, dev::stream()),
               "gemm_fp8_e4m3");
    dC.download(C, mn * sizeof(float));
}

}  // namespace lh
