// quant.cpp -- lh:: quantizers (reference quant.cpp:34-249) on the MI355X
// backend: stage host data on the device, run the gfx950 quantizer behind the
// C ABI, copy the result back.
#include "kernels/quant.hpp"

#include <cstring>

#include "kernels/device.hpp"
#include "longhorn_hip.h"

namespace lh {

namespace {

using dev::Buffer;

// Per-tensor quantize: src f32 [n] -> dst [n] of `ebytes`-byte codes + scale.
template <typename Fn>
void per_tensor(const float* src, void* dst, float* scale_out, int64_t n, Fn fn, const char* what) {
    const size_t count = n > 0 ? static_cast<size_t>(n) : 0;
    Buffer s(count * sizeof(float)), d(count), sc(sizeof(float));
    s.upload(src, count * sizeof(float));
    dev::check(fn(s.get(), d.get(), sc.as<float>(), n), what);
    d.download(dst, count);
    sc.download(scale_out, sizeof(float));
}

// Per-tensor dequantize with a host-side scale.
template <typename Fn>
void per_tensor_dq(const void* src, float scale, float* dst, int64_t n, Fn fn, const char* what) {
    const size_t count = n > 0 ? static_cast<size_t>(n) : 0;
    Buffer s(count), sc(sizeof(float)), d(count * sizeof(float));
    s.upload(src, count);
    sc.upload(&scale, sizeof(float));
    dev::check(fn(s.get(), sc.as<float>(), d.as<float>(), n), what);
    d.download(dst, count * sizeof(float));
}

// [rows, cols] quantize with one scale per row (nscales = rows) or column.
template <typename Fn>
void shaped(const float* src, void* dst, float* scales_out, int rows, int cols, size_t nscales, Fn fn,
            const char* what) {
    const size_t count = rows > 0 && cols > 0 ? static_cast<size_t>(rows) * cols : 0;
    Buffer s(count * sizeof(float)), d(count), sc(nscales * sizeof(float));
    s.upload(src, count * sizeof(float));
    dev::check(fn(s.as<float>(), d.get(), sc.as<float>(), rows, cols), what);
    d.download(dst, count);
    sc.download(scales_out, nscales * sizeof(float));
}

template <typename Fn>
void shaped_dq(const void* src, const float* scales, float* dst, int rows, int cols, size_t nscales, Fn fn,
               const char* what) {
    const size_t count = rows > 0 && cols > 0 ? static_cast<size_t>(rows) * cols : 0;
    Buffer s(count), sc(nscales * sizeof(float)), d(count * sizeof(float));
    s.upload(src, count);
    sc.upload(scales, nscales * sizeof(float));
    dev::check(fn(s.get(), sc.as<float>(), d.as<float>(), rows, cols), what);
    d.download(dst, count * sizeof(float));
}

size_t nonneg(int v) { return v > 0 ? static_cast<size_t>(v) : 0; }

}  // namespace

// --- INT8 -------------------------------------------------------------------

void q8_quantize_per_tensor(const float* src, int8_t* dst, float* scale_out, int64_t n) {
    per_tensor(src, dst, scale_out, n, [](void* s, void* d, float* sc, int64_t k) {
        return lhq_q8_quantize_per_tensor(static_cast<const float*>(s), static_cast<int8_t*>(d), sc, k, dev::stream());
    }, "q8_quantize_per_tensor");
}

void q8_dequantize_per_tensor(const int8_t* src, float scale, float* dst, int64_t n) {
    per_tensor_dq(src, scale, dst, n, [](const void* s, const float* sc, float* d, int64_t k) {
        return lhq_q8_dequantize_per_tensor(static_cast<const int8_t*>(s), sc, d, k, dev::stream());
    }, "q8_dequantize_per_tensor");
}

void q8_quantize_per_row(const float* src, int8_t* dst, float* scales_out, int rows, int dim) {
    shaped(src, dst, scales_out, rows, dim, nonneg(rows), [](const float* s, void* d, float* sc, int r, int c) {
        return lhq_q8_quantize_per_row(s, static_cast<int8_t*>(d), sc, r, c, dev::stream());
    }, "q8_quantize_per_row");
}

void q8_dequantize_per_row(const int8_t* src, const float* scales, float* dst, int rows, int dim) {
    shaped_dq(src, scales, dst, rows, dim, nonneg(rows), [](const void* s, const float* sc, float* d, int r, int c) {
        return lhq_q8_dequantize_per_row(static_cast<const int8_t*>(s), sc, d, r, c, dev::stream());
    }, "q8_dequantize_per_row");
}

void q8_quantize_per_col(const float* src, int8_t* dst, float* scales_out, int rows, int cols) {
    shaped(src, dst, scales_out, rows, cols, nonneg(cols), [](const float* s, void* d, float* sc, int r, int c) {
        return lhq_q8_quantize_per_col(s, static_cast<int8_t*>(d), sc, r, c, dev::stream());
    }, "q8_quantize_per_col");
}

void q8_dequantize_per_col(const int8_t* src, const float* scales, float* dst, int rows, int cols) {
    shaped_dq(src, scales, dst, rows, cols, nonneg(cols), [](const void* s, const float* sc, float* d, int r, int c) {
        return lhq_q8_dequantize_per_col(static_cast<const int8_t*>(s), sc, d, r, c, dev::stream());
    }, "q8_dequantize_per_col");
}

// --- INT4 -------------------------------------------------------------------

void q4_quantize_groupwise(const float* src, uint8_t* packed, float* scales_out, int K, int N, int group_size) {
    const size_t kn = nonneg(K) * nonneg(N);
    const size_t ns = group_size > 0 ? nonneg(K / group_size) * nonneg(N) : 0;
    Buffer s(kn * sizeof(float)), p(kn / 2), sc(ns * sizeof(float));
    s.upload(src, kn * sizeof(float));
    dev::check(lhq_q4_quantize_groupwise(s.as<float>(), p.as<uint8_t>(), sc.as<float>(), K, N, group_size,
                                         dev::stream()),
               "q4_quantize_groupwise");
    p.download(packed, kn / 2);
    sc.download(scales_out, ns * sizeof(float));
}

void q4_dequantize_groupwise(const uint8_t* packed, const float* scales, float* dst, int K, int N, int group_size) {
    const size_t kn = nonneg(K) * nonneg(N);
    const size_t ns = group_size > 0 ? nonneg(K / group_size) * nonneg(N) : 0;
    Buffer p(kn / 2), sc(ns * sizeof(float)), d(kn * sizeof(float));
    p.upload(packed, kn / 2);
    sc.upload(scales, ns * sizeof(float));
    dev::check(lhq_q4_dequantize_groupwise(p.as<uint8_t>(), sc.as<float>(), d.as<float>(), K, N, group_size,
                                           dev::stream()),
               "q4_dequantize_groupwise");
    d.download(dst, kn * sizeof(float));
}

// --- FP8 E4M3 (fp8_e4m3 is a one-byte bit container) ------------------------

static_assert(sizeof(fp8_e4m3) == 1, "fp8_e4m3 must be a single byte");

void fp8_quantize_per_tensor(const float* src, fp8_e4m3* dst, float* scale_out, int64_t n) {
    per_tensor(src, dst, scale_out, n, [](void* s, void* d, float* sc, int64_t k) {
        return lhq_fp8_quantize_per_tensor(static_cast<const float*>(s), static_cast<uint8_t*>(d), sc, k, dev::stream());
    }, "fp8_quantize_per_tensor");
}

void fp8_dequantize_per_tensor(const fp8_e4m3* src, float scale, float* dst, int64_t n) {
    per_tensor_dq(src, scale, dst, n, [](const void* s, const float* sc, float* d, int64_t k) {
        return lhq_fp8_dequantize_per_tensor(static_cast<const uint8_t*>(s), sc, d, k, dev::stream());
    }, "fp8_dequantize_per_tensor");
}

void fp8_quantize_per_row(const float* src, fp8_e4m3* dst, float* scales_out, int rows, int dim) {
    shaped(src, dst, scales_out, rows, dim, nonneg(rows), [](const float* s, void* d, float* sc, int r, int c) {
        return lhq_fp8_quantize_per_row(s, static_cast<uint8_t*>(d), sc, r, c, dev::stream());
    }, "fp8_quantize_per_row");
}

void fp8_dequantize_per_row(const fp8_e4m3* src, const float* scales, float* dst, int rows, int dim) {
    shaped_dq(src, scales, dst, rows, dim, nonneg(rows), [](const void* s, const float* sc, float* d, int r, int c) {
        return lhq_fp8_dequantize_per_row(static_cast<const uint8_t*>(s), sc, d, r, c, dev::stream());
    }, "fp8_dequantize_per_row");
}

void fp8_quantize_per_col(const float* src, fp8_e4m3* dst, float* scales_out, int rows, int cols) {
    shaped(src, dst, scales_out, rows, cols, nonneg(cols), [](const float* s, void* d, float* sc, int r, int c) {
        return lhq_fp8_quantize_per_col(s, static_cast<uint8_t*>(d), sc, r, c, dev::stream());
    }, "fp8_quantize_per_col");
}

void fp8_dequantize_per_col(const fp8_e4m3* src, const float* scales, float* dst, int rows, int cols) {
    shaped_dq(src, scales, dst, rows, cols, nonneg(cols), [](const void* s, const float* sc, float* d, int r, int c) {
        return lhq_fp8_dequantize_per_col(static_cast<const uint8_t*>(s), sc, d, r, c, dev::stream());
    }, "fp8_dequantize_per_col");
}

}  // namespace lh
