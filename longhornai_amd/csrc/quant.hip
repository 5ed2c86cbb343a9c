// quant.hip -- int8 / int4 / fp8 quantizers and dequantizers for gfx950,
// bit-exact with the reference (quant.cpp:12-249).
//
// Bit-exactness rests on three facts the kernels respect:
//   * max|x| is order-independent (the reference's `a > m` never lets NaN
//     win, quant.cpp:21-28; the kernels use the same compare-and-select), so
//     any reduction tree gives the reference's maximum;
//   * the scale uses the same IEEE operations: m / 127 (or /7, /448) and
//     1 / scale are correctly rounded divisions in HIP device code;
//   * rounding is saturate-then-round-to-nearest-even (quant.cpp:12-19), with
//     per-row / per-tensor multiplying by the reciprocal and per-column /
//     int4 group dividing by the scale, exactly as the reference does.
//   * no multiply-add is fused anywhere in this file.
#include "common.hpp"

#pragma clang fp contract(off)

namespace lhq {
namespace {

constexpr int kBlock = 256;

// max(m, a) in the reference's form `if (a > m) m = a` (quant.cpp:21-28):
// a NaN `a` never replaces m, whatever kind of NaN it is.
__device__ __forceinline__ float amax(float m, float a) { return (a > m) ? a : m; }

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = amax(v, __shfl_xor(v, off, 64));
    return v;
}

// Block-wide max of non-negative values (NaN never wins); result broadcast.
__device__ float block_max(float v) {
    __shared__ float part[kBlock / 64];
    v = wave_max(v);
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    if (lane == 0) part[w] = v;
    __syncthreads();
    float r = part[0];
#pragma unroll
    for (int i = 1; i < kBlock / 64; ++i) r = amax(r, part[i]);
    __syncthreads();
    return r;
}

template <typename T> __device__ __forceinline__ float load_f(const T* p, int64_t i);
template <> __device__ __forceinline__ float load_f<float>(const float* p, int64_t i) { return p[i]; }
template <> __device__ __forceinline__ float load_f<uint16_t>(const uint16_t* p, int64_t i) {
    return bf16_to_f32(p[i]);
}

// Quantize one value with a reciprocal (per-row / per-tensor) -- int8 or fp8.
template <bool FP8>
__device__ __forceinline__ uint8_t quant_mul(float x, float inv) {
    if constexpr (FP8) return f32_to_e4m3(x * inv);
    else return static_cast<uint8_t>(static_cast<int8_t>(sat_rint(x * inv, 127)));
}
template <bool FP8>
__device__ __forceinline__ uint8_t quant_div(float x, float s) {
    if constexpr (FP8) return f32_to_e4m3(x / s);
    else return static_cast<uint8_t>(static_cast<int8_t>(sat_rint(x / s, 127)));
}

// One workgroup per row: max-abs, scale = m / QMAX (1 if m == 0),
// inv = 1 / scale, q = round(x * inv)  (quant.cpp:52-63, 195-206).
template <typename T, bool FP8>
__global__ __launch_bounds__(kBlock) void quant_per_row_kernel(const T* __restrict__ src,
                                                               uint8_t* __restrict__ dst,
                                                               float* __restrict__ scales, int dim) {
    const int64_t base = static_cast<int64_t>(blockIdx.x) * dim;
    float m = 0.0f;
    for (int i = threadIdx.x; i < dim; i += kBlock) m = amax(m, fabsf(load_f(src, base + i)));
    m = block_max(m);
    const float qmax = FP8 ? 448.0f : 127.0f;
    const float scale = (m > 0.0f) ? m / qmax : 1.0f;
    const float inv = 1.0f / scale;
    for (int i = threadIdx.x; i < dim; i += kBlock) dst[base + i] = quant_mul<FP8>(load_f(src, base + i), inv);
    if (threadIdx.x == 0) scales[blockIdx.x] = scale;
}

// fp32 rows whose length is a multiple of 4: 16-byte loads and 4-byte
// stores; rows of up to 4 * 4 * kBlock elements stay in registers between
// the max-abs pass and the quantizing pass (one read of the row), longer
// rows are read again (from L2).  Same rule as quant_per_row_kernel.
template <bool FP8>
__global__ __launch_bounds__(kBlock) void quant_per_row_f32_vec_kernel(const float* __restrict__ src,
                                                                       uint8_t* __restrict__ dst,
                                                                       float* __restrict__ scales, int dim) {
    constexpr int R = 4;  // float4 chunks a thread keeps
    const int64_t base = static_cast<int64_t>(blockIdx.x) * dim;
    const f32x4_t* s4 = reinterpret_cast<const f32x4_t*>(src + base);
    const int n4 = dim >> 2;
    const bool cached = n4 <= R * kBlock;
    f32x4_t keep[R];
    float m = 0.0f;
    if (cached) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int i = threadIdx.x + r * kBlock;
            keep[r] = i < n4 ? s4[i] : f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int j = 0; j < 4; ++j) m = amax(m, fabsf(keep[r][j]));
        }
    } else {
        for (int i = threadIdx.x; i < n4; i += kBlock) {
            const f32x4_t v = s4[i];
#pragma unroll
            for (int j = 0; j < 4; ++j) m = amax(m, fabsf(v[j]));
        }
    }
    m = block_max(m);
    const float qmax = FP8 ? 448.0f : 127.0f;
    const float scale = (m > 0.0f) ? m / qmax : 1.0f;
    const float inv = 1.0f / scale;
    uint32_t* d4 = reinterpret_cast<uint32_t*>(dst + base);
    auto put = [&](int i, const f32x4_t& v) {
        uint32_t w = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) w |= static_cast<uint32_t>(quant_mul<FP8>(v[j], inv)) << (8 * j);
        d4[i] = w;
    };
    if (cached) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int i = threadIdx.x + r * kBlock;
            if (i < n4) put(i, keep[r]);
        }
    } else {
        for (int i = threadIdx.x; i < n4; i += kBlock) put(i, s4[i]);
    }
    if (threadIdx.x == 0) scales[blockIdx.x] = scale;
}

// bf16 rows whose length is a multiple of 8: 16-byte loads, the row is read
// twice (the second pass hits in L2), 8-byte stores.
template <bool FP8>
__global__ __launch_bounds__(kBlock) void quant_per_row_bf16_vec_kernel(const uint16_t* __restrict__ src,
                                                                        uint8_t* __restrict__ dst,
                                                                        float* __restrict__ scales,
                                                                        int dim) {
    const int64_t base = static_cast<int64_t>(blockIdx.x) * dim;
    const u32x4_t* s4 = reinterpret_cast<const u32x4_t*>(src + base);
    const int n8 = dim >> 3;
    float m = 0.0f;
    for (int i = threadIdx.x; i < n8; i += kBlock) {
        const u32x4_t v = s4[i];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            m = amax(m, fabsf(__uint_as_float(v[j] << 16)));
            m = amax(m, fabsf(__uint_as_float(v[j] & 0xffff0000u)));
        }
    }
    m = block_max(m);
    const float qmax = FP8 ? 448.0f : 127.0f;
    const float scale = (m > 0.0f) ? m / qmax : 1.0f;
    const float inv = 1.0f / scale;
    u32x2_t* d2 = reinterpret_cast<u32x2_t*>(dst + base);
    for (int i = threadIdx.x; i < n8; i += kBlock) {
        const u32x4_t v = s4[i];
        u32x2_t o;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t lo = quant_mul<FP8>(__uint_as_float(v[j] << 16), inv);
            const uint32_t hi = quant_mul<FP8>(__uint_as_float(v[j] & 0xffff0000u), inv);
            const uint32_t pair = lo | (hi << 8);
            if (j & 1) o[j >> 1] |= pair << 16;
            else o[j >> 1] = pair;
        }
        d2[i] = o;
    }
    if (threadIdx.x == 0) scales[blockIdx.x] = scale;
}

// Per-column scales (quant.cpp:75-96, 218-238), in three launches that need
// no scratch memory: the scales array first holds the running max |x| of its
// column as float bits (non-negative floats order like their bit patterns),
// then the scale m / QMAX (1 where m == 0).
//   (1) zero the scales;
//   (2) a grid of (column block) x (row chunk) workgroups: each thread reduces
//       VEC adjacent columns over kColRows rows with 16-byte loads, then one
//       atomic max per column and chunk -- the max is order-independent and
//       NaN never wins, so any split gives the reference's maximum;
//   (3) turn each max into its scale.
constexpr int kColRows = 64;

__global__ void zero_f32_kernel(float* __restrict__ p, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0.0f;
}

template <int VEC>
__global__ __launch_bounds__(kBlock) void col_max_kernel(const float* __restrict__ src,
                                                         float* __restrict__ maxw, int rows, int cols) {
    const int c0 = (blockIdx.x * kBlock + threadIdx.x) * VEC;
    if (c0 >= cols) return;
    float m[VEC];
#pragma unroll
    for (int j = 0; j < VEC; ++j) m[j] = 0.0f;
    // row chunks blockIdx.y, blockIdx.y + gridDim.y, ... (the grid's y extent
    // is capped, so very tall inputs give a workgroup several chunks)
    for (int r0 = blockIdx.y * kColRows; r0 < rows; r0 += gridDim.y * kColRows) {
        const int r1 = min(rows, r0 + kColRows);
        for (int r = r0; r < r1; ++r) {
            const float* row = src + static_cast<int64_t>(r) * cols + c0;
            if constexpr (VEC == 4) {
                const f32x4_t v = *reinterpret_cast<const f32x4_t*>(row);
#pragma unroll
                for (int j = 0; j < 4; ++j) m[j] = amax(m[j], fabsf(v[j]));
            } else {
                m[0] = amax(m[0], fabsf(row[0]));
            }
        }
    }
#pragma unroll
    for (int j = 0; j < VEC; ++j)
        if (m[j] > 0.0f) atomicMax(reinterpret_cast<unsigned int*>(maxw + c0 + j), __float_as_uint(m[j]));
}

template <bool FP8>
__global__ void col_finalize_kernel(float* __restrict__ scales, int cols) {
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= cols) return;
    const float m = scales[c];
    const float qmax = FP8 ? 448.0f : 127.0f;
    scales[c] = (m > 0.0f) ? m / qmax : 1.0f;
}

// q = round(x / scale[c]); VEC adjacent elements per thread (VEC divides cols).
template <bool FP8, int VEC>
__global__ void quant_per_col_kernel(const float* __restrict__ src, const float* __restrict__ scales,
                                     uint8_t* __restrict__ dst, int cols, int64_t n) {
    const int64_t i = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) * VEC;
    if (i >= n) return;
    const int c = static_cast<int>(i % cols);
    if constexpr (VEC == 4) {
        const f32x4_t v = *reinterpret_cast<const f32x4_t*>(src + i);
        const f32x4_t sc = *reinterpret_cast<const f32x4_t*>(scales + c);
        uint32_t o = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) o |= static_cast<uint32_t>(quant_div<FP8>(v[j], sc[j])) << (8 * j);
        *reinterpret_cast<uint32_t*>(dst + i) = o;
    } else {
        dst[i] = quant_div<FP8>(src[i], scales[c]);
    }
}

// Per-tensor: (1) clear the max word, (2) atomic max of |x| bits (non-negative
// floats order like their bit patterns; NaN is skipped), (3) quantize with the
// reciprocal, (4) turn the max into the scale.  The max lives in scale_out
// until step 4, so no scratch memory is needed.
__global__ void clear_word_kernel(float* w) { *w = 0.0f; }

__global__ void tensor_max_kernel(const float* __restrict__ src, int64_t n, float* __restrict__ maxw) {
    float m = 0.0f;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * kBlock)
        m = amax(m, fabsf(src[i]));
    m = block_max(m);
    if (threadIdx.x == 0 && m > 0.0f) atomicMax(reinterpret_cast<unsigned int*>(maxw), __float_as_uint(m));
}

template <bool FP8>
__global__ void quant_tensor_kernel(const float* __restrict__ src, uint8_t* __restrict__ dst, int64_t n,
                                    const float* __restrict__ maxw) {
    const float m = *maxw;
    const float qmax = FP8 ? 448.0f : 127.0f;
    const float scale = (m > 0.0f) ? m / qmax : 1.0f;
    const float inv = 1.0f / scale;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * kBlock)
        dst[i] = quant_mul<FP8>(src[i], inv);
}

template <bool FP8>
__global__ void finalize_tensor_scale_kernel(float* w) {
    const float m = *w;
    const float qmax = FP8 ? 448.0f : 127.0f;
    *w = (m > 0.0f) ? m / qmax : 1.0f;
}

// Dequantizers: dst = decode(src) * scale (quant.cpp:47-50, 65-73, 98-105,
// 190-193, 208-216, 240-249); MODE 0 = per-tensor, 1 = per-row, 2 = per-col.
template <bool FP8, int MODE>
__global__ void dequant_kernel(const uint8_t* __restrict__ src, const float* __restrict__ scales,
                               float* __restrict__ dst, int dim, int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float s = (MODE == 0) ? scales[0] : (MODE == 1) ? scales[i / dim] : scales[i % dim];
    const float v = FP8 ? e4m3_to_f32(src[i]) : static_cast<float>(static_cast<int8_t>(src[i]));
    dst[i] = v * s;
}

// int4 symmetric, reference layout.  Scales: a thread per (group, column):
// m = max |w| over the group, s = m / 7 (1 if 0)  (quant.cpp:128-144).
__global__ void q4_scales_kernel(const float* __restrict__ src, float* __restrict__ scales, int N, int G,
                                 int64_t total) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= total) return;
    const int n = static_cast<int>(t % N);
    const int64_t g = t / N;
    float m = 0.0f;
    for (int kk = 0; kk < G; ++kk) m = amax(m, fabsf(src[(g * G + kk) * N + n]));
    scales[t] = (m > 0.0f) ? m / 7.0f : 1.0f;
}

// Pack rows (2i, 2i+1) of column n into byte i*N + n, low nibble first; each
// row uses its own group's scale, division then saturating round to [-7, 7]
// (quant.cpp:146-159).
__global__ void q4_pack_kernel(const float* __restrict__ src, const float* __restrict__ scales,
                               uint8_t* __restrict__ packed, int N, int G, int64_t total) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= total) return;
    const int n = static_cast<int>(t % N);
    const int64_t i = t / N;
    const int64_t k = 2 * i;
    const float s0 = scales[(k / G) * N + n];
    const float s1 = scales[((k + 1) / G) * N + n];
    const int q0 = sat_rint(src[k * N + n] / s0, 7);
    const int q1 = sat_rint(src[(k + 1) * N + n] / s1, 7);
    packed[t] = static_cast<uint8_t>((q0 & 0xf) | ((q1 & 0xf) << 4));
}

__global__ void q4_dequant_kernel(const uint8_t* __restrict__ packed, const float* __restrict__ scales,
                                  float* __restrict__ dst, int N, int G, int64_t total) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= total) return;
    const int n = static_cast<int>(t % N);
    const int64_t k = t / N;
    const uint8_t b = packed[(k >> 1) * N + n];
    const int nib = (k & 1) ? (b >> 4) : (b & 0xf);
    const int q = nib >= 8 ? nib - 16 : nib;  // sign extension, quant.hpp:73-74
    dst[t] = static_cast<float>(q) * scales[(k / G) * N + n];
}

// Asymmetric int4 (no reference counterpart): per (group, column) the range
// is widened to contain 0, s = fp16((hi - lo) / 15) (1 if the range is empty,
// at least 2^-14), z = clamp(rint(-lo / s), 0, 15); codes
// u = clamp(rint(w / s) + z, 0, 15) use the fp16-rounded s.
__global__ void q4a_params_kernel(const float* __restrict__ src, uint16_t* __restrict__ scales,
                                  uint8_t* __restrict__ zeros, int N, int G, int64_t total) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= total) return;
    const int n = static_cast<int>(t % N);
    const int64_t g = t / N;
    float lo = 0.0f, hi = 0.0f;
    for (int kk = 0; kk < G; ++kk) {
        const float w = src[(g * G + kk) * N + n];
        if (w < lo) lo = w;
        if (w > hi) hi = w;
    }
    float s = (hi - lo) / 15.0f;
    if (!(s > 0.0f)) s = 1.0f;
    _Float16 sh = static_cast<_Float16>(s);  // RNE, like dtypes.hpp:17-55 for normal values
    float sq = static_cast<float>(sh);
    if (sq < 0x1p-14f) {
        sh = static_cast<_Float16>(0x1p-14f);
        sq = 0x1p-14f;
    }
    float zf = __builtin_rintf(-lo / sq);
    zf = fminf(fmaxf(zf, 0.0f), 15.0f);
    scales[t] = __builtin_bit_cast(uint16_t, sh);
    zeros[t] = static_cast<uint8_t>(zf);
}

__global__ void q4a_pack_kernel(const float* __restrict__ src, const uint16_t* __restrict__ scales,
                                const uint8_t* __restrict__ zeros, uint8_t* __restrict__ packed, int N,
                                int G, int64_t total) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= total) return;
    const int n = static_cast<int>(t % N);
    const int64_t i = t / N;
    uint32_t b = 0;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int64_t k = 2 * i + h;
        const int64_t gi = (k / G) * N + n;
        const float sq = f16_to_f32(scales[gi]);
        float v = __builtin_rintf(src[k * N + n] / sq) + static_cast<float>(zeros[gi]);
        v = fminf(fmaxf(v, 0.0f), 15.0f);
        b |= static_cast<uint32_t>(v) << (4 * h);
    }
    packed[t] = static_cast<uint8_t>(b);
}

__global__ void q4a_dequant_kernel(const uint8_t* __restrict__ packed, const uint16_t* __restrict__ scales,
                                   const uint8_t* __restrict__ zeros, float* __restrict__ dst, int N, int G,
                                   int64_t total) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= total) return;
    const int n = static_cast<int>(t % N);
    const int64_t k = t / N;
    const uint8_t b = packed[(k >> 1) * N + n];
    const int u = (k & 1) ? (b >> 4) : (b & 0xf);
    const int64_t gi = (k / G) * N + n;
    dst[t] = static_cast<float>(u - static_cast<int>(zeros[gi])) * f16_to_f32(scales[gi]);
}

inline unsigned blocks_for(int64_t n, int bs = kBlock) { return static_cast<unsigned>(ceil_div64(n, bs)); }

// Per-tensor grid: enough workgroups to cover the chip, grid-stride beyond.
inline unsigned tensor_grid(int64_t n) {
    const int64_t b = ceil_div64(n, kBlock);
    return static_cast<unsigned>(b < 2048 ? (b > 0 ? b : 1) : 2048);
}

template <bool FP8>
int quantize_per_tensor(const float* src, uint8_t* dst, float* scale_out, int64_t n, void* stream,
                        const char* who) {
    LHQ_REQUIRE(src && dst && scale_out, "%s: null pointer", who);
    LHQ_REQUIRE(n >= 0, "%s: negative n", who);
    hipStream_t s = as_stream(stream);
    clear_word_kernel<<<1, 1, 0, s>>>(scale_out);
    if (n > 0) {
        tensor_max_kernel<<<tensor_grid(n), kBlock, 0, s>>>(src, n, scale_out);
        quant_tensor_kernel<FP8><<<tensor_grid(n), kBlock, 0, s>>>(src, dst, n, scale_out);
    }
    finalize_tensor_scale_kernel<FP8><<<1, 1, 0, s>>>(scale_out);
    return check_launch(who);
}

template <bool FP8, int MODE>
int dequantize(const uint8_t* src, const float* scales, float* dst, int64_t n, int dim, void* stream,
               const char* who) {
    LHQ_REQUIRE(src && scales && dst, "%s: null pointer", who);
    LHQ_REQUIRE(n >= 0 && (MODE == 0 || dim > 0 || n == 0), "%s: bad dims", who);
    if (n == 0) return LHQ_OK;
    dequant_kernel<FP8, MODE><<<blocks_for(n), kBlock, 0, as_stream(stream)>>>(src, scales, dst, dim, n);
    return check_launch(who);
}

template <typename T, bool FP8>
int quantize_per_row(const T* src, uint8_t* dst, float* scales, int rows, int dim, void* stream,
                     const char* who) {
    LHQ_REQUIRE(src && dst && scales, "%s: null pointer", who);
    LHQ_REQUIRE(rows >= 0 && dim >= 0, "%s: negative dims", who);
    if (rows == 0) return LHQ_OK;
    hipStream_t s = as_stream(stream);
    const bool vec = sizeof(T) == 2 && dim % 8 == 0 && (reinterpret_cast<uintptr_t>(src) & 15) == 0 &&
                     (reinterpret_cast<uintptr_t>(dst) & 7) == 0;
    if constexpr (sizeof(T) == 2) {
        if (vec) {
            quant_per_row_bf16_vec_kernel<FP8><<<rows, kBlock, 0, s>>>(src, dst, scales, dim);
            return check_launch(who);
        }
    } else {
        if (dim % 4 == 0 && (reinterpret_cast<uintptr_t>(src) & 15) == 0 &&
            (reinterpret_cast<uintptr_t>(dst) & 3) == 0) {
            quant_per_row_f32_vec_kernel<FP8><<<rows, kBlock, 0, s>>>(src, dst, scales, dim);
            return check_launch(who);
        }
    }
    quant_per_row_kernel<T, FP8><<<rows, kBlock, 0, s>>>(src, dst, scales, dim);
    return check_launch(who);
}

template <bool FP8>
int quantize_per_col(const float* src, uint8_t* dst, float* scales, int rows, int cols, void* stream,
                     const char* who) {
    LHQ_REQUIRE(src && dst && scales, "%s: null pointer", who);
    LHQ_REQUIRE(rows >= 0 && cols >= 0, "%s: negative dims", who);
    if (cols == 0) return LHQ_OK;
    hipStream_t s = as_stream(stream);
    // 16-byte loads need 4 | cols and aligned rows; scales and dst are then
    // read / written in 16- and 4-byte units at multiples of 4 elements.
    const bool vec = cols % 4 == 0 && (reinterpret_cast<uintptr_t>(src) & 15) == 0 &&
                     (reinterpret_cast<uintptr_t>(scales) & 15) == 0 && (reinterpret_cast<uintptr_t>(dst) & 3) == 0;
    zero_f32_kernel<<<blocks_for(cols), kBlock, 0, s>>>(scales, cols);
    if (rows > 0) {
        const int vcols = vec ? cols / 4 : cols;
        const dim3 grid(static_cast<unsigned>(ceil_div(vcols, kBlock)),
                        static_cast<unsigned>(min(ceil_div(rows, kColRows), 65535)));
        if (vec) col_max_kernel<4><<<grid, kBlock, 0, s>>>(src, scales, rows, cols);
        else col_max_kernel<1><<<grid, kBlock, 0, s>>>(src, scales, rows, cols);
    }
    col_finalize_kernel<FP8><<<blocks_for(cols), kBlock, 0, s>>>(scales, cols);
    const int64_t n = static_cast<int64_t>(rows) * cols;
    if (n > 0) {
        if (vec) quant_per_col_kernel<FP8, 4><<<blocks_for(n / 4), kBlock, 0, s>>>(src, scales, dst, cols, n);
        else quant_per_col_kernel<FP8, 1><<<blocks_for(n), kBlock, 0, s>>>(src, scales, dst, cols, n);
    }
    return check_launch(who);
}

bool q4_dims_ok(int K, int N, int G) { return K > 0 && N > 0 && G > 0 && K % G == 0 && K % 2 == 0; }

}  // namespace
}  // namespace lhq

using namespace lhq;

extern "C" {

int lhq_q8_quantize_per_tensor(const float* src, int8_t* dst, float* scale_out, int64_t n, void* stream) {
    return quantize_per_tensor<false>(src, reinterpret_cast<uint8_t*>(dst), scale_out, n, stream,
                                      "q8_quantize_per_tensor");
}
int lhq_q8_dequantize_per_tensor(const int8_t* src, const float* scale, float* dst, int64_t n, void* stream) {
    return dequantize<false, 0>(reinterpret_cast<const uint8_t*>(src), scale, dst, n, 1, stream,
                                "q8_dequantize_per_tensor");
}
int lhq_q8_quantize_per_row(const float* src, int8_t* dst, float* scales, int rows, int dim, void* stream) {
    return quantize_per_row<float, false>(src, reinterpret_cast<uint8_t*>(dst), scales, rows, dim, stream,
                                          "q8_quantize_per_row");
}
int lhq_q8_quantize_per_row_bf16(const uint16_t* src, int8_t* dst, float* scales, int rows, int dim,
                                 void* stream) {
    return quantize_per_row<uint16_t, false>(src, reinterpret_cast<uint8_t*>(dst), scales, rows, dim, stream,
                                             "q8_quantize_per_row_bf16");
}
int lhq_q8_dequantize_per_row(const int8_t* src, const float* scales, float* dst, int rows, int dim,
                              void* stream) {
    LHQ_REQUIRE(rows >= 0 && dim >= 0, "q8_dequantize_per_row: negative dims");
    return dequantize<false, 1>(reinterpret_cast<const uint8_t*>(src), scales, dst,
                                static_cast<int64_t>(rows) * dim, dim, stream, "q8_dequantize_per_row");
}
int lhq_q8_quantize_per_col(const float* src, int8_t* dst, float* scales, int rows, int cols, void* stream) {
    return quantize_per_col<false>(src, reinterpret_cast<uint8_t*>(dst), scales, rows, cols, stream,
                                   "q8_quantize_per_col");
}
int lhq_q8_dequantize_per_col(const int8_t* src, const float* scales, float* dst, int rows, int cols,
                              void* stream) {
    LHQ_REQUIRE(rows >= 0 && cols >= 0, "q8_dequantize_per_col: negative dims");
    return dequantize<false, 2>(reinterpret_cast<const uint8_t*>(src), scales, dst,
                                static_cast<int64_t>(rows) * cols, cols, stream, "q8_dequantize_per_col");
}

int lhq_fp8_quantize_per_tensor(const float* src, uint8_t* dst, float* scale_out, int64_t n, void* stream) {
    return quantize_per_tensor<true>(src, dst, scale_out, n, stream, "fp8_quantize_per_tensor");
}
int lhq_fp8_dequantize_per_tensor(const uint8_t* src, const float* scale, float* dst, int64_t n,
                                  void* stream) {
    return dequantize<true, 0>(src, scale, dst, n, 1, stream, "fp8_dequantize_per_tensor");
}
int lhq_fp8_quantize_per_row(const float* src, uint8_t* dst, float* scales, int rows, int dim, void* stream) {
    return quantize_per_row<float, true>(src, dst, scales, rows, dim, stream, "fp8_quantize_per_row");
}
int lhq_fp8_dequantize_per_row(const uint8_t* src, const float* scales, float* dst, int rows, int dim,
                               void* stream) {
    LHQ_REQUIRE(rows >= 0 && dim >= 0, "fp8_dequantize_per_row: negative dims");
    return dequantize<true, 1>(src, scales, dst, static_cast<int64_t>(rows) * dim, dim, stream,
                               "fp8_dequantize_per_row");
}
int lhq_fp8_quantize_per_col(const float* src, uint8_t* dst, float* scales, int rows, int cols, void* stream) {
    return quantize_per_col<true>(src, dst, scales, rows, cols, stream, "fp8_quantize_per_col");
}
int lhq_fp8_dequantize_per_col(const uint8_t* src, const float* scales, float* dst, int rows, int cols,
                               void* stream) {
    LHQ_REQUIRE(rows >= 0 && cols >= 0, "fp8_dequantize_per_col: negative dims");
    return dequantize<true, 2>(src, scales, dst, static_cast<int64_t>(rows) * cols, cols, stream,
                               "fp8_dequantize_per_col");
}

int lhq_q4_quantize_groupwise(const float* src, uint8_t* packed, float* scales, int K, int N, int G,
                              void* stream) {
    LHQ_REQUIRE(src && packed && scales, "q4_quantize_groupwise: null pointer");
    LHQ_REQUIRE(q4_dims_ok(K, N, G), "q4_quantize_groupwise: need K,N,G > 0, K even, G | K (K=%d N=%d G=%d)",
                K, N, G);
    hipStream_t s = as_stream(stream);
    const int64_t ns = static_cast<int64_t>(K / G) * N, np = static_cast<int64_t>(K / 2) * N;
    q4_scales_kernel<<<blocks_for(ns), kBlock, 0, s>>>(src, scales, N, G, ns);
    q4_pack_kernel<<<blocks_for(np), kBlock, 0, s>>>(src, scales, packed, N, G, np);
    return check_launch("q4_quantize_groupwise");
}

int lhq_q4_dequantize_groupwise(const uint8_t* packed, const float* scales, float* dst, int K, int N, int G,
                                void* stream) {
    LHQ_REQUIRE(packed && scales && dst, "q4_dequantize_groupwise: null pointer");
    LHQ_REQUIRE(q4_dims_ok(K, N, G), "q4_dequantize_groupwise: bad dims (K=%d N=%d G=%d)", K, N, G);
    const int64_t n = static_cast<int64_t>(K) * N;
    q4_dequant_kernel<<<blocks_for(n), kBlock, 0, as_stream(stream)>>>(packed, scales, dst, N, G, n);
    return check_launch("q4_dequantize_groupwise");
}

int lhq_q4a_quantize_groupwise(const float* src, uint8_t* packed, uint16_t* scales, uint8_t* zeros, int K,
                               int N, int G, void* stream) {
    LHQ_REQUIRE(src && packed && scales && zeros, "q4a_quantize_groupwise: null pointer");
    LHQ_REQUIRE(q4_dims_ok(K, N, G), "q4a_quantize_groupwise: bad dims (K=%d N=%d G=%d)", K, N, G);
    hipStream_t s = as_stream(stream);
    const int64_t ns = static_cast<int64_t>(K / G) * N, np = static_cast<int64_t>(K / 2) * N;
    q4a_params_kernel<<<blocks_for(ns), kBlock, 0, s>>>(src, scales, zeros, N, G, ns);
    q4a_pack_kernel<<<blocks_for(np), kBlock, 0, s>>>(src, scales, zeros, packed, N, G, np);
    return check_launch("q4a_quantize_groupwise");
}

int lhq_q4a_dequantize_groupwise(const uint8_t* packed, const uint16_t* scales, const uint8_t* zeros,
                                 float* dst, int K, int N, int G, void* stream) {
    LHQ_REQUIRE(packed && scales && zeros && dst, "q4a_dequantize_groupwise: null pointer");
    LHQ_REQUIRE(q4_dims_ok(K, N, G), "q4a_dequantize_groupwise: bad dims (K=%d N=%d G=%d)", K, N, G);
    const int64_t n = static_cast<int64_t>(K) * N;
    q4a_dequant_kernel<<<blocks_for(n), kBlock, 0, as_stream(stream)>>>(packed, scales, zeros, dst, N, G, n);
    return check_launch("q4a_dequantize_groupwise");
}

}  // extern "C"
