// mfma_probe.hip -- matrix-core rate probes for the benchmark (a diagnostics
// library, liblonghorn_diag.so, apart from the product library: these
// kernels measure the hardware, they are not part of the quantized-GEMM
// path or of the reference interface).  bench.py reads the sustained MFMA
// rate on register operands and on the GEMMs' own operand values from them.
#include <cstdarg>
#include <cstdio>

#include "longhorn_diag.h"
#include "common.hpp"

namespace lhd {
namespace {

thread_local char g_last_error[512] = "";

int set_error(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
    return code;
}

int launch_status(const char* what) {
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? LHD_OK : set_error(LHD_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

#define LHD_REQUIRE(cond, ...)                                        \
    do {                                                              \
        if (!(cond)) return ::lhd::set_error(LHD_ERR_INVALID, __VA_ARGS__); \
    } while (0)

using lhq::as_stream;
using namespace lhq;

// Matrix-core rate probe: each wave runs `iters` rounds of four
// independent MFMA chains on register operands, with no memory traffic in
// the loop, so the launch's duration gives the matrix cores' sustained rate
// with every CU loaded (the clock and power limits included).  One result
// per workgroup goes to sink (keeps the chains live).
// KIND 0: v_mfma_i32_32x32x32_i8 (the W8A8 kernel's instruction),
// KIND 1: v_mfma_f32_16x16x32_bf16 (the W4A16 kernels' instruction),
// KIND 2: v_mfma_f32_32x32x16_bf16, KIND 3: v_mfma_i32_16x16x64_i8;
// KIND 4, 5: KIND 1's loop with 2 or 4 independent integer VALU operations
// per MFMA (does the VALU work hide under the matrix core's?).
template <int KIND>
__global__ __launch_bounds__(256) void mfma_rate_kernel(int iters, int* sink) {
    const uint32_t t = threadIdx.x;
    // bf16 operands are small normal numbers (1 + t/2^7 and 1 - t/2^8 in
    // the high half): no Inf, NaN or subnormal on any path
    constexpr bool I8 = KIND == 0 || KIND == 3;
    const uint32_t ea = I8 ? (t * 0x01010101u) ^ 0x5a3c96e1u : 0x3f803f80u + (t & 0x7fu) * 0x00010001u;
    const uint32_t eb = I8 ? (t * 0x00ff00ffu) ^ 0x1e2d3c4bu : 0x3f7f3f7fu - (t & 0x7fu) * 0x00010000u;
    const u32x4_t a = {ea, ea + 1u, ea ^ 3u, ea + 7u}, b = {eb, eb ^ 5u, eb + 2u, eb ^ 9u};
    if constexpr (KIND == 0) {
        i32x16_t c0 = {}, c1 = {}, c2 = {}, c3 = {};
        for (int i = 0; i < iters; ++i) {
            c0 = mfma_i8_32x32x32(a, b, c0);
            c1 = mfma_i8_32x32x32(b, a, c1);
            c2 = mfma_i8_32x32x32(a, a, c2);
            c3 = mfma_i8_32x32x32(b, b, c3);
        }
        int r = 0;
#pragma unroll
        for (int j = 0; j < 16; ++j) r += c0[j] ^ c1[j] ^ c2[j] ^ c3[j];
        if (t == 0) sink[blockIdx.x] = r;
    } else if constexpr (KIND == 2) {
        f32x16_t c0 = {}, c1 = {}, c2 = {}, c3 = {};
        for (int i = 0; i < iters; ++i) {
            c0 = mfma_bf16_32x32x16(a, b, c0);
            c1 = mfma_bf16_32x32x16(b, a, c1);
            c2 = mfma_bf16_32x32x16(a, a, c2);
            c3 = mfma_bf16_32x32x16(b, b, c3);
        }
        float r = 0.0f;
#pragma unroll
        for (int j = 0; j < 16; ++j) r += c0[j] + c1[j] + c2[j] + c3[j];
        if (t == 0) sink[blockIdx.x] = __float_as_int(r);
    } else if constexpr (KIND == 3) {
        i32x4_t c0 = {}, c1 = {}, c2 = {}, c3 = {};
        for (int i = 0; i < iters; ++i) {
            c0 = mfma_i8_16x16x64(a, b, c0);
            c1 = mfma_i8_16x16x64(b, a, c1);
            c2 = mfma_i8_16x16x64(a, a, c2);
            c3 = mfma_i8_16x16x64(b, b, c3);
        }
        int r = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) r += c0[j] ^ c1[j] ^ c2[j] ^ c3[j];
        if (t == 0) sink[blockIdx.x] = r;
    } else if constexpr (KIND == 6 || KIND == 7) {
        // one dependent chain: every MFMA accumulates onto the previous one's
        // result (bf16 16x16x32, or int8 16x16x64)
        using acc_t = typename std::conditional<KIND == 6, f32x4_t, i32x4_t>::type;
        acc_t c0 = {};
        for (int i = 0; i < iters; ++i) {
            if constexpr (KIND == 6) {
                c0 = mfma_bf16_16x16x32(a, b, c0);
                c0 = mfma_bf16_16x16x32(b, a, c0);
                c0 = mfma_bf16_16x16x32(a, a, c0);
                c0 = mfma_bf16_16x16x32(b, b, c0);
            } else {
                c0 = mfma_i8_16x16x64(a, b, c0);
                c0 = mfma_i8_16x16x64(b, a, c0);
                c0 = mfma_i8_16x16x64(a, a, c0);
                c0 = mfma_i8_16x16x64(b, b, c0);
            }
        }
        if constexpr (KIND == 6) {
            float r = 0.0f;
#pragma unroll
            for (int j = 0; j < 4; ++j) r += c0[j];
            if (t == 0) sink[blockIdx.x] = __float_as_int(r);
        } else {
            int r = 0;
#pragma unroll
            for (int j = 0; j < 4; ++j) r += c0[j];
            if (t == 0) sink[blockIdx.x] = r;
        }
    } else if constexpr (KIND == 4 || KIND == 5) {
        constexpr int NV = KIND == 4 ? 2 : 4;  // VALU operations per MFMA
        f32x4_t c0 = {}, c1 = {}, c2 = {}, c3 = {};
        uint32_t v[4] = {ea, eb, ea ^ eb, ea + eb};
        for (int i = 0; i < iters; ++i) {
            c0 = mfma_bf16_16x16x32(a, b, c0);
#pragma unroll
            for (int q = 0; q < NV; ++q) v[q] = __builtin_amdgcn_perm(v[q], v[(q + 1) & 3], 0x05010400u) + 0x01010101u;
            c1 = mfma_bf16_16x16x32(b, a, c1);
#pragma unroll
            for (int q = 0; q < NV; ++q) v[q] = __builtin_amdgcn_perm(v[q], v[(q + 2) & 3], 0x07030602u) ^ 0x80808080u;
            c2 = mfma_bf16_16x16x32(a, a, c2);
#pragma unroll
            for (int q = 0; q < NV; ++q) v[q] = __builtin_amdgcn_perm(v[q], v[(q + 3) & 3], 0x05040100u) + 0x00ff00ffu;
            c3 = mfma_bf16_16x16x32(b, b, c3);
#pragma unroll
            for (int q = 0; q < NV; ++q) v[q] = __builtin_amdgcn_perm(v[q], v[(q + 1) & 3], 0x07060302u) ^ 0x0f0f0f0fu;
        }
        float r = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; ++j) r += c0[j] + c1[j] + c2[j] + c3[j];
        if (t == 0) sink[blockIdx.x] = __float_as_int(r) ^ static_cast<int>(v[0] ^ v[1] ^ v[2] ^ v[3]);
    } else {
        f32x4_t c0 = {}, c1 = {}, c2 = {}, c3 = {};
        for (int i = 0; i < iters; ++i) {
            c0 = mfma_bf16_16x16x32(a, b, c0);
            c1 = mfma_bf16_16x16x32(b, a, c1);
            c2 = mfma_bf16_16x16x32(a, a, c2);
            c3 = mfma_bf16_16x16x32(b, b, c3);
        }
        float r = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; ++j) r += c0[j] + c1[j] + c2[j] + c3[j];
        if (t == 0) sink[blockIdx.x] = __float_as_int(r);
    }
}


// Matrix-core rate on operands read from memory, in a GEMM tile's issue
// order.  Each wave loads two sets of 8 operand fragments (4 A blocks, 4 B
// blocks) once; one round is two k steps, each issuing one MFMA on each of
// the 16 accumulators (A block i x B block j) in turn, as the W8A8 and FP8
// tiles do.  There is no memory traffic in the loop, but the operand values
// are the caller's: the matrix cores draw more power on dense, changing bit
// patterns, and under the power limit the clock falls with it.
// KIND 0: v_mfma_i32_32x32x32_i8 (16-byte fragments), KIND 1:
// v_mfma_scale_f32_32x32x64_f8f6f4 on e4m3 with unit scales (32-byte
// fragments, low halves at ops, high halves at ops + 16 KiB), KIND 2:
// v_mfma_f32_16x16x32_bf16 (16-byte fragments), KINDs 3 and 4: KIND 0's
// instruction and operands issued as k chains of 2 and 4 on one accumulator
// (32 and 64 MFMAs per iteration; KIND 0-2 issue 32), KINDs 5 and 6:
// v_mfma_i32_16x16x64_i8 on the same fragments as k chains of 4 (64 MFMAs
// per iteration) and one per accumulator in turn (32), KIND 7: the same
// as k chains of 2 (32).  Fragment x of set s for
// lane l: the 16 bytes at ops + ((8s + x) * 64 + l) * 16.
// clocks (optional): per workgroup, wave 0's shader-clock ticks
// (s_memtime) and 100 MHz reference ticks (s_memrealtime) over its loop.
template <int KIND>
__global__ __launch_bounds__(256) void mfma_operand_rate_kernel(const uint8_t* __restrict__ ops, int iters,
                                                                int* sink, unsigned long long* clocks) {
    const int lane = threadIdx.x & 63;
    u32x4_t f[2][8], h[2][8];
#pragma unroll
    for (int st = 0; st < 2; ++st)
#pragma unroll
        for (int x = 0; x < 8; ++x) {
            const size_t off = static_cast<size_t>((8 * st + x) * 64 + lane) * 16;
            f[st][x] = *reinterpret_cast<const u32x4_t*>(ops + off);
            if constexpr (KIND == 1) h[st][x] = *reinterpret_cast<const u32x4_t*>(ops + 16384 + off);
        }
    using acc_t = typename std::conditional<KIND == 0 || KIND >= 3, i32x16_t,
                                            typename std::conditional<KIND == 1, f32x16_t, f32x4_t>::type>::type;
    acc_t acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = acc_t{};
    i32x4_t acc4[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc4[i][j] = i32x4_t{};
    const unsigned long long t0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
    for (int it = 0; it < iters; ++it) {
        if constexpr (KIND == 7) {
            // v_mfma_i32_16x16x64_i8 as k chains of 2 (32 MFMAs per iteration)
#pragma unroll
            for (int t = 0; t < 16; ++t)
#pragma unroll
                for (int kk = 0; kk < 2; ++kk) {
                    const int i = t / 4, j = t % 4;
                    acc4[i][j] = mfma_i8_16x16x64(f[kk][4 + j], f[kk][i], acc4[i][j]);
                    __builtin_amdgcn_sched_barrier(0);
                }
        } else if constexpr (KIND == 5 || KIND == 6) {
            // v_mfma_i32_16x16x64_i8 on the same fragments (16 bytes of a
            // 16x64 block per lane): KIND 5 as k chains of 4 on one
            // accumulator, KIND 6 one MFMA per accumulator in turn
#pragma unroll
            for (int r = 0; r < (KIND == 5 ? 16 : 2); ++r)
#pragma unroll
                for (int c = 0; c < (KIND == 5 ? 4 : 16); ++c) {
                    const int t = KIND == 5 ? r : c, kk = KIND == 5 ? (c & 1) : r;
                    const int i = t / 4, j = t % 4;
                    acc4[i][j] = mfma_i8_16x16x64(f[kk][4 + j], f[kk][i], acc4[i][j]);
                    __builtin_amdgcn_sched_barrier(0);
                }
        } else if constexpr (KIND == 3 || KIND == 4) {
            // k chains: 2 (KIND 3) or 4 (KIND 4) MFMAs in a row on one
            // accumulator, each taking the previous one's result as SrcC
            constexpr int kChain = KIND == 3 ? 2 : 4;
#pragma unroll
            for (int t = 0; t < 16; ++t)
#pragma unroll
                for (int c = 0; c < kChain; ++c) {
                    const int i = t / 4, j = t % 4, kk = c & 1;
                    acc[i][j] = mfma_i8_32x32x32(f[kk][4 + j], f[kk][i], acc[i][j]);
                    __builtin_amdgcn_sched_barrier(0);
                }
        } else {
#pragma unroll
            for (int kk = 0; kk < 2; ++kk)
#pragma unroll
                for (int t = 0; t < 16; ++t) {
                    const int i = t / 4, j = t % 4;
                    if constexpr (KIND == 0)
                        acc[i][j] = mfma_i8_32x32x32(f[kk][4 + j], f[kk][i], acc[i][j]);
                    else if constexpr (KIND == 1)
                        acc[i][j] = mfma_fp8_32x32x64(f[kk][4 + j], h[kk][4 + j], f[kk][i], h[kk][i], acc[i][j]);
                    else
                        acc[i][j] = mfma_bf16_16x16x32(f[kk][4 + j], f[kk][i], acc[i][j]);
                    __builtin_amdgcn_sched_barrier(0);
                }
        }
    }
    const unsigned long long t1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
    int r = 0;
    float rf = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int e = 0; e < static_cast<int>(sizeof(acc_t) / 4); ++e) {
                if constexpr (KIND == 0 || KIND >= 3) r += acc[i][j][e];
                else rf += acc[i][j][e];
            }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) r += acc4[i][j][e];
    if (threadIdx.x == 0) {
        sink[blockIdx.x] = (KIND == 0 || KIND >= 3) ? r : __float_as_int(rf);
        if (clocks) {
            clocks[2 * blockIdx.x] = t1 - t0;
            clocks[2 * blockIdx.x + 1] = r1 - r0;
        }
    }
}

}  // namespace
}  // namespace lhd

using namespace lhd;

extern "C" const char* lhd_last_error(void) { return lhd::g_last_error; }

extern "C" int lhd_probe_mfma_rate(int kind, int blocks, int iters, int* sink, void* stream) {
    LHD_REQUIRE(sink, "probe_mfma_rate: null sink");
    LHD_REQUIRE(kind >= 0 && kind <= 7, "probe_mfma_rate: kind %d (0..7)", kind);
    LHD_REQUIRE(blocks >= 1 && iters >= 1, "probe_mfma_rate: blocks %d, iters %d", blocks, iters);
    hipStream_t s = as_stream(stream);
    if (kind == 0) mfma_rate_kernel<0><<<blocks, 256, 0, s>>>(iters, sink);
    else if (kind == 1) mfma_rate_kernel<1><<<blocks, 256, 0, s>>>(iters, sink);
    else if (kind == 2) mfma_rate_kernel<2><<<blocks, 256, 0, s>>>(iters, sink);
    else if (kind == 3) mfma_rate_kernel<3><<<blocks, 256, 0, s>>>(iters, sink);
    else if (kind == 4) mfma_rate_kernel<4><<<blocks, 256, 0, s>>>(iters, sink);
    else if (kind == 5) mfma_rate_kernel<5><<<blocks, 256, 0, s>>>(iters, sink);
    else if (kind == 6) mfma_rate_kernel<6><<<blocks, 256, 0, s>>>(iters, sink);
    else mfma_rate_kernel<7><<<blocks, 256, 0, s>>>(iters, sink);
    return launch_status("probe_mfma_rate");
}

extern "C" int lhd_probe_mfma_operands(int kind, const void* operands, int blocks, int iters, int* sink,
                                       unsigned long long* clocks, void* stream) {
    LHD_REQUIRE(operands && sink, "probe_mfma_operands: null operands or sink");
    LHD_REQUIRE(kind >= 0 && kind <= 7, "probe_mfma_operands: kind %d (0..7)", kind);
    LHD_REQUIRE(blocks >= 1 && iters >= 1, "probe_mfma_operands: blocks %d, iters %d", blocks, iters);
    hipStream_t s = as_stream(stream);
    auto src = static_cast<const uint8_t*>(operands);
    if (kind == 0) mfma_operand_rate_kernel<0><<<blocks, 256, 0, s>>>(src, iters, sink, clocks);
    else if (kind == 1) mfma_operand_rate_kernel<1><<<blocks, 256, 0, s>>>(src, iters, sink, clocks);
    else if (kind == 2) mfma_operand_rate_kernel<2><<<blocks, 256, 0, s>>>(src, iters, sink, clocks);
    else if (kind == 3) mfma_operand_rate_kernel<3><<<blocks, 256, 0, s>>>(src, iters, sink, clocks);
    else if (kind == 4) mfma_operand_rate_kernel<4><<<blocks, 256, 0, s>>>(src, iters, sink, clocks);
    else if (kind == 5) mfma_operand_rate_kernel<5><<<blocks, 256, 0, s>>>(src, iters, sink, clocks);
    else if (kind == 6) mfma_operand_rate_kernel<6><<<blocks, 256, 0, s>>>(src, iters, sink, clocks);
    else mfma_operand_rate_kernel<7><<<blocks, 256, 0, s>>>(src, iters, sink, clocks);
    return launch_status("probe_mfma_operands");
}

