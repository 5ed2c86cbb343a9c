// prepack.hip -- one-time re-tiling of quantized weights into the layouts the
// gfx950 GEMM kernels stream.
//
// The reference keeps int4 weights as [K/2, N] bytes (quant.hpp:52-59) and
// int8 weights as [K, N] (gemm_quant.hpp:37), and reads them with a stride of
// N bytes per k step (gemm_quant.cpp:42, quant.hpp:71).  On the GPU that
// stride would make every wave touch K/2 separate rows for one column; these
// kernels rewrite the weights once so each wave reads contiguous 1 KiB runs
// that are already in MFMA operand order.
#include "common.hpp"

namespace lhq {
namespace {

// One thread per (tile, lane): assemble the 16 bytes lane `l` of tile
// (nt, kt) will load -- the four 16x16x32 B operands of column 16*nt + (l&15).
template <bool ASYM>
__global__ void w4_prepack_qweight_kernel(const uint8_t* __restrict__ packed,
                                          uint8_t* __restrict__ qweight, int K, int N,
                                          int Kt, int64_t total_lanes) {
    int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= total_lanes) return;
    const int lane = static_cast<int>(t & 63);
    const int64_t tile = t >> 6;
    const int kt = static_cast<int>(tile % Kt);
    const int nt = static_cast<int>(tile / Kt);
    const int n = nt * kW4TileN + (lane & 15);
    u32x4_t out;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        uint32_t d = 0;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int k = kt * kW4TileK + 32 * j + 8 * (lane >> 4) + e;
            uint32_t u = 0;
            if (n < N && k < K) {
                const uint8_t b = packed[static_cast<int64_t>(k >> 1) * N + n];
                const uint32_t nib = (k & 1) ? (b >> 4) : (b & 0xfu);
                // symmetric: two's-complement q in [-8,7] -> q + 8 (quant.hpp:73-74)
                u = ASYM ? nib : ((nib ^ 8u) & 0xfu);
            }
            d |= u << (4 * w4_slot(e));
        }
        out[j] = d;
    }
    *reinterpret_cast<u32x4_t*>(qweight + t * 16) = out;
}

template <typename S>
__global__ void w4_prepack_scales_kernel(const S* __restrict__ scales, S* __restrict__ out,
                                         int N, int NG, int64_t total) {
    int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= total) return;
    const int c = static_cast<int>(t & 15);
    const int64_t r = t >> 4;
    const int g = static_cast<int>(r % NG);
    const int nt = static_cast<int>(r / NG);
    const int n = nt * kW4TileN + c;
    out[t] = (n < N) ? scales[static_cast<int64_t>(g) * N + n] : S(0);
}

__global__ void w4_prepack_zeros_kernel(const uint8_t* __restrict__ zeros,
                                        uint32_t* __restrict__ out, int N, int NG, int NG8,
                                        int64_t total) {
    int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= total) return;
    const int c = static_cast<int>(t & 15);
    const int64_t r = t >> 4;
    const int g8 = static_cast<int>(r % NG8);
    const int nt = static_cast<int>(r / NG8);
    const int n = nt * kW4TileN + c;
    uint32_t v = 0;
    if (n < N) {
        for (int i = 0; i < 8; ++i) {
            const int g = g8 * 8 + i;
            if (g < NG) v |= (static_cast<uint32_t>(zeros[static_cast<int64_t>(g) * N + n]) & 0xfu) << (4 * i);
        }
    }
    out[t] = v;
}

// Bt[n][k] = B[k][n] for n < N, k < K, zero elsewhere: a 64x64-byte tile is
// transposed through LDS so both the reads and the writes are coalesced.
__global__ __launch_bounds__(256) void b8_prepack_kernel(const uint8_t* __restrict__ B,
                                                        uint8_t* __restrict__ Bt, int K, int N,
                                                        int Kp) {
    __shared__ uint8_t tile[64][65];
    const int k0 = blockIdx.x * 64, n0 = blockIdx.y * 64;
    for (int i = threadIdx.x; i < 64 * 64; i += 256) {
        const int kk = i >> 6, nn = i & 63;
        const int k = k0 + kk, n = n0 + nn;
        tile[kk][nn] = (k < K && n < N) ? B[static_cast<int64_t>(k) * N + n] : 0;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < 64 * 64; i += 256) {
        const int nn = i >> 6, kk = i & 63;
        Bt[static_cast<int64_t>(n0 + nn) * Kp + k0 + kk] = tile[kk][nn];
    }
}

// Interleave two prepacked W4 tensors by column tile: output block 2i is
// block i of `a`, block 2i + 1 is block i of `b` (a block is everything one
// column tile owns: blk16 16-byte units).  One 16-byte copy per thread.
__global__ void w4_interleave_kernel(const u32x4_t* __restrict__ a, const u32x4_t* __restrict__ b,
                                     u32x4_t* __restrict__ out, int64_t blk16, int64_t total16) {
    const int64_t d = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (d >= total16) return;
    const int64_t blk = d / blk16, off = d - blk * blk16;
    const u32x4_t* src = (blk & 1) ? b : a;
    out[d] = src[(blk >> 1) * blk16 + off];
}

int launch_interleave(const void* a, const void* b, void* out, int64_t blk_bytes, int tiles, hipStream_t s) {
    const int64_t blk16 = blk_bytes / 16, total16 = 2 * blk16 * tiles;
    if (total16 == 0) return LHQ_OK;
    w4_interleave_kernel<<<static_cast<unsigned>(ceil_div64(total16, 256)), 256, 0, s>>>(
        static_cast<const u32x4_t*>(a), static_cast<const u32x4_t*>(b), static_cast<u32x4_t*>(out), blk16, total16);
    return check_launch("w4_interleave_gate_up");
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

}  // namespace lhq

using namespace lhq;

extern "C" {

int lhq_w4_prepack_sym(const uint8_t* packed, const float* scales, int K, int N, int G,
                       uint8_t* qweight, float* scales_out, void* stream) {
    LHQ_REQUIRE(packed && scales && qweight && scales_out, "w4_prepack_sym: null pointer");
    LHQ_REQUIRE(w4_dims_ok(K, N, G), "w4_prepack_sym: need K,N,G > 0, K even, G | K (K=%d N=%d G=%d)", K, N, G);
    const int Nt = ceil_div(N, kW4TileN), Kt = ceil_div(K, kW4TileK), NG = K / G;
    const int64_t lanes = static_cast<int64_t>(Nt) * Kt * 64;
    hipStream_t s = as_stream(stream);
    w4_prepack_qweight_kernel<false><<<static_cast<unsigned>(ceil_div64(lanes, 256)), 256, 0, s>>>(
        packed, qweight, K, N, Kt, lanes);
    const int64_t ns = static_cast<int64_t>(Nt) * NG * 16;
    w4_prepack_scales_kernel<float><<<static_cast<unsigned>(ceil_div64(ns, 256)), 256, 0, s>>>(
        scales, scales_out, N, NG, ns);
    return check_launch("w4_prepack_sym");
}

int lhq_w4_prepack_asym(const uint8_t* packed, const uint16_t* scales_f16, const uint8_t* zeros,
                        int K, int N, int G, uint8_t* qweight, uint16_t* scales_out,
                        uint32_t* zeros_out, void* stream) {
    LHQ_REQUIRE(packed && scales_f16 && zeros && qweight && scales_out && zeros_out,
                "w4_prepack_asym: null pointer");
    LHQ_REQUIRE(w4_dims_ok(K, N, G), "w4_prepack_asym: need K,N,G > 0, K even, G | K (K=%d N=%d G=%d)", K, N, G);
    const int Nt = ceil_div(N, kW4TileN), Kt = ceil_div(K, kW4TileK), NG = K / G;
    const int NG8 = ceil_div(NG, 8);
    const int64_t lanes = static_cast<int64_t>(Nt) * Kt * 64;
    hipStream_t s = as_stream(stream);
    w4_prepack_qweight_kernel<true><<<static_cast<unsigned>(ceil_div64(lanes, 256)), 256, 0, s>>>(
        packed, qweight, K, N, Kt, lanes);
    const int64_t ns = static_cast<int64_t>(Nt) * NG * 16;
    w4_prepack_scales_kernel<uint16_t><<<static_cast<unsigned>(ceil_div64(ns, 256)), 256, 0, s>>>(
        scales_f16, scales_out, N, NG, ns);
    const int64_t nz = static_cast<int64_t>(Nt) * NG8 * 16;
    w4_prepack_zeros_kernel<<<static_cast<unsigned>(ceil_div64(nz, 256)), 256, 0, s>>>(
        zeros, zeros_out, N, NG, NG8, nz);
    return check_launch("w4_prepack_asym");
}

int lhq_w4_interleave_gate_up(const uint8_t* gate_qweight, const uint16_t* gate_scales,
                              const uint32_t* gate_zeros, const uint8_t* up_qweight,
                              const uint16_t* up_scales, const uint32_t* up_zeros, int K, int I, int G,
                              uint8_t* qweight, uint16_t* scales_out, uint32_t* zeros_out, void* stream) {
    LHQ_REQUIRE(gate_qweight && gate_scales && gate_zeros && up_qweight && up_scales && up_zeros && qweight &&
                    scales_out && zeros_out,
                "w4_interleave_gate_up: null pointer");
    LHQ_REQUIRE(w4_dims_ok(K, I, G), "w4_interleave_gate_up: need K,I,G > 0, K even, G | K (K=%d I=%d G=%d)", K, I,
                G);
    const void* all[9] = {gate_qweight, gate_scales, gate_zeros, up_qweight, up_scales, up_zeros,
                          qweight,      scales_out,  zeros_out};
    for (const void* ptr : all) LHQ_REQUIRE(aligned16(ptr), "w4_interleave_gate_up: pointers must be 16-byte aligned");
    const int Nt = ceil_div(I, kW4TileN), Kt = ceil_div(K, kW4TileK), NG = K / G, NG8 = ceil_div(NG, 8);
    hipStream_t s = as_stream(stream);
    if (int st = launch_interleave(gate_qweight, up_qweight, qweight, static_cast<int64_t>(Kt) * kW4TileBytes, Nt, s))
        return st;
    if (int st = launch_interleave(gate_scales, up_scales, scales_out, static_cast<int64_t>(NG) * kW4TileN * 2, Nt, s))
        return st;
    return launch_interleave(gate_zeros, up_zeros, zeros_out, static_cast<int64_t>(NG8) * kW4TileN * 4, Nt, s);
}

int64_t lhq_b8_prepacked_bytes(int K, int N) {
    if (K <= 0 || N <= 0) return 0;
    return static_cast<int64_t>(ceil_div(N, 256)) * 256 * (static_cast<int64_t>(ceil_div(K, 128)) * 128);
}

int lhq_b8_prepack(const uint8_t* B, int K, int N, uint8_t* Bt, void* stream) {
    LHQ_REQUIRE(B && Bt, "b8_prepack: null pointer");
    LHQ_REQUIRE(K > 0 && N > 0, "b8_prepack: need K, N > 0 (K=%d N=%d)", K, N);
    const int Kp = ceil_div(K, 128) * 128, Np = ceil_div(N, 256) * 256;
    dim3 grid(Kp / 64, Np / 64);
    b8_prepack_kernel<<<grid, 256, 0, as_stream(stream)>>>(B, Bt, K, N, Kp);
    return check_launch("b8_prepack");
}

}  // extern "C"
