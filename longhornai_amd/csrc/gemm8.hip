// gemm8.hip -- 8-bit-operand GEMMs for gfx950: W8A8 int8 (int32 accumulate)
// and FP8 E4M3 (fp32 accumulate), LDS-staged MFMA tiles.
//
// Reference: gemm_w8a8 (gemm_quant.cpp:29-49) runs an int32 dot product per
// output with B strided by N, then C += ((alpha*a_s)*b_s)*float(acc);
// gemm_fp8_e4m3 (gemm_quant.cpp:87-104) accumulates decoded e4m3 products in
// fp32 and adds ((alpha*sA)*sB)*acc.
//
// Here a 256-thread workgroup owns a 256x256 output tile; the four waves
// (2x2) each own 128x128 = 4x4 blocks of 32x32 MFMA accumulators.  A (row
// major [M,K]) and the prepacked k-contiguous B^T ([Np,Kp], lhq_b8_prepack)
// are staged through double-buffered LDS tiles of 256 x 128 bytes with a
// 16-byte row pad (conflict-free 128-bit LDS reads).  Integer accumulation is
// exact, so the int32 result equals the reference's bit for bit at any tiling;
// the fp32 epilogue repeats the reference's multiply order with no fused
// multiply-add, so the fp32 output is bit-exact too.  Workgroups are mapped
// XCD-aware: consecutive tiles of one group of tile rows land on one XCD so
// its L2 sees the A rows and B columns they share.
#include <cstdlib>
#include <type_traits>

#include "common.hpp"

#pragma clang fp contract(off)

namespace lhq {
namespace {

constexpr int BM = 256, BN = 256, BK = 128;
constexpr int LROW = BK + 16;                 // LDS row pitch in bytes
constexpr int TILE_BYTES = BM * LROW;         // one operand tile
constexpr int NTHREADS = 256;
constexpr int CHUNKS = BM * BK / 16 / NTHREADS;  // 16-byte chunks per thread per operand (8)

enum : int { OP_I8 = 0, OP_FP8 = 1 };
enum : int { EPI_I32 = 0, EPI_F32 = 1, EPI_BF16 = 2 };

struct Gemm8Args {
    const uint8_t* A;
    const uint8_t* Bt;
    const float* As;  // int8: per-row scales [M]; fp8: per-tensor scale (1 value)
    const float* Bs;  // int8: per-col scales [N]; fp8: per-tensor scale (1 value)
    void* C;
    int M, N, K, Kp;
    int tiles_m, tiles_n, group_m;
    float alpha, beta;
};

// Tile order: workgroup b runs on XCD (b % 8); give each XCD a contiguous
// range of tile ids, and walk tile ids in groups of `group_m` tile rows
// (column-major inside a group) so concurrently running tiles share A rows
// and B columns.
__device__ __forceinline__ void tile_of(int b, const Gemm8Args& p, int& tm, int& tn) {
    // XCD x receives blocks x, x+8, ...: q + (x < r) of them; hand it the
    // contiguous id range starting at x*q + min(x, r) (a bijection).
    const int total = p.tiles_m * p.tiles_n;
    const int q = total / 8, r = total % 8;
    const int xcd = b % 8, slot = b / 8;
    const int id = xcd * q + min(xcd, r) + slot;
    const int gm = p.group_m;
    const int per_group = gm * p.tiles_n;
    const int group = id / per_group;
    const int first = group * gm;
    const int rows = min(p.tiles_m - first, gm);
    const int in = id - group * per_group;
    tm = first + in % rows;
    tn = in / rows;
}

template <int OP, int EPI>
__global__ __launch_bounds__(NTHREADS) void gemm8_kernel(Gemm8Args p) {
    __shared__ __attribute__((aligned(16))) uint8_t lds[2][2][TILE_BYTES];

    int tm, tn;
    tile_of(blockIdx.x, p, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;

    // global -> register staging
    u32x4_t ra[CHUNKS], rb[CHUNKS];
    auto load_stage = [&](int k0) {
#pragma unroll
        for (int i = 0; i < CHUNKS; ++i) {
            const int c = tid + NTHREADS * i;
            const int r = c >> 3, kc = (c & 7) * 16;
            const int gm = m0 + r, gk = k0 + kc;
            if (gm < p.M && gk < p.K)
                ra[i] = *reinterpret_cast<const u32x4_t*>(p.A + static_cast<int64_t>(gm) * p.K + gk);
            else
                ra[i] = u32x4_t{0, 0, 0, 0};
            rb[i] = *reinterpret_cast<const u32x4_t*>(p.Bt + static_cast<int64_t>(n0 + r) * p.Kp + gk);
        }
    };
    auto store_stage = [&](int buf) {
#pragma unroll
        for (int i = 0; i < CHUNKS; ++i) {
            const int c = tid + NTHREADS * i;
            const int r = c >> 3, kc = (c & 7) * 16;
            *reinterpret_cast<u32x4_t*>(&lds[buf][0][r * LROW + kc]) = ra[i];
            *reinterpret_cast<u32x4_t*>(&lds[buf][1][r * LROW + kc]) = rb[i];
        }
    };

    using Acc = typename std::conditional<OP == OP_I8, i32x16_t, f32x16_t>::type;
    Acc acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = Acc{};

    const int nk = p.Kp / BK;
    load_stage(0);
    store_stage(0);
    __syncthreads();

    const int a_off = (wm * 128 + (lane & 31)) * LROW + 16 * (lane >> 5);
    const int b_off = (wn * 128 + (lane & 31)) * LROW + 16 * (lane >> 5);
    for (int kt = 0; kt < nk; ++kt) {
        const int buf = kt & 1;
        if (kt + 1 < nk) load_stage((kt + 1) * BK);
        const uint8_t* la = &lds[buf][0][a_off];
        const uint8_t* lb = &lds[buf][1][b_off];
#pragma unroll
        for (int kk = 0; kk < BK / 32; ++kk) {
            u32x4_t fa[4], fb[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                fa[i] = *reinterpret_cast<const u32x4_t*>(la + i * 32 * LROW + kk * 32);
                fb[i] = *reinterpret_cast<const u32x4_t*>(lb + i * 32 * LROW + kk * 32);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    if constexpr (OP == OP_I8) {
                        acc[i][j] = mfma_i8_32x32x32(fa[i], fb[j], acc[i][j]);
                    } else {
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_fp8_fp8(
                            __builtin_bit_cast(long, u32x2_t{fa[i][0], fa[i][1]}),
                            __builtin_bit_cast(long, u32x2_t{fb[j][0], fb[j][1]}), acc[i][j], 0, 0, 0);
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_fp8_fp8(
                            __builtin_bit_cast(long, u32x2_t{fa[i][2], fa[i][3]}),
                            __builtin_bit_cast(long, u32x2_t{fb[j][2], fb[j][3]}), acc[i][j], 0, 0, 0);
                    }
                }
        }
        if (kt + 1 < nk) store_stage(buf ^ 1);
        __syncthreads();
    }

    // Epilogue.  Lane l of block (i, j) holds rows 8*(e>>2) + 4*(l>>5) + (e&3)
    // and column l & 31 of that 32x32 block.
    float combined = 0.0f;
    if constexpr (OP == OP_FP8) {
        if constexpr (EPI != EPI_I32) {
            combined = p.alpha * p.As[0];
            combined = combined * p.Bs[0];
        }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int col = n0 + wn * 128 + j * 32 + (lane & 31);
        if (col >= p.N) continue;
        float bs = 0.0f;
        if constexpr (OP == OP_I8 && EPI != EPI_I32) bs = p.Bs[col];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int row = m0 + wm * 128 + i * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
                if (row >= p.M) continue;
                const int64_t o = static_cast<int64_t>(row) * p.N + col;
                if constexpr (EPI == EPI_I32) {
                    static_cast<int32_t*>(p.C)[o] = acc[i][j][e];
                } else {
                    float f;
                    if constexpr (OP == OP_I8) {
                        f = p.alpha * p.As[row];            // gemm_quant.cpp:44-45, left to right
                        f = f * bs;
                        f = f * static_cast<float>(acc[i][j][e]);
                    } else {
                        f = combined * acc[i][j][e];        // gemm_quant.cpp:101
                    }
                    if constexpr (EPI == EPI_F32) {
                        float* Cp = static_cast<float*>(p.C);
                        // apply_beta (gemm_quant.cpp:12-21), then C += rescaled
                        const float base = (p.beta == 0.0f) ? 0.0f
                                           : (p.beta == 1.0f) ? Cp[o] : Cp[o] * p.beta;
                        Cp[o] = base + f;
                    } else {
                        static_cast<uint16_t*>(p.C)[o] = f32_to_bf16(0.0f + f);
                    }
                }
            }
        }
    }
}

int env_int(const char* name, int dflt) {
    const char* v = std::getenv(name);
    return v ? std::atoi(v) : dflt;
}

template <int OP, int EPI>
int launch_gemm8(const uint8_t* A, const uint8_t* Bt, const float* As, const float* Bs, void* C, int M,
                 int N, int K, float alpha, float beta, void* stream, const char* who) {
    LHQ_REQUIRE(M >= 0 && N > 0 && K > 0, "%s: bad dims M=%d N=%d K=%d", who, M, N, K);
    LHQ_SUPPORTED(K % 16 == 0, "%s: K=%d must be a multiple of 16 (pad A and B with zeros)", who, K);
    LHQ_REQUIRE(Bt && C && (A || M == 0), "%s: null pointer", who);
    if (EPI != EPI_I32) LHQ_REQUIRE(As && Bs, "%s: null scale pointer", who);
    if (M == 0) return LHQ_OK;
    static const int group_m = env_int("LHQ_GEMM8_GROUP_M", 4);
    Gemm8Args p{};
    p.A = A; p.Bt = Bt; p.As = As; p.Bs = Bs; p.C = C;
    p.M = M; p.N = N; p.K = K; p.Kp = ceil_div(K, BK) * BK;
    p.tiles_m = ceil_div(M, BM);
    p.tiles_n = ceil_div(N, BN);
    p.group_m = group_m > 0 ? group_m : 4;
    p.alpha = alpha; p.beta = beta;
    const int tiles = p.tiles_m * p.tiles_n;
    gemm8_kernel<OP, EPI><<<tiles, NTHREADS, 0, as_stream(stream)>>>(p);
    return check_launch(who);
}

}  // namespace
}  // namespace lhq

using namespace lhq;

extern "C" {

int lhq_gemm_w8a8(const int8_t* Aq, const int8_t* Bt, const float* A_s, const float* B_s, float* C, int M,
                  int N, int K, float alpha, float beta, void* stream) {
    return launch_gemm8<OP_I8, EPI_F32>(reinterpret_cast<const uint8_t*>(Aq),
                                        reinterpret_cast<const uint8_t*>(Bt), A_s, B_s, C, M, N, K, alpha,
                                        beta, stream, "gemm_w8a8");
}

int lhq_gemm_w8a8_bf16(const int8_t* Aq, const int8_t* Bt, const float* A_s, const float* B_s, uint16_t* C,
                       int M, int N, int K, void* stream) {
    return launch_gemm8<OP_I8, EPI_BF16>(reinterpret_cast<const uint8_t*>(Aq),
                                         reinterpret_cast<const uint8_t*>(Bt), A_s, B_s, C, M, N, K, 1.0f,
                                         0.0f, stream, "gemm_w8a8_bf16");
}

int lhq_gemm_w8a8_i32(const int8_t* Aq, const int8_t* Bt, int32_t* acc, int M, int N, int K, void* stream) {
    return launch_gemm8<OP_I8, EPI_I32>(reinterpret_cast<const uint8_t*>(Aq),
                                        reinterpret_cast<const uint8_t*>(Bt), nullptr, nullptr, acc, M, N, K,
                                        1.0f, 0.0f, stream, "gemm_w8a8_i32");
}

int lhq_gemm_fp8_e4m3(const uint8_t* A, const uint8_t* Bt, const float* A_scale, const float* B_scale,
                      float* C, int M, int N, int K, float alpha, float beta, void* stream) {
    return launch_gemm8<OP_FP8, EPI_F32>(A, Bt, A_scale, B_scale, C, M, N, K, alpha, beta, stream,
                                         "gemm_fp8_e4m3");
}

}  // extern "C"
