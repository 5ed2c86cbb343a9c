// w4a16.hip -- W4A16 GEMM for gfx950: int4 weights (prepacked, see
// common.hpp), 16-bit or fp32 activations, fp32 accumulation.
//
// Reference: gemm_w4a16_groupwise (gemm_quant.hpp:47-57, gemm_quant.cpp:54-82)
// dequantizes a [G, N] fp32 panel per K-group and runs an fp32 axpy over it.
// Here nothing is dequantized to memory.  The decode/skinny kernel below
// (M <= 16 per row block) streams each 1 KiB weight tile once with 128-bit
// loads and feeds the MFMA the EXACT integers 16 + u as bf16 (one shift and
// one and-or per pair of nibbles).  Per K-segment of the group it forms
//     t  = sum_k x[m,k] * (16 + u[k,n])          (MFMA, fp32 accumulate)
//     xs = sum_k x[m,k]                           (MFMA against a ones operand)
// and adds s[g,n] * (t - (16 + z[g,n]) * xs) to the fp32 accumulator, which is
// sum_k x * (u - z) * s up to fp32 reassociation -- the reference's value.
// fp32 activations are split into bf16 hi + lo (two MFMAs), which keeps the
// product error near 2^-17 relative.  K is split across the waves of a
// workgroup and reduced through LDS in a fixed order (deterministic).
#include <cstdlib>

#include "common.hpp"

namespace lhq {
namespace {

constexpr uint32_t kOnesBf16x2 = 0x3F803F80u;  // bf16 pair (1.0, 1.0)

struct W4Args {
    const void* A;
    const uint8_t* qw;
    const void* scales;
    const uint32_t* zeros;
    void* C;
    int M, N, K, G, Nt, Kt, NG, NG8;
    float alpha, beta;
    // per-matrix strides for uniform batches (grid.z): elements of A / C,
    // bytes of qweight, elements of scales / zeros
    int64_t a_bs, c_bs, qw_bs, s_bs, z_bs;
    // ragged groups (device-resident table): rows [offsets[e], offsets[e+1])
    // use weights qws[e], scs[e], zss[e]; num_groups == 0 means not grouped
    const int32_t* offsets;
    const uint8_t* const* qws;
    const void* const* scs;
    const uint32_t* const* zss;
    int num_groups, row_capacity;
};

// Map blockIdx.y of a grouped launch to (group, first row, row end): groups
// take ceil(rows/16) row blocks each, in order.  Offsets are clamped to
// [0, row_capacity] so a malformed table can never index outside A or C.
__device__ __forceinline__ bool resolve_group(const W4Args& p, int y, int& e, int& m0, int& m_end) {
    for (e = 0; e < p.num_groups; ++e) {
        const int r0 = min(max(p.offsets[e], 0), p.row_capacity);
        const int r1 = min(max(p.offsets[e + 1], r0), p.row_capacity);
        const int nb = (r1 - r0 + 15) >> 4;
        if (y < nb) {
            m0 = r0 + 16 * y;
            m_end = r1;
            return true;
        }
        y -= nb;
    }
    return false;
}

// Eight activations (row `off / K`, k = off % K .. +7) as bf16 MFMA operands.
template <bool F32A>
__device__ __forceinline__ void load_a8(const void* A, int64_t off, bool ok, u32x4_t& hi,
                                        u32x4_t& lo) {
    if (!ok) {
        hi = u32x4_t{0, 0, 0, 0};
        lo = u32x4_t{0, 0, 0, 0};
        return;
    }
    if constexpr (F32A) {
        const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(A) + off);
        const float4 x0 = p[0], x1 = p[1];
        const float v[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint16_t h0 = f32_to_bf16(v[2 * i]), h1 = f32_to_bf16(v[2 * i + 1]);
            hi[i] = static_cast<uint32_t>(h0) | (static_cast<uint32_t>(h1) << 16);
            lo[i] = pack_bf16x2(v[2 * i] - bf16_to_f32(h0), v[2 * i + 1] - bf16_to_f32(h1));
        }
    } else {
        hi = *reinterpret_cast<const u32x4_t*>(static_cast<const uint16_t*>(A) + off);
        lo = u32x4_t{0, 0, 0, 0};
    }
}

// Decode / skinny W4A16.  grid = (ceil(Nt/T), ceil(M/16), batch); a
// workgroup of WAVES waves owns T column tiles and 16 rows; wave w walks its
// share of the K tiles.  BPS = 32-wide k blocks per scale segment
// (min(G,128)/32).
template <bool F32A, bool ASYM, bool F32C, int T, int WAVES, int BPS, bool GROUPED>
__global__ __launch_bounds__(64 * WAVES) void w4_gemv_kernel(W4Args p) {
    constexpr int SEGS = 4 / BPS;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int nt0 = blockIdx.x * T;
    int m0 = blockIdx.y * 16, m_end = p.M;
    const int z = blockIdx.z;
    const char* A = static_cast<const char*>(p.A) + z * p.a_bs * (F32A ? 4 : 2);
    const uint8_t* qw = p.qw + z * p.qw_bs;
    const void* scales = p.scales;
    const uint32_t* zeros = p.zeros;
    if constexpr (GROUPED) {
        int e;
        if (!resolve_group(p, blockIdx.y, e, m0, m_end)) return;  // uniform per workgroup
        qw = p.qws[e];
        scales = p.scs[e];
        zeros = p.zss[e];
    } else {
        scales = static_cast<const char*>(scales) + z * p.s_bs * (ASYM ? 2 : 4);
        if constexpr (ASYM) zeros += z * p.z_bs;
    }
    const int col = lane & 15;
    const int row = m0 + col;  // the A row this lane feeds (row operand index l & 15)
    const bool row_ok = row < m_end;
    const int per = (p.Kt + WAVES - 1) / WAVES;
    const int kb = wave * per;
    const int ke = min(p.Kt, kb + per);

    int ntc[T];
#pragma unroll
    for (int t = 0; t < T; ++t) ntc[t] = min(nt0 + t, p.Nt - 1);

    f32x4_t acc[T];
#pragma unroll
    for (int t = 0; t < T; ++t) acc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    const u32x4_t ones = {kOnesBf16x2, kOnesBf16x2, kOnesBf16x2, kOnesBf16x2};

    for (int kt = kb; kt < ke; ++kt) {
        u32x4_t w[T];
#pragma unroll
        for (int t = 0; t < T; ++t)
            w[t] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(
                qw + ((static_cast<int64_t>(ntc[t]) * p.Kt + kt) * 64 + lane) * 16));
        u32x4_t ah[4], al[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int k = kt * kW4TileK + 32 * j + 8 * (lane >> 4);
            load_a8<F32A>(A, static_cast<int64_t>(row) * p.K + k, row_ok && k < p.K, ah[j], al[j]);
        }
#pragma unroll
        for (int s = 0; s < SEGS; ++s) {
            f32x4_t xs = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int jj = 0; jj < BPS; ++jj) {
                const int j = s * BPS + jj;
                xs = mfma_bf16_16x16x32(ah[j], ones, xs);
                if constexpr (F32A) xs = mfma_bf16_16x16x32(al[j], ones, xs);
            }
            const int g = min((kt * kW4TileK + s * BPS * 32) / p.G, p.NG - 1);
#pragma unroll
            for (int t = 0; t < T; ++t) {
                f32x4_t acc_t = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int jj = 0; jj < BPS; ++jj) {
                    const int j = s * BPS + jj;
                    u32x4_t b;
#pragma unroll
                    for (int q = 0; q < 4; ++q) b[q] = w4_pair_16pu(w[t][j], q);
                    acc_t = mfma_bf16_16x16x32(ah[j], b, acc_t);
                    if constexpr (F32A) acc_t = mfma_bf16_16x16x32(al[j], b, acc_t);
                }
                const int64_t si = (static_cast<int64_t>(ntc[t]) * p.NG + g) * 16 + col;
                float sc, zc;
                if constexpr (ASYM) {
                    sc = f16_to_f32(static_cast<const uint16_t*>(scales)[si]);
                    const uint32_t zw = zeros[(static_cast<int64_t>(ntc[t]) * p.NG8 + (g >> 3)) * 16 + col];
                    zc = 16.0f + static_cast<float>((zw >> (4 * (g & 7))) & 15u);
                } else {
                    sc = static_cast<const float*>(scales)[si];
                    zc = 24.0f;  // 16 + implied zero point 8
                }
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    acc[t][i] = __builtin_fmaf(sc, __builtin_fmaf(-zc, xs[i], acc_t[i]), acc[t][i]);
            }
        }
    }

    auto store = [&](int t, int i, int ln, float v) {
        const int r = m0 + 4 * (ln >> 4) + i;
        const int c = (nt0 + t) * kW4TileN + (ln & 15);
        if (r >= m_end || c >= p.N || nt0 + t >= p.Nt) return;
        const int64_t o = z * p.c_bs + static_cast<int64_t>(r) * p.N + c;
        if constexpr (F32C) {
            float* Cp = static_cast<float*>(p.C);
            float out = p.alpha * v;
            if (p.beta != 0.0f) out = p.beta * Cp[o] + out;
            Cp[o] = out;
        } else {
            static_cast<uint16_t*>(p.C)[o] = f32_to_bf16(v);
        }
    };

    if constexpr (WAVES == 1) {
#pragma unroll
        for (int t = 0; t < T; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) store(t, i, lane, acc[t][i]);
    } else {
        __shared__ float red[WAVES][T][4][64];
#pragma unroll
        for (int t = 0; t < T; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) red[wave][t][i][lane] = acc[t][i];
        __syncthreads();
        for (int idx = threadIdx.x; idx < T * 4 * 64; idx += 64 * WAVES) {
            const int t = idx >> 8, i = (idx >> 6) & 3, ln = idx & 63;
            float sum = 0.0f;
#pragma unroll
            for (int w = 0; w < WAVES; ++w) sum += red[w][t][i][ln];
            store(t, i, ln, sum);
        }
    }
}

// Tuning knobs (read once): LHQ_W4_TILES (1|2) and LHQ_W4_WAVES (2|4|8)
// override the shape heuristic; unset = heuristic.
int env_int(const char* name) {
    const char* v = std::getenv(name);
    return v ? std::atoi(v) : 0;
}

template <bool F32A, bool ASYM, bool F32C, int T, int WAVES, bool GR>
void launch_bps(const W4Args& a, dim3 grid, int bps, hipStream_t s) {
    switch (bps) {
        case 1: w4_gemv_kernel<F32A, ASYM, F32C, T, WAVES, 1, GR><<<grid, 64 * WAVES, 0, s>>>(a); break;
        case 2: w4_gemv_kernel<F32A, ASYM, F32C, T, WAVES, 2, GR><<<grid, 64 * WAVES, 0, s>>>(a); break;
        default: w4_gemv_kernel<F32A, ASYM, F32C, T, WAVES, 4, GR><<<grid, 64 * WAVES, 0, s>>>(a); break;
    }
}

// mblocks: 16-row blocks along grid.y (for a grouped launch, an upper bound
// on the sum over groups of ceil(rows_e / 16)).
template <bool F32A, bool ASYM, bool F32C, bool GR = false>
int launch_w4_gemv(W4Args a, int batch, hipStream_t s, int mblocks = -1) {
    static const int env_t = env_int("LHQ_W4_TILES");
    static const int env_w = env_int("LHQ_W4_WAVES");
    if (mblocks < 0) mblocks = ceil_div(a.M, 16);
    int T = (a.Nt >= 1024) ? 2 : 1;
    if (env_t == 1 || env_t == 2) T = env_t;
    // Enough waves to cover 256 CUs several times over, but at least four
    // K tiles per wave so each wave keeps loads in flight.
    const int64_t wgs = static_cast<int64_t>(ceil_div(a.Nt, T)) * mblocks * batch;
    int W = 2;
    while (W < 8 && wgs * W < 4096 && a.Kt / (2 * W) >= 4) W *= 2;
    if (env_w == 2 || env_w == 4 || env_w == 8) W = env_w;
    const int bps = a.G >= 128 ? 4 : a.G / 32;
    dim3 grid(ceil_div(a.Nt, T), mblocks, batch);
    if (T == 1) {
        if (W == 2) launch_bps<F32A, ASYM, F32C, 1, 2, GR>(a, grid, bps, s);
        else if (W == 4) launch_bps<F32A, ASYM, F32C, 1, 4, GR>(a, grid, bps, s);
        else launch_bps<F32A, ASYM, F32C, 1, 8, GR>(a, grid, bps, s);
    } else {
        if (W == 2) launch_bps<F32A, ASYM, F32C, 2, 2, GR>(a, grid, bps, s);
        else if (W == 4) launch_bps<F32A, ASYM, F32C, 2, 4, GR>(a, grid, bps, s);
        else launch_bps<F32A, ASYM, F32C, 2, 8, GR>(a, grid, bps, s);
    }
    return check_launch("w4a16 gemv");
}

// The MFMA segment structure needs 32 | G, and each 128-wide tile must hold
// whole segments: G in {32, 64} or a multiple of 128.
int check_w4_shape(const char* who, int M, int N, int K, int G) {
    if (M < 0 || N <= 0 || K <= 0 || G <= 0 || K % G != 0)
        return set_error(LHQ_ERR_INVALID, "%s: bad dims M=%d N=%d K=%d G=%d (need G | K)", who, M, N, K, G);
    if (!(G == 32 || G == 64 || G % 128 == 0))
        return set_error(LHQ_ERR_UNSUPPORTED, "%s: group_size %d unsupported (32, 64 or a multiple of 128)", who, G);
    return LHQ_OK;
}

W4Args make_args(const void* A, const uint8_t* qw, const void* sc, const uint32_t* zs, void* C,
                 int M, int N, int K, int G, float alpha, float beta) {
    W4Args a{};
    a.A = A; a.qw = qw; a.scales = sc; a.zeros = zs; a.C = C;
    a.M = M; a.N = N; a.K = K; a.G = G;
    a.Nt = ceil_div(N, kW4TileN); a.Kt = ceil_div(K, kW4TileK);
    a.NG = K / G; a.NG8 = ceil_div(a.NG, 8);
    a.alpha = alpha; a.beta = beta;
    return a;
}

}  // namespace
}  // namespace lhq

using namespace lhq;

extern "C" {

int lhq_gemm_w4a16(const float* A, const uint8_t* qweight, const float* scales, float* C, int M,
                   int N, int K, int G, float alpha, float beta, void* stream) {
    if (int st = check_w4_shape("gemm_w4a16", M, N, K, G)) return st;
    LHQ_REQUIRE(qweight && scales && C && (A || M == 0), "gemm_w4a16: null pointer");
    if (M == 0) return LHQ_OK;
    W4Args a = make_args(A, qweight, scales, nullptr, C, M, N, K, G, alpha, beta);
    return launch_w4_gemv<true, false, true>(a, 1, as_stream(stream));
}

int lhq_gemm_w4a16_bf16(const uint16_t* A, const uint8_t* qweight, const uint16_t* scales,
                        const uint32_t* zeros, uint16_t* C, int M, int N, int K, int G,
                        void* stream) {
    if (int st = check_w4_shape("gemm_w4a16_bf16", M, N, K, G)) return st;
    LHQ_REQUIRE(qweight && scales && zeros && C && (A || M == 0), "gemm_w4a16_bf16: null pointer");
    if (M == 0) return LHQ_OK;
    W4Args a = make_args(A, qweight, scales, zeros, C, M, N, K, G, 1.0f, 0.0f);
    return launch_w4_gemv<false, true, false>(a, 1, as_stream(stream));
}

int lhq_gemm_w4a16_bf16_batched(const uint16_t* A, const uint8_t* qweight, const uint16_t* scales,
                                const uint32_t* zeros, uint16_t* C, int batch, int M, int N, int K,
                                int G, void* stream) {
    if (int st = check_w4_shape("gemm_w4a16_bf16_batched", M, N, K, G)) return st;
    LHQ_REQUIRE(batch >= 0 && batch <= 65535, "gemm_w4a16_bf16_batched: batch %d out of range", batch);
    LHQ_REQUIRE(qweight && scales && zeros && C && (A || M == 0), "gemm_w4a16_bf16_batched: null pointer");
    if (M == 0 || batch == 0) return LHQ_OK;
    W4Args a = make_args(A, qweight, scales, zeros, C, M, N, K, G, 1.0f, 0.0f);
    a.a_bs = static_cast<int64_t>(M) * K;
    a.c_bs = static_cast<int64_t>(M) * N;
    a.qw_bs = lhq_w4_qweight_bytes(K, N);
    a.s_bs = static_cast<int64_t>(a.Nt) * a.NG * 16;
    a.z_bs = static_cast<int64_t>(a.Nt) * a.NG8 * 16;
    return launch_w4_gemv<false, true, false>(a, batch, as_stream(stream));
}

int lhq_gemm_w4a16_bf16_grouped(const uint16_t* A, const int32_t* offsets, const uint8_t* const* qweights,
                                const uint16_t* const* scales, const uint32_t* const* zeros, uint16_t* C,
                                int num_groups, int row_capacity, int N, int K, int G, void* stream) {
    if (int st = check_w4_shape("gemm_w4a16_bf16_grouped", row_capacity, N, K, G)) return st;
    LHQ_REQUIRE(num_groups >= 0, "gemm_w4a16_bf16_grouped: negative num_groups");
    LHQ_REQUIRE(offsets && qweights && scales && zeros && C && (A || row_capacity == 0),
                "gemm_w4a16_bf16_grouped: null pointer");
    if (num_groups == 0 || row_capacity == 0) return LHQ_OK;
    W4Args a = make_args(A, nullptr, nullptr, nullptr, C, row_capacity, N, K, G, 1.0f, 0.0f);
    a.offsets = offsets;
    a.qws = qweights;
    a.scs = reinterpret_cast<const void* const*>(scales);
    a.zss = zeros;
    a.num_groups = num_groups;
    a.row_capacity = row_capacity;
    // sum_e ceil(rows_e / 16) <= ceil(row_capacity / 16) + num_groups
    const int64_t mblocks = ceil_div64(row_capacity, 16) + num_groups;
    LHQ_SUPPORTED(mblocks <= 65535, "gemm_w4a16_bf16_grouped: %lld row blocks exceed the grid limit",
                  static_cast<long long>(mblocks));
    return launch_w4_gemv<false, true, false, true>(a, 1, as_stream(stream), static_cast<int>(mblocks));
}

}  // extern "C"
