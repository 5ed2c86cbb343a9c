// w4a16.hip -- W4A16 GEMM for gfx950: int4 weights (prepacked, see
// common.hpp), 16-bit or fp32 activations, fp32 accumulation.
//
// Reference: gemm_w4a16_groupwise (gemm_quant.hpp:47-57, gemm_quant.cpp:54-82)
// dequantizes a [G, N] fp32 panel per K-group and runs an fp32 axpy over it.
// Here nothing is dequantized to memory.  Each 1 KiB weight tile is streamed
// once with 128-bit loads and fed to the MFMA as the EXACT integers 128 + u
// (bf16; w4_operand).  Per K-segment of a group the kernels form
//     t  = sum_k x[m,k] * (128 + u[k,n])          (MFMA, fp32 accumulate)
//     xs = sum_k x[m,k]                            (MFMA against a ones operand)
// and add s[g,n] * (t - (128 + z[g,n]) * xs) to an fp32 accumulator: that is
// sum_k x * (u - z) * s up to fp32 reassociation, the reference's value.
// fp32 activations are split into bf16 hi + lo (two MFMAs), which keeps the
// product error near 2^-17 relative.
//
// Three kernels share that arithmetic:
//   w4_decode_kernel -- M <= 16 with the activations small enough to stage in
//     LDS: a streaming GEMV whose only global loads in the main loop are the
//     weight tiles and their scales / zero points.
//   w4_gemv_kernel   -- any M in 16-row blocks, uniform batches and ragged
//     grouped launches (device-side group table).
//   w4_mma_kernel    -- bf16 prefill tiles (many rows per weight tile).
// w4_decode_i8_kernel (M = 1) computes the same sums on the int8 MFMA, with
// the activations as exact fixed-point digit planes (see its comment).
// The GEMV kernels split K over the waves of a workgroup and reduce through
// LDS in wave order, so results are deterministic.
#include <algorithm>
#include <cstdlib>
#include <mutex>
#include <type_traits>

#include "common.hpp"

namespace lhq {
namespace {

constexpr uint32_t kOnesBf16x2 = 0x3F803F80u;  // bf16 pair (1.0, 1.0)
constexpr uint32_t kM144Bf16x2 = 0xC310C310u;  // bf16 pair (-144.0, -144.0), exact

struct W4Args {
    const void* A;
    const uint8_t* qw;
    const void* scales;
    const uint32_t* zeros;
    void* C;
    int M, N, K, G, Nt, Kt, NG, NG8;
    // group of tile kt when G > 128: __umulhi(kt, gmul), gmul = ceil(2^32 / (G/128))
    // (exact for kt, G/128 < 2^16); 0 when G <= 128
    uint32_t gmul;
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
    int group_rb;  // rows per row block of a grouped decode launch
    // split-K tile launches (grid.z = split): split s covers K tiles
    // [s * kps, (s + 1) * kps) and writes fp32 partial sums ws[s][M][N]
    float* ws;
    int kps;
    // persistent grouped launches: the workspace's 64 KiB partial-sum slots
    // (at ws) and the launch's worker count
    int64_t pk_slots;
    int pk_workers;
};

// Scale group of segment s of K tile kt; a segment is BPS 32-wide k blocks
// (min(G,128) k values), so G <= 128 needs no division at all.
template <int BPS>
__device__ __forceinline__ int group_of(int kt, int s, uint32_t gmul) {
    if constexpr (BPS < 4) return kt * (4 / BPS) + s;
    else return gmul ? static_cast<int>(__umulhi(static_cast<uint32_t>(kt), gmul)) : kt;
}
// The same with G > 128 known at compile time (GBIG) or known false.
template <int BPS, bool GBIG>
__device__ __forceinline__ int group_of_c(int kt, int s, uint32_t gmul) {
    if constexpr (BPS < 4) return kt * (4 / BPS) + s;
    else if constexpr (GBIG) return static_cast<int>(__umulhi(static_cast<uint32_t>(kt), gmul));
    else return kt;
}

// The group of a segment as read from the scale / zero arrays: with G < 128
// and K % 128 != 0 the last K tile has segments past K (their activations
// are zero), and their scale and zero point are read from the last group so
// every load stays inside the arrays.
template <int BPS, bool GBIG>
__device__ __forceinline__ int seg_group(int kt, int s, const W4Args& p) {
    const int g = group_of_c<BPS, GBIG>(kt, s, p.gmul);
    if constexpr (BPS < 4) return min(g, p.NG - 1);
    else return g;
}

// Map blockIdx.y of a grouped launch to (group, first row, row end): groups
// take ceil(rows/RB) row blocks each, in order.  Offsets are clamped to
// [0, row_capacity] so a malformed table can never index outside A or C.
// The wave resolves 64 groups per step: lane i takes group e0 + i, a prefix
// sum over the lanes gives each group's first block, and a ballot finds the
// group holding block y (4 steps for 256 experts, where a serial walk of the
// table by every workgroup cost milliseconds per layer).  The results are
// the same in every lane and wave (y is uniform): the return is uniform per
// workgroup.  rb: rows per block (a compile-time constant through
// resolve_group<RB>; a run-time one for the grouped decode kernel).
__device__ __forceinline__ bool resolve_group_rows(const W4Args& p, int y, int rb, int& e, int& m0, int& m_end) {
    const int lane = threadIdx.x & 63;
    int base = 0;  // row blocks of the groups before this step's
    for (int e0 = 0; e0 < p.num_groups; e0 += 64) {
        const int g = e0 + lane;
        int r0 = 0, r1 = 0;
        if (g < p.num_groups) {
            r0 = min(max(p.offsets[g], 0), p.row_capacity);
            r1 = min(max(p.offsets[g + 1], r0), p.row_capacity);
        }
        const int nb = (r1 - r0 + rb - 1) / rb;
        int incl = nb;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const int v = __shfl_up(incl, d, 64);
            if (lane >= d) incl += v;
        }
        const int excl = incl - nb;
        const uint64_t hit = __ballot(y >= base + excl && y < base + incl);
        if (hit) {
            const int src = __builtin_ctzll(hit);
            e = __builtin_amdgcn_readfirstlane(e0 + src);
            m0 = __builtin_amdgcn_readfirstlane(__shfl(r0, src, 64) + rb * (y - base - __shfl(excl, src, 64)));
            m_end = __builtin_amdgcn_readfirstlane(__shfl(r1, src, 64));
            return true;
        }
        base += __shfl(incl, 63, 64);
    }
    return false;
}
template <int RB = 16>
__device__ __forceinline__ bool resolve_group(const W4Args& p, int y, int& e, int& m0, int& m_end) {
    return resolve_group_rows(p, y, RB, e, m0, m_end);
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

// Output element (row r, column c) of a W4 GEMM: fp32 with the reference's
// alpha / beta (beta == 0 never reads C, gemm_quant.cpp:12-21) or bf16 RNE.
template <bool F32C>
__device__ __forceinline__ void w4_store(const W4Args& p, int64_t o, float v) {
    if constexpr (F32C) {
        float* Cp = static_cast<float*>(p.C);
        float out = p.alpha * v;
        if (p.beta != 0.0f) out = p.beta * Cp[o] + out;
        Cp[o] = out;
    } else {
        static_cast<uint16_t*>(p.C)[o] = f32_to_bf16(v);
    }
}

// SwiGLU of one (gate, up) pair, moe.cpp:144-146 and :191: silu(g) * u with
// silu(v) = v / (1 + exp(-v)), fp32, IEEE division.
__device__ __forceinline__ float swiglu(float g, float u) { return g / (1.0f + expf(-g)) * u; }

// SwiGLU epilogue (SWI): the weights interleave the gate and up projections
// by column tile (lhq_w4_interleave_gate_up): tile 2j holds gate columns
// 16j .. 16j+15 and tile 2j+1 the same up columns, so the accumulators of
// one gate column and its up column sit in the same lane of two adjacent
// tiles.  The kernel then writes act[r][16j + c] = bf16(swiglu(g, u)) with
// p.N = the intermediate width (act's row length) and p.Nt = 2 ceil(N/16).

// ---------------------------------------------------------------------------
// Generic kernel.  grid = (ceil(Nt/T), row blocks, batch); a workgroup of
// WAVES waves owns T column tiles and 16 rows; wave w walks its share of the
// K tiles.  BPS = 32-wide k blocks per scale segment (min(G,128)/32).
// ---------------------------------------------------------------------------
// PIPE (bf16 activations, plain launches of one or two column tiles per
// workgroup): the K loop keeps the next tile's loads in flight while the
// current tile is consumed; its extra registers cost occupancy, which the
// many-workgroup grouped and wide launches need more.
template <bool F32A, bool ASYM, bool F32C, int T, int WAVES, int BPS, bool GROUPED, bool SWI = false, bool PIPE = false>
__global__ __launch_bounds__(64 * WAVES) void w4_gemv_kernel(W4Args p) {
    static_assert(!SWI || ((T == 2 || T == 4 || T == 8) && !F32C), "SwiGLU pairs the column tiles of a workgroup");
    static_assert(!PIPE || (!F32A && !GROUPED && !SWI && T <= 2), "pipelined K loop: plain bf16 launches of 1-2 tiles");
    constexpr int SEGS = 4 / BPS;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
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

    if constexpr (PIPE) {
        // The K tiles run in passes of P tiles whose loads (weights,
        // activations, scales, zero words) are all issued before any is
        // used, and the next pass's loads are in flight while the current
        // pass is consumed, so a wave waits for memory once per pass instead
        // of once per tile.  Every load is unconditional: tiles past this
        // wave's range re-read its last tile (never consumed), rows past the
        // block's end read its last row (their outputs are not stored; an
        // output row depends on its own activation row only), and k past K
        // reads the row's last 8 elements, zeroed at use.  One tile per pass
        // measured faster than two (M=8, K=N=8192: 10.6 against 11.1 us),
        // which hold more registers.
        constexpr int P = 1;
        constexpr int NZ = ASYM ? 1 : 0;
        struct Pass {
            u32x4_t w[P][T];
            u32x4_t a[P][4];
            uint32_t sr[P][T][SEGS];
            uint32_t zw[P][T][NZ > 0 ? SEGS : 1];
        };
        const int64_t arow = static_cast<int64_t>(min(row, m_end - 1)) * p.K;
        auto issue = [&](Pass& Q, int kt0) {
#pragma unroll
            for (int i = 0; i < P; ++i) {
                const int kt = min(kt0 + i, ke - 1);
#pragma unroll
                for (int t = 0; t < T; ++t)
                    Q.w[i][t] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(
                        qw + ((static_cast<int64_t>(ntc[t]) * p.Kt + kt) * 64 + lane) * 16));
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int k = min(kt * kW4TileK + 32 * j + 8 * (lane >> 4), p.K - 8);
                    Q.a[i][j] = *reinterpret_cast<const u32x4_t*>(static_cast<const uint16_t*>(static_cast<const void*>(A)) +
                                                                  (arow + k));
                }
#pragma unroll
                for (int s2 = 0; s2 < SEGS; ++s2) {
                    const int g = (BPS < 4) ? min(group_of<BPS>(kt, s2, p.gmul), p.NG - 1) : group_of<BPS>(kt, s2, p.gmul);
#pragma unroll
                    for (int t = 0; t < T; ++t) {
                        const int64_t si = (static_cast<int64_t>(ntc[t]) * p.NG + g) * 16 + col;
                        if constexpr (ASYM) {
                            Q.sr[i][t][s2] = static_cast<const uint16_t*>(scales)[si];
                            Q.zw[i][t][s2] = zeros[(static_cast<int64_t>(ntc[t]) * p.NG8 + (g >> 3)) * 16 + col];
                        } else {
                            Q.sr[i][t][s2] = static_cast<const uint32_t*>(scales)[si];
                        }
                    }
                }
            }
        };
        // tile i of pass Q, K tile kt
        auto consume1 = [&](const Pass& Q, int i, int kt) {
            u32x4_t ah[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) ah[j] = Q.a[i][j];
            if (kt == p.Kt - 1 && (p.K & (kW4TileK - 1))) {
                // the zero padding of the last K tile (uniform branch)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    if (kt * kW4TileK + 32 * j + 8 * (lane >> 4) >= p.K) ah[j] = u32x4_t{0, 0, 0, 0};
            }
#pragma unroll
            for (int s2 = 0; s2 < SEGS; ++s2) {
                f32x4_t xs = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int jj = 0; jj < BPS; ++jj) xs = mfma_bf16_16x16x32(ah[s2 * BPS + jj], ones, xs);
                const int g = (BPS < 4) ? min(group_of<BPS>(kt, s2, p.gmul), p.NG - 1) : group_of<BPS>(kt, s2, p.gmul);
#pragma unroll
                for (int t = 0; t < T; ++t) {
                    f32x4_t acc_t = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int jj = 0; jj < BPS; ++jj) {
                        const int j = s2 * BPS + jj;
                        acc_t = mfma_bf16_16x16x32(ah[j], w4_operand(Q.w[i][t][j]), acc_t);
                    }
                    float sc, zc;
                    if constexpr (ASYM) {
                        sc = f16_to_f32(static_cast<uint16_t>(Q.sr[i][t][s2]));
                        zc = kW4Bias + static_cast<float>((Q.zw[i][t][s2] >> (4 * (g & 7))) & 15u);
                    } else {
                        sc = __uint_as_float(Q.sr[i][t][s2]);
                        zc = kW4Bias + 8.0f;  // implied zero point 8
                    }
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        acc[t][r] = __builtin_fmaf(sc, __builtin_fmaf(-zc, xs[r], acc_t[r]), acc[t][r]);
                }
            }
        };
        auto consume = [&](const Pass& Q, int kt0) {
#pragma unroll
            for (int i = 0; i < P; ++i)
                if (kt0 + i < ke) consume1(Q, i, kt0 + i);
        };
        if (kb < ke) {
            Pass pa, pb;
            issue(pa, kb);
            int k0 = kb;
            for (; k0 + 2 * P < ke; k0 += 2 * P) {
                issue(pb, k0 + P);
                consume(pa, k0);
                issue(pa, k0 + 2 * P);
                consume(pb, k0 + P);
            }
            if (k0 + P < ke) {
                issue(pb, k0 + P);
                consume(pa, k0);
                consume(pb, k0 + P);
            } else {
                consume(pa, k0);
            }
        }
    } else {
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
                const int g = (BPS < 4) ? min(group_of<BPS>(kt, s, p.gmul), p.NG - 1) : group_of<BPS>(kt, s, p.gmul);
#pragma unroll
                for (int t = 0; t < T; ++t) {
                    f32x4_t acc_t = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int jj = 0; jj < BPS; ++jj) {
                        const int j = s * BPS + jj;
                        const u32x4_t b = w4_operand(w[t][j]);
                        acc_t = mfma_bf16_16x16x32(ah[j], b, acc_t);
                        if constexpr (F32A) acc_t = mfma_bf16_16x16x32(al[j], b, acc_t);
                    }
                    const int64_t si = (static_cast<int64_t>(ntc[t]) * p.NG + g) * 16 + col;
                    float sc, zc;
                    if constexpr (ASYM) {
                        sc = f16_to_f32(static_cast<const uint16_t*>(scales)[si]);
                        const uint32_t zw = zeros[(static_cast<int64_t>(ntc[t]) * p.NG8 + (g >> 3)) * 16 + col];
                        zc = kW4Bias + static_cast<float>((zw >> (4 * (g & 7))) & 15u);
                    } else {
                        sc = static_cast<const float*>(scales)[si];
                        zc = kW4Bias + 8.0f;  // implied zero point 8
                    }
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        acc[t][i] = __builtin_fmaf(sc, __builtin_fmaf(-zc, xs[i], acc_t[i]), acc[t][i]);
                }
            }
        }
    }

    auto store = [&](int t, int i, int ln, float v) {
        const int r = m0 + 4 * (ln >> 4) + i;
        const int c = (nt0 + t) * kW4TileN + (ln & 15);
        if (r >= m_end || c >= p.N || nt0 + t >= p.Nt) return;
        w4_store<F32C>(p, z * p.c_bs + static_cast<int64_t>(r) * p.N + c, v);
    };
    // SWI: tiles nt0 + 2h (gate) and nt0 + 2h + 1 (up) -> act column tile
    // nt0 / 2 + h
    auto store_act = [&](int h, int i, int ln, float g, float u) {
        const int r = m0 + 4 * (ln >> 4) + i;
        const int c = (nt0 / 2 + h) * kW4TileN + (ln & 15);
        if (r >= m_end || c >= p.N) return;
        static_cast<uint16_t*>(p.C)[z * p.c_bs + static_cast<int64_t>(r) * p.N + c] = f32_to_bf16(swiglu(g, u));
    };

    if constexpr (SWI && WAVES == 1) {
#pragma unroll
        for (int h = 0; h < T / 2; ++h)
#pragma unroll
            for (int i = 0; i < 4; ++i) store_act(h, i, lane, acc[2 * h][i], acc[2 * h + 1][i]);
    } else if constexpr (SWI) {
        __shared__ float red[WAVES][T][4][64];
#pragma unroll
        for (int t = 0; t < T; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) red[wave][t][i][lane] = acc[t][i];
        __syncthreads();
        for (int idx = threadIdx.x; idx < (T / 2) * 4 * 64; idx += 64 * WAVES) {
            const int h = idx >> 8, i = (idx >> 6) & 3, ln = idx & 63;
            float g = 0.0f, u = 0.0f;
#pragma unroll
            for (int w = 0; w < WAVES; ++w) {
                g += red[w][2 * h][i][ln];
                u += red[w][2 * h + 1][i][ln];
            }
            store_act(h, i, ln, g, u);
        }
    } else if constexpr (WAVES == 1) {
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

// ---------------------------------------------------------------------------
// Decode kernel (M <= 16 rows, one 16-row block).  The workgroup stages its
// activation rows [min(M,16), Kp] in LDS once (fp32 activations as bf16
// hi / lo planes), so the main loop's only global loads are weight tiles and
// their scales / zero points.  Vector-memory loads complete in order: an
// activation fetch queued behind weight tiles would wait for all of them.
//
// Each wave owns NPW consecutive K tiles of T column tiles per pass; a pass
// issues all of its loads first and then consumes them in issue order, so
// the wave waits for the memory system once per pass and nothing loaded is
// carried across a loop edge.  Overlap comes from the many resident waves.
// grid = (ceil(Nt/T), 1, batch), blockDim = 64*S: the S waves cover S*NPW
// consecutive tiles per pass (passes repeat until Kt is covered) and are
// reduced through LDS in wave order (deterministic).
// ---------------------------------------------------------------------------

// Every load a wave issues is unconditional (out-of-range addresses are
// clamped to valid ones, the values discarded): the compiler counts
// outstanding loads per path, and a load that only some paths issue would
// turn each later wait into a wait for everything.
// MR: accumulator rows per lane that can hold an output row.  Lane l holds
// rows 4*(l >> 4) + r, r < 4; with M == 1 only row 0 (r = 0 of lanes 0..15)
// is real, so MR = 1 skips the per-group correction of the other three.
// Launch bounds: one-column-tile bf16-activation variants are held to four
// waves per SIMD (<= 128 VGPRs; they need ~90).  Two-column-tile variants
// need ~136 and would spill inside the loop under that bound.
// GR: ragged groups (bf16 activations and output, fp16 scales): grid.y
// walks row blocks of p.group_rb rows over the groups (resolve_group_rows),
// each staged whole; SWI adds the SwiGLU epilogue on the two column tiles
// of a workgroup (gate 2j, up 2j + 1).
template <bool F32A, bool ASYM, bool F32C, int T, int NPW, int BPS, bool GBIG, int MR, bool GR = false,
          bool SWI = false>
__global__ __launch_bounds__(T == 1 ? 1024 : 512, (F32A || T == 2) ? 1 : 4) void w4_decode_kernel(W4Args p) {
    static_assert(NPW == 4 || NPW == 8, "passes start at multiples of NPW tiles");
    static_assert(MR == 1 || MR == 4, "one row or all four");
    static_assert(!GR || (!F32A && ASYM && !F32C && MR == 4), "grouped: bf16 in and out, fp16 scales");
    static_assert(!SWI || (GR && T == 2), "SwiGLU pairs the two column tiles of a workgroup");
    constexpr int SEGS = 4 / BPS;
    // zero words (8 groups each) per pass: G < 128 -> the pass's words
    // (passes start at multiples of 8 tiles); G == 128 -> one shared word;
    // G > 128 -> one per tile
    constexpr int NZW = (BPS < 4) ? (NPW * SEGS + 7) / 8 : (GBIG ? NPW : 1);
    // [F32A ? 2 : 1 planes][Ml rows][Kp], bf16 (fp32 activations: hi, lo);
    // after the main loop the same memory holds the cross-wave reduction
    // (the launcher sizes it for both), so a workgroup takes no more LDS
    // than its activations and more workgroups fit on a CU
    extern __shared__ __attribute__((aligned(16))) uint16_t a_lds[];

    const int S = blockDim.x >> 6;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int z = blockIdx.z;
    const uint8_t* qw = p.qw + z * p.qw_bs;
    const char* scales = static_cast<const char*>(p.scales) + z * p.s_bs * (ASYM ? 2 : 4);
    const uint32_t* zeros = ASYM ? p.zeros + z * p.z_bs : nullptr;
    int m0 = 0, Ml = min(p.M, 16);  // first row and row count of this workgroup
    if constexpr (GR) {
        int e, m_end;
        if (!resolve_group_rows(p, blockIdx.y, p.group_rb, e, m0, m_end)) return;  // uniform per workgroup
        qw = p.qws[e];
        scales = static_cast<const char*>(p.scs[e]);
        zeros = p.zss[e];
        Ml = min(m_end - m0, p.group_rb);
    }
    const int col = lane & 15;
    const int Kp = p.Kt * kW4TileK;

    // Column tiles past Nt (odd Nt with T = 2) alias the last one; their
    // outputs are never stored.  Bases are wave-uniform; the per-lane parts
    // of every address below are 32-bit offsets.
    const uint8_t* qwb[T];
    const char* scb[T];
    const char* zwb[T];
#pragma unroll
    for (int t = 0; t < T; ++t) {
        const int64_t nt = min(static_cast<int>(blockIdx.x) * T + t, p.Nt - 1);
        qwb[t] = qw + nt * p.Kt * kW4TileBytes;
        scb[t] = scales + nt * p.NG * 16 * (ASYM ? 2 : 4);
        zwb[t] = ASYM ? reinterpret_cast<const char*>(zeros + nt * p.NG8 * 16) : nullptr;
    }
    // fp16 scales are fetched as the aligned dword holding columns
    // (col & ~1, col | 1); the lane's half is selected at use
    const uint32_t s_half = ASYM ? 16u * (col & 1) : 0u;
    const uint32_t s_col = ASYM ? static_cast<uint32_t>((col & ~1) * 2) : static_cast<uint32_t>(col * 4);

    // one pass worth of loaded operands; two of them alternate so the next
    // pass's loads are in flight while the current pass is consumed
    struct Pass {
        u32x4_t w[NPW][T];
        uint32_t sw[NPW][T][SEGS];
        uint32_t zw[NZW][T];
    };
    // All loads of the pass starting at tile kt0, in consumption order (zero
    // words first: the first tile needs them); tiles past Kt re-read the
    // last tile (the same lines, never consumed).
    auto issue = [&](Pass& P, int kt0) {
        if constexpr (ASYM) {
#pragma unroll
            for (int q = 0; q < NZW; ++q) {
                const int g = (BPS < 4) ? group_of_c<BPS, GBIG>(min(kt0, p.Kt - 1), 0, 0) + 8 * q
                                        : group_of_c<BPS, GBIG>(min(kt0 + q, p.Kt - 1), 0, p.gmul);
                const uint32_t off = static_cast<uint32_t>((min(g >> 3, p.NG8 - 1) * 16 + col) * 4);
#pragma unroll
                for (int t = 0; t < T; ++t) P.zw[q][t] = *reinterpret_cast<const uint32_t*>(zwb[t] + off);
            }
        }
#pragma unroll
        for (int i = 0; i < NPW; ++i) {
            const int kt = min(kt0 + i, p.Kt - 1);
#pragma unroll
            for (int t = 0; t < T; ++t) {
#pragma unroll
                for (int s = 0; s < SEGS; ++s) {
                    const uint32_t off = static_cast<uint32_t>(seg_group<BPS, GBIG>(kt, s, p) * 16 * (ASYM ? 2 : 4)) + s_col;
                    P.sw[i][t][s] = *reinterpret_cast<const uint32_t*>(scb[t] + off);
                }
                P.w[i][t] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(
                    qwb[t] + static_cast<uint32_t>(kt * kW4TileBytes + lane * 16)));
            }
        }
    };

    // 1. activation loads first, then the first pass's weights: the wait
    //    for the activations then covers nothing behind them
    const int span = S * NPW;  // tiles per pass over the workgroup
    const int rc = Kp >> 3;    // 8-element chunks per padded row
    const int chunks = Ml * rc;
    const char* A = static_cast<const char*>(p.A) + (z * p.a_bs + static_cast<int64_t>(m0) * p.K) * (F32A ? 4 : 2);
    constexpr int B = 4;  // chunks per thread per staging batch
    u32x4_t av[B], av2[B];
    auto stage_load = [&](int c0) {
#pragma unroll
        for (int b = 0; b < B; ++b) {
            const int c = c0 + b * 64 * S;
            const int r = c / rc, k = (c - r * rc) * 8;
            const bool ok = c < chunks && k < p.K;
            const int64_t e = ok ? static_cast<int64_t>(r) * p.K + k : 0;  // element 0 always exists
            if constexpr (F32A) {
                av[b] = *reinterpret_cast<const u32x4_t*>(A + e * 4);
                av2[b] = *reinterpret_cast<const u32x4_t*>(A + e * 4 + 16);
            } else {
                av[b] = *reinterpret_cast<const u32x4_t*>(A + e * 2);
            }
        }
    };
    auto stage_store = [&](int c0) {
#pragma unroll
        for (int b = 0; b < B; ++b) {
            const int c = c0 + b * 64 * S;
            const int r = c / rc, k = (c - r * rc) * 8;
            const bool ok = c < chunks && k < p.K;
            if (c < chunks) {
                const u32x4_t zero = {0, 0, 0, 0};
                if constexpr (F32A) {
                    const u32x4_t x0 = ok ? av[b] : zero, x1 = ok ? av2[b] : zero;
                    const float f[8] = {__uint_as_float(x0[0]), __uint_as_float(x0[1]),
                                        __uint_as_float(x0[2]), __uint_as_float(x0[3]),
                                        __uint_as_float(x1[0]), __uint_as_float(x1[1]),
                                        __uint_as_float(x1[2]), __uint_as_float(x1[3])};
                    u32x4_t hi, lo;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const uint16_t h0 = f32_to_bf16(f[2 * i]), h1 = f32_to_bf16(f[2 * i + 1]);
                        hi[i] = static_cast<uint32_t>(h0) | (static_cast<uint32_t>(h1) << 16);
                        lo[i] = pack_bf16x2(f[2 * i] - bf16_to_f32(h0), f[2 * i + 1] - bf16_to_f32(h1));
                    }
                    *reinterpret_cast<u32x4_t*>(a_lds + static_cast<uint32_t>(c) * 8) = hi;
                    *reinterpret_cast<u32x4_t*>(a_lds + static_cast<uint32_t>(Ml * Kp + c * 8)) = lo;
                } else {
                    *reinterpret_cast<u32x4_t*>(a_lds + static_cast<uint32_t>(c) * 8) = ok ? av[b] : zero;
                }
            }
        }
    };
    const int kb0 = wave * NPW;
    stage_load(threadIdx.x);
    Pass pa, pb;
    issue(pa, kb0);
    stage_store(threadIdx.x);
    // activations beyond the first batch (large M*K): staged after the
    // first pass's loads are out
    for (int c0 = threadIdx.x + B * 64 * S; c0 < chunks; c0 += B * 64 * S) {
        stage_load(c0);
        stage_store(c0);
    }
    __syncthreads();

    // rows >= M read row M-1 (their outputs are discarded), so every LDS
    // read stays inside the staged rows
    const uint16_t* arow = a_lds + static_cast<uint32_t>(min(col, Ml - 1) * Kp + 8 * (lane >> 4));
    const u32x4_t ones = {kOnesBf16x2, kOnesBf16x2, kOnesBf16x2, kOnesBf16x2};
    f32x4_t acc[T];
#pragma unroll
    for (int t = 0; t < T; ++t) acc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    auto tile = [&](const Pass& P, int i, int kt) {
        u32x4_t ah[4], al[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            ah[j] = *reinterpret_cast<const u32x4_t*>(arow + kt * kW4TileK + 32 * j);
            if constexpr (F32A)
                al[j] = *reinterpret_cast<const u32x4_t*>(arow + Ml * Kp + kt * kW4TileK + 32 * j);
        }
#pragma unroll
        for (int s = 0; s < SEGS; ++s) {
            f32x4_t xs = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int jj = 0; jj < BPS; ++jj) {
                xs = mfma_bf16_16x16x32(ah[s * BPS + jj], ones, xs);
                if constexpr (F32A) xs = mfma_bf16_16x16x32(al[s * BPS + jj], ones, xs);
            }
            const int g = seg_group<BPS, GBIG>(kt, s, p);
#pragma unroll
            for (int t = 0; t < T; ++t) {
                f32x4_t tt = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int jj = 0; jj < BPS; ++jj) {
                    const int j = s * BPS + jj;
                    const u32x4_t b = w4_operand(P.w[i][t][j]);
                    tt = mfma_bf16_16x16x32(ah[j], b, tt);
                    if constexpr (F32A) tt = mfma_bf16_16x16x32(al[j], b, tt);
                }
                float sc, zc;
                if constexpr (ASYM) {
                    sc = f16_to_f32(static_cast<uint16_t>(P.sw[i][t][s] >> s_half));
                    const uint32_t word = P.zw[(BPS < 4) ? (i * SEGS + s) / 8 : (GBIG ? i : 0)][t];
                    zc = kW4Bias + static_cast<float>((word >> (4 * (g & 7))) & 15u);
                } else {
                    sc = __uint_as_float(P.sw[i][t][s]);
                    zc = kW4Bias + 8.0f;  // implied zero point 8
                }
#pragma unroll
                for (int r = 0; r < MR; ++r)
                    acc[t][r] = __builtin_fmaf(sc, __builtin_fmaf(-zc, xs[r], tt[r]), acc[t][r]);
            }
        }
    };
    // a full pass runs its tiles without a branch between them, so the
    // compiler can overlap one tile's MFMA latency with the next tile's decode
    auto consume = [&](const Pass& P, int kb) {
        const int n = min(NPW, p.Kt - kb);
        if (n == NPW) {
#pragma unroll
            for (int i = 0; i < NPW; ++i) tile(P, i, kb + i);
        } else {
#pragma unroll
            for (int i = 0; i < NPW; ++i)
                if (i < n) tile(P, i, kb + i);
        }
    };
    // passes of this wave: kb0 + q*span for q < np.  Pairs of passes run
    // with the loads of the next pass issued before the current one is
    // consumed; every issue is unconditional within its block, so each wait
    // the compiler places covers exactly the pass being consumed.
    const int np = (p.Kt - kb0 + span - 1) / span;
    int q = 0;
    for (; q + 2 < np; q += 2) {
        issue(pb, kb0 + (q + 1) * span);
        consume(pa, kb0 + q * span);
        issue(pa, kb0 + (q + 2) * span);
        consume(pb, kb0 + (q + 1) * span);
    }
    if (q + 1 < np) {
        issue(pb, kb0 + (q + 1) * span);
        consume(pa, kb0 + q * span);
        consume(pb, kb0 + (q + 1) * span);
    } else {
        consume(pa, kb0 + q * span);
    }

    auto store = [&](int t, int r_in, int ln, float v) {
        const int r = 4 * (ln >> 4) + r_in;
        const int ntt = static_cast<int>(blockIdx.x) * T + t;
        const int c = ntt * kW4TileN + (ln & 15);
        if (r >= Ml || c >= p.N || ntt >= p.Nt) return;
        w4_store<F32C>(p, z * p.c_bs + static_cast<int64_t>(m0 + r) * p.N + c, v);
    };
    // red[wave][t][r][lane], r < MR, in the activation area once every
    // wave is done reading it
    float* const red = reinterpret_cast<float*>(a_lds);
    __syncthreads();
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
        for (int r = 0; r < MR; ++r) red[((wave * T + t) * MR + r) * 64 + lane] = acc[t][r];
    __syncthreads();
    if constexpr (SWI) {
        // tiles 2j (gate) and 2j + 1 (up) -> act column tile j = blockIdx.x
        for (int idx = threadIdx.x; idx < MR * 64; idx += 64 * S) {
            const int r_in = idx / 64, ln = idx & 63;
            float g = 0.0f, u = 0.0f;
            for (int w2 = 0; w2 < S; ++w2) {
                g += red[((w2 * T + 0) * MR + r_in) * 64 + ln];
                u += red[((w2 * T + 1) * MR + r_in) * 64 + ln];
            }
            const int r = 4 * (ln >> 4) + r_in;
            const int c = static_cast<int>(blockIdx.x) * kW4TileN + (ln & 15);
            if (r < Ml && c < p.N)
                static_cast<uint16_t*>(p.C)[static_cast<int64_t>(m0 + r) * p.N + c] = f32_to_bf16(swiglu(g, u));
        }
    } else {
        for (int idx = threadIdx.x; idx < T * MR * 64; idx += 64 * S) {
            const int t = idx / (MR * 64), r = (idx / 64) % MR, ln = idx & 63;
            float sum = 0.0f;
            for (int w2 = 0; w2 < S; ++w2) sum += red[((w2 * T + t) * MR + r) * 64 + ln];
            store(t, r, ln, sum);
        }
    }
}

// ---------------------------------------------------------------------------
// Integer decode kernel (G = 64 or a multiple of 128; written for M <= 4
// rows, launched for M = 1, where converting the activations costs least).
//
// The workgroup converts its activation rows once, into LDS, to fixed point
// per 128-wide K block: q = round(x * 2^-E), with E taken from the block's
// largest magnitude so that |q| < 2^21, written as three signed base-256
// digits q = d0 + 256 d1 + 65536 d2 (d0, d1 in [-128, 127], |d2| <= 32).
// The 4-bit codes u (0..15) are int8 operands after one mask (and a shift),
// so the dot products run on v_mfma_i32_16x16x64_i8: A row 4p + r is digit
// plane p of activation row r, and accumulator rows 4p + r come out as the
// exact sums S_p = sum_k d_p[k] u[k].  Per block and scale segment,
//     sum_k x[k] (u[k] - z) = 2^E (S_0 + 256 S_1 + 65536 S_2 - z XS),
// XS = sum_k q[k] being an exact integer sum taken during the conversion.
// Lane group p of the accumulator layout holds plane p, so each lane adds
// s 2^E (w_p S_p - [p == 0] z XS) to its own fp32 accumulator (w = 1, 256,
// 65536; lane group 3 weighs 0) and the planes meet once, in the final
// cross-wave reduction.  Per 1 KiB weight tile and column tile that is 12
// decode instructions and two MFMAs, against 28 and four (plus the
// activation-sum MFMAs) for the bf16 form.
// Precision: a bf16 activation within 2^-13 of its block's largest is
// represented exactly, anything smaller (and any fp32 activation) to within
// 2^-21 of that largest; a block holding Inf or NaN makes its row's
// outputs NaN.
//
// LDS: digit planes [3][Ml][Kp] bytes, each row in MFMA operand order (the
// 16 bytes lane l reads for MFMA m of tile kt are k = 128 kt + 64 m + 32 h
// + 8 (l >> 4) + e, h = 0, 1, e = 0..7: the codes of the prepacked weight
// dwords 2m and 2m + 1 of that lane), then one float4 per (row, K tile):
// {2^E, 2^E XS(first 64-wide segment or whole tile), 2^E XS(second), 0}.
// Passes, loads and the wave-ordered reduction follow the bf16 decode kernel.
// ---------------------------------------------------------------------------
constexpr float kQMagic = 12615808.0f;         // 1.5 * 2^23 + 0x8080
constexpr uint32_t kQMagicBits = 0x4B408080u;  // bits of (kQMagic + q) for |q| < 2^22
constexpr uint32_t kNib = 0x0F0F0F0Fu;

__device__ __forceinline__ uint32_t umax32(uint32_t a, uint32_t b) { return a > b ? a : b; }
template <int CTRL>
__device__ __forceinline__ uint32_t dpp(uint32_t x) {
    return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(x), CTRL, 0xf, 0xf, false));
}
// All-reduce over the 16 lanes of a DPP row (row_ror 8, 4, 2, 1) and over
// each half row (quad_perm xor 1, xor 2, then row_half_mirror).
__device__ __forceinline__ uint32_t row16_max(uint32_t x) {
    x = umax32(x, dpp<0x128>(x));
    x = umax32(x, dpp<0x124>(x));
    x = umax32(x, dpp<0x122>(x));
    return umax32(x, dpp<0x121>(x));
}
__device__ __forceinline__ uint32_t row16_sum(uint32_t x) {
    x += dpp<0x128>(x);
    x += dpp<0x124>(x);
    x += dpp<0x122>(x);
    return x + dpp<0x121>(x);
}
__device__ __forceinline__ uint32_t row8_sum(uint32_t x) {
    x += dpp<0xB1>(x);
    x += dpp<0x4E>(x);
    return x + dpp<0x141>(x);
}

// GR (bf16, asymmetric weights): a ragged group table; grid.y walks the
// groups' rows one at a time (resolve_group_rows with one-row blocks), each
// workgroup staging its row and streaming its group's weight tiles; SWI:
// the SwiGLU epilogue over the gate / up tile pair of the workgroup (T = 2).
template <bool F32A, bool ASYM, bool F32C, int T, int NPW, int BPS, bool GBIG, int MR, bool GR = false,
          bool SWI = false>
__global__ __launch_bounds__(T == 1 ? 1024 : 512) void w4_decode_i8_kernel(W4Args p) {
    static_assert(BPS == 2 || BPS == 4, "scale segments of 64 or 128 k");
    static_assert(NPW == 4 || NPW == 8, "passes start at multiples of NPW tiles");
    static_assert(MR == 1 || MR == 4, "one row or all four");
    static_assert(!GR || (MR == 1 && !F32A && ASYM && !F32C), "grouped: one bf16 row per workgroup");
    static_assert(!SWI || (GR && T == 2), "SwiGLU: the gate / up pair of a grouped workgroup");
    constexpr int SEGS = 4 / BPS;
    constexpr int NZW = (BPS < 4) ? (NPW * SEGS + 7) / 8 : (GBIG ? NPW : 1);
    extern __shared__ __attribute__((aligned(16))) uint8_t q_lds[];

    const int S = blockDim.x >> 6;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int z = GR ? 0 : blockIdx.z;
    int m0 = 0;  // the group row of a grouped workgroup
    const uint8_t* qw = p.qw;
    const void* scales = p.scales;
    const uint32_t* zeros = p.zeros;
    if constexpr (GR) {
        int e, m_end;
        if (!resolve_group_rows(p, blockIdx.y, 1, e, m0, m_end)) return;  // uniform per workgroup
        qw = p.qws[e];
        scales = p.scs[e];
        zeros = p.zss[e];
    }
    const int Ml = GR ? 1 : min(p.M, 4);
    const int col = lane & 15;
    const int Kp = p.Kt * kW4TileK;
    uint8_t* const dig = q_lds;
    float4* const tab = reinterpret_cast<float4*>(q_lds + 3 * Ml * Kp);

    const uint8_t* qwb[T];
    const char* scb[T];
    const char* zwb[T];
#pragma unroll
    for (int t = 0; t < T; ++t) {
        const int64_t nt = min(static_cast<int>(blockIdx.x) * T + t, p.Nt - 1);
        qwb[t] = qw + z * p.qw_bs + nt * p.Kt * kW4TileBytes;
        scb[t] = static_cast<const char*>(scales) + (z * p.s_bs + nt * p.NG * 16) * (ASYM ? 2 : 4);
        zwb[t] = ASYM ? reinterpret_cast<const char*>(zeros + z * p.z_bs + nt * p.NG8 * 16) : nullptr;
    }
    const uint32_t s_col = static_cast<uint32_t>(col * (ASYM ? 2 : 4));

    struct Pass {
        u32x4_t w[NPW][T];
        uint32_t sw[NPW][T][SEGS];
        uint32_t zw[NZW][T];
    };
    auto issue = [&](Pass& P, int kt0) {
        if constexpr (ASYM) {
#pragma unroll
            for (int q = 0; q < NZW; ++q) {
                const int g = (BPS < 4) ? group_of_c<BPS, GBIG>(min(kt0, p.Kt - 1), 0, 0) + 8 * q
                                        : group_of_c<BPS, GBIG>(min(kt0 + q, p.Kt - 1), 0, p.gmul);
                const uint32_t off = static_cast<uint32_t>((min(g >> 3, p.NG8 - 1) * 16 + col) * 4);
#pragma unroll
                for (int t = 0; t < T; ++t) P.zw[q][t] = *reinterpret_cast<const uint32_t*>(zwb[t] + off);
            }
        }
#pragma unroll
        for (int i = 0; i < NPW; ++i) {
            const int kt = min(kt0 + i, p.Kt - 1);
#pragma unroll
            for (int t = 0; t < T; ++t) {
#pragma unroll
                for (int s = 0; s < SEGS; ++s) {
                    const uint32_t off = static_cast<uint32_t>(seg_group<BPS, GBIG>(kt, s, p) * 16 * (ASYM ? 2 : 4)) + s_col;
                    if constexpr (ASYM) P.sw[i][t][s] = *reinterpret_cast<const uint16_t*>(scb[t] + off);
                    else P.sw[i][t][s] = *reinterpret_cast<const uint32_t*>(scb[t] + off);
                }
                P.w[i][t] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(
                    qwb[t] + static_cast<uint32_t>(kt * kW4TileBytes + lane * 16)));
            }
        }
    };

    // 1. activations: loads first, then the first pass's weights, then the
    //    conversion (the weights are in flight meanwhile)
    const int span = S * NPW;
    const int rc = Kp >> 3;  // 8-element chunks per padded row; 16 per K tile
    const int chunks = Ml * rc;
    const char* A = static_cast<const char*>(p.A) + (z * p.a_bs + static_cast<int64_t>(m0) * p.K) * (F32A ? 4 : 2);
    constexpr int B = 4;  // chunks per thread per batch
    u32x4_t av[B], av2[B];
    auto stage_load = [&](int c0) {
#pragma unroll
        for (int b = 0; b < B; ++b) {
            const int c = c0 + b * 64 * S;
            const int r = c / rc, k = (c - r * rc) * 8;
            const bool ok = c < chunks && k < p.K;
            const int64_t e = ok ? static_cast<int64_t>(r) * p.K + k : 0;
            if constexpr (F32A) {
                av[b] = *reinterpret_cast<const u32x4_t*>(A + e * 4);
                av2[b] = *reinterpret_cast<const u32x4_t*>(A + e * 4 + 16);
            } else {
                av[b] = *reinterpret_cast<const u32x4_t*>(A + e * 2);
            }
        }
    };
    // Chunk c (row r, k = kk .. kk+7) -> digits.  Chunks are dealt to
    // consecutive threads and a K tile is 16 chunks, so each DPP row of 16
    // lanes holds exactly one (row, K tile) block, valid or past the end as a
    // whole: the block reductions are row reductions.
    auto stage_store = [&](int c0) {
#pragma unroll
        for (int b = 0; b < B; ++b) {
            const int c = c0 + b * 64 * S;
            const int r = c / rc, kk = (c - r * rc) * 8;
            // a chunk past K (the zero padding of the last tile) or past the
            // last row holds whatever the clamped load read: it takes no part
            // in the block maximum and is scaled by 0 (q = 0); only non-finite
            // values there could leak, and those sit in row 0, whose outputs
            // are then NaN anyway
            const bool ok = c < chunks && kk < p.K;
            float f[8];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                if constexpr (F32A) {
                    f[i] = __uint_as_float(av[b][i]);
                    f[i + 4] = __uint_as_float(av2[b][i]);
                } else {
                    f[2 * i] = __uint_as_float(av[b][i] << 16);
                    f[2 * i + 1] = __uint_as_float(av[b][i] & 0xffff0000u);
                }
            }
            uint32_t mx = 0;
#pragma unroll
            for (int i = 0; i < 8; ++i) mx = umax32(mx, __float_as_uint(f[i]) & 0x7fffffffu);
            mx = row16_max(ok ? mx : 0u);
            const int be = static_cast<int>(mx >> 23);  // 255: Inf or NaN in the block
            const int E = min(max(be - 147, -126), 107);
            const float inv = ok ? __uint_as_float(static_cast<uint32_t>(127 - E) << 23) : 0.0f;
            // q = round(f * 2^-E): bits(kQMagic + f*2^-E) = kQMagicBits + q, so
            // d = bits - 0x4B400000 = q + 0x8080, whose byte 2 is the top digit
            // and whose bytes 0, 1 are the low digits + 128 (re-biased below,
            // four at a time, once they are packed into planes)
            uint32_t d[8], vs = 0;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                d[i] = __float_as_uint(__builtin_fmaf(f[i], inv, kQMagic)) - (kQMagicBits - 0x8080u);
                vs += d[i];
            }
            uint32_t pl[3][2];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const uint32_t* e = d + 4 * h;
                const uint32_t x01 = __builtin_amdgcn_perm(e[1], e[0], 0x05010400u);
                const uint32_t x23 = __builtin_amdgcn_perm(e[3], e[2], 0x05010400u);
                const uint32_t y01 = __builtin_amdgcn_perm(e[1], e[0], 0x06020602u);
                const uint32_t y23 = __builtin_amdgcn_perm(e[3], e[2], 0x06020602u);
                pl[0][h] = __builtin_amdgcn_perm(x23, x01, 0x05040100u) ^ 0x80808080u;
                pl[1][h] = __builtin_amdgcn_perm(x23, x01, 0x07060302u) ^ 0x80808080u;
                pl[2][h] = __builtin_amdgcn_perm(y23, y01, 0x05040100u);
            }
            const int pos = (kk & ~63) + 16 * ((kk >> 3) & 3) + 8 * ((kk >> 5) & 1);
            if (c < chunks) {
#pragma unroll
                for (int pp = 0; pp < 3; ++pp)
                    *reinterpret_cast<u32x2_t*>(dig + (pp * Ml + r) * Kp + pos) = u32x2_t{pl[pp][0], pl[pp][1]};
            }
            const uint32_t xs = vs - 8u * 0x8080u;  // this chunk's sum of q
            const float sc = (be == 255) ? __uint_as_float(0x7fc00000u)
                                         : __uint_as_float(static_cast<uint32_t>(127 + E) << 23);
            float4 tv;
            if constexpr (BPS == 4) {
                const uint32_t x16 = row16_sum(xs);
                tv = float4{sc, static_cast<float>(static_cast<int>(x16)) * sc, 0.0f, 0.0f};
            } else {
                const uint32_t x8 = row8_sum(xs);
                const uint32_t x8b = dpp<0x128>(x8);  // the second half row's sum
                tv = float4{sc, static_cast<float>(static_cast<int>(x8)) * sc,
                            static_cast<float>(static_cast<int>(x8b)) * sc, 0.0f};
            }
            if ((lane & 15) == 0 && c < chunks) tab[r * p.Kt + (kk >> 7)] = tv;
        }
    };
    const int kb0 = wave * NPW;
    stage_load(threadIdx.x);
    Pass pa, pb;
    issue(pa, kb0);
    stage_store(threadIdx.x);
    for (int c0 = threadIdx.x + B * 64 * S; c0 < chunks; c0 += B * 64 * S) {
        stage_load(c0);
        stage_store(c0);
    }
    __syncthreads();

    // 2. main loop.  A row (lane & 15) = 4p + r reads digit plane p of row r
    //    (plane 3 does not exist: those rows read plane 2 and weigh 0; rows
    //    r >= M read row M-1, their outputs are never stored)
    const int g4 = lane >> 4;
    const float wl = g4 == 0 ? 1.0f : (g4 == 1 ? 256.0f : (g4 == 2 ? 65536.0f : 0.0f));
    const float zl = g4 == 0 ? 1.0f : 0.0f;
    const uint8_t* const abase =
        dig + (min((lane & 15) >> 2, 2) * Ml + min(lane & 3, Ml - 1)) * Kp + 16 * g4;
    float acc[T][MR];
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
        for (int j = 0; j < MR; ++j) acc[t][j] = 0.0f;

    auto tile = [&](const Pass& P, int i, int kt) {
        const u32x4_t a0 = *reinterpret_cast<const u32x4_t*>(abase + kt * kW4TileK);
        const u32x4_t a1 = *reinterpret_cast<const u32x4_t*>(abase + kt * kW4TileK + 64);
        float W[MR], Z0[MR], Z1[MR];
#pragma unroll
        for (int j = 0; j < MR; ++j) {
            const float4 tb = tab[min(j, Ml - 1) * p.Kt + kt];
            W[j] = wl * tb.x;
            Z0[j] = zl * tb.y;
            Z1[j] = zl * tb.z;
        }
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const u32x4_t w = P.w[i][t];
            const u32x4_t b0 = {w[0] & kNib, (w[0] >> 4) & kNib, w[1] & kNib, (w[1] >> 4) & kNib};
            const u32x4_t b1 = {w[2] & kNib, (w[2] >> 4) & kNib, w[3] & kNib, (w[3] >> 4) & kNib};
            const i32x4_t zero4 = {0, 0, 0, 0};
            i32x4_t sv[SEGS];
            if constexpr (BPS == 4) {
                sv[0] = mfma_i8_16x16x64(a1, b1, mfma_i8_16x16x64(a0, b0, zero4));
            } else {
                sv[0] = mfma_i8_16x16x64(a0, b0, zero4);
                sv[1] = mfma_i8_16x16x64(a1, b1, zero4);
            }
#pragma unroll
            for (int s = 0; s < SEGS; ++s) {
                const int g = seg_group<BPS, GBIG>(kt, s, p);
                float sc, zc;
                if constexpr (ASYM) {
                    sc = f16_to_f32(static_cast<uint16_t>(P.sw[i][t][s]));
                    const uint32_t word = P.zw[(BPS < 4) ? (i * SEGS + s) / 8 : (GBIG ? i : 0)][t];
                    zc = static_cast<float>((word >> (4 * (g & 7))) & 15u);
                } else {
                    sc = __uint_as_float(P.sw[i][t][s]);
                    zc = 8.0f;  // implied zero point
                }
#pragma unroll
                for (int j = 0; j < MR; ++j) {
                    const float part = static_cast<float>(sv[s][j]) * W[j];
                    acc[t][j] = __builtin_fmaf(sc, __builtin_fmaf(-zc, s == 0 ? Z0[j] : Z1[j], part), acc[t][j]);
                }
            }
        }
    };
    // a full pass runs its tiles without a branch between them, so the
    // compiler can overlap one tile's MFMA latency with the next tile's decode
    auto consume = [&](const Pass& P, int kb) {
        const int n = min(NPW, p.Kt - kb);
        if (n == NPW) {
#pragma unroll
            for (int i = 0; i < NPW; ++i) tile(P, i, kb + i);
        } else {
#pragma unroll
            for (int i = 0; i < NPW; ++i)
                if (i < n) tile(P, i, kb + i);
        }
    };
    const int np = (p.Kt - kb0 + span - 1) / span;
    int q = 0;
    for (; q + 2 < np; q += 2) {
        issue(pb, kb0 + (q + 1) * span);
        consume(pa, kb0 + q * span);
        issue(pa, kb0 + (q + 2) * span);
        consume(pb, kb0 + (q + 1) * span);
    }
    if (q + 1 < np) {
        issue(pb, kb0 + (q + 1) * span);
        consume(pa, kb0 + q * span);
        consume(pb, kb0 + (q + 1) * span);
    } else {
        consume(pa, kb0 + q * span);
    }

    // 3. red[wave][t][j][lane]; output (row j, column c) sums the waves in
    //    order, then the three digit-plane lane groups
    float* const red = reinterpret_cast<float*>(q_lds);
    __syncthreads();
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
        for (int j = 0; j < MR; ++j) red[((wave * T + t) * MR + j) * 64 + lane] = acc[t][j];
    __syncthreads();
    if constexpr (SWI) {
        // tiles 2j (gate) and 2j + 1 (up) -> act column tile j = blockIdx.x
        for (int c = threadIdx.x; c < 16; c += 64 * S) {
            float g = 0.0f, u = 0.0f;
            for (int w2 = 0; w2 < S; ++w2) {
                const float* gp = red + (w2 * T + 0) * 64 + c;
                const float* up = red + (w2 * T + 1) * 64 + c;
                g += gp[0] + gp[16] + gp[32];
                u += up[0] + up[16] + up[32];
            }
            const int cn = static_cast<int>(blockIdx.x) * kW4TileN + c;
            if (cn < p.N)
                static_cast<uint16_t*>(p.C)[static_cast<int64_t>(m0) * p.N + cn] = f32_to_bf16(swiglu(g, u));
        }
        return;
    }
    for (int idx = threadIdx.x; idx < T * MR * 16; idx += 64 * S) {
        const int t = idx / (MR * 16), j = (idx / 16) % MR, c = idx & 15;
        float sum = 0.0f;
        for (int w2 = 0; w2 < S; ++w2) {
            const float* rp = red + ((w2 * T + t) * MR + j) * 64 + c;
            sum += rp[0] + rp[16] + rp[32];
        }
        const int ntt = static_cast<int>(blockIdx.x) * T + t;
        const int cn = ntt * kW4TileN + c;
        if (j < (GR ? 1 : p.M) && cn < p.N && ntt < p.Nt)
            w4_store<F32C>(p, z * p.c_bs + static_cast<int64_t>(m0 + j) * p.N + cn, sum);
    }
}

// ---------------------------------------------------------------------------
// Prefill tile kernel: bf16 activations and output, asymmetric int4 weights,
// many rows (plain, uniform batches, ragged groups).  A 256-thread
// workgroup owns an output tile in one of three layouts (L):
//   L = 0: 128 x 128, waves (wm, wn) in 2 x 2;
//   L = 1:  64 x 256, waves wn = 0..3 on the same 64 rows (a ragged group's
//           rows are padded to 64, not 128);
//   L = 2:  64 x 128 with K split in two, waves (ks, wn) in 2 x 2: half ks
//           walks K tiles ks*ceil(Kt/2) .. and half 1 hands its accumulators
//           to half 0 through LDS at the end (a fixed order: deterministic);
//           twice the workgroups of L = 1 where those cannot fill the chip;
//   L = 3:  64 x 128 with K split in four, eight waves (ks, wn) in 4 x 2;
//   L = 4:  64 x 256 with K split in two, eight waves (ks, wn) in 2 x 4
//           (split-K launches: two waves per SIMD on L = 1's grid).
// A wave owns 64 rows x 64 columns (4 column tiles) as 4 x 4 blocks of
// 16x16x32 MFMA accumulators in every layout.  Per 128-deep K tile:
//   - the workgroup's activations (64 rows x 128 k per row group or K half)
//     go global -> LDS
//     by DMA into one of two buffers; 16-byte chunk c of row r sits in slot
//     c ^ (r & 15), so the 16 rows of a fragment read hit 16 different bank
//     groups;
//   - each wave loads its four 1 KiB weight tiles and their scales / zero
//     words straight into registers, one K tile ahead of their use;
//   - per K tile and row block: xs = -144 * sum_k x (an MFMA against a -144
//     operand) seeds each column tile's chain t = xs + sum_k x*(144 + u - z)
//     (MFMA on exact bf16 integers, the zero point folded into the codes),
//     so t = sum_k x*(u - z) and the group correction is acc += s * t; each
//     weight tile is decoded once per 64 rows instead of once per 16.
// The K loop alternates two register sets (A buffer and weights of the tile
// in flight vs the tile in use) and meets at one `s_waitcnt vmcnt(0)` +
// `s_barrier` per tile: before it, only the tile about to be used is in
// flight.  Every load is unconditional (rows past the end read the last
// row; column tiles past Nt re-read the last one).  Requires K % 128 == 0
// (the activations are not zero-padded in LDS).
// ---------------------------------------------------------------------------
constexpr int MM_CT = 4;  // column tiles per wave
// word 3 of a raw buffer resource (gfx9 family): 32-bit data format, no
// swizzle, offsets taken as given
constexpr int kBufWord3 = 0x00020000;
// rows per workgroup tile: L == 0 ? 128 : 16 * RB; column tiles per
// workgroup: (L == 1 || L == 4 ? 4 : 2) * MM_CT; K parts: 2 (L == 2, 4) or
// 4 (L == 3); one activation buffer: 128 rows (L == 0) or one region of
// 16 * RB rows per K part, of 128 k x 2 bytes

#define LHQ_LDS_AS __attribute__((address_space(3)))

// SK (split-K, plain launches only): grid.z is the K split instead of the
// batch; the workgroup's K parts share its split's K range, and it writes
// fp32 partial sums to p.ws[split][M][N] for w4_splitk_reduce_kernel to add
// in split order.  RB (L != 0): 16-row blocks per wave, 64 rows at RB = 4;
// RB = 1 or 2 serve up to 16 or 32 rows without the MFMAs of 64.
// F32 (the reference interface, gemm_quant.cpp:54-82): fp32 activations,
// symmetric weights (implied zero point 8) with fp32 scales, fp32 output
// with alpha / beta.  The activation tile is staged in LDS as fp32 (512
// bytes per row) and each fragment is split into bf16 hi + lo operands as it
// is read, so every product runs twice on the bf16 MFMA (product error near
// 2^-17 relative, as in the 16-row kernel's fp32 form); 64 x 256 tiles only.

// Persistent grouped launches (PK): one 64 x 256 tile's fp32 partial sums,
// in f32x4 (one workspace slot, 64 KiB)
constexpr int kPkTileVecs = 4 * 4 * MM_CT * 64;
constexpr int64_t kPkSlotBytes = int64_t{kPkTileVecs} * 16;
constexpr int kPkMinSegKt = 4;  // K tiles per stream-K part at least

// Row blocks of rb rows over a grouped launch's table, counted as
// resolve_group_rows lays them out (the same clamps); uniform.
__device__ __forceinline__ int count_row_blocks(const W4Args& p, int rb) {
    const int lane = threadIdx.x & 63;
    int total = 0;
    for (int e0 = 0; e0 < p.num_groups; e0 += 64) {
        const int g = e0 + lane;
        int nb = 0;
        if (g < p.num_groups) {
            const int r0 = min(max(p.offsets[g], 0), p.row_capacity);
            const int r1 = min(max(p.offsets[g + 1], r0), p.row_capacity);
            nb = (r1 - r0 + rb - 1) / rb;
        }
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) nb += __shfl_xor(nb, d, 64);
        total += nb;
    }
    return __builtin_amdgcn_readfirstlane(total);
}

// The work split of a persistent grouped launch over P workers (the tile
// kernel and the fixup kernel derive the same plan from the same table).
struct PkPlan {
    int X;             // column groups of 256
    int64_t dp_tiles;  // tiles dealt out whole
    int64_t R;         // tiles past the last whole round
    bool sk;           // the R tiles spread along K (only when R = T < P)
    int64_t I;         // their K tiles, R * Kt
    int Ps;            // workers sharing them
};
__device__ __forceinline__ PkPlan pk_plan(const W4Args& p, int P) {
    PkPlan pl;
    pl.X = (p.Nt + 4 * MM_CT - 1) / (4 * MM_CT);
    const int64_t T = static_cast<int64_t>(pl.X) * count_row_blocks(p, 64);
    const int64_t q = T / P;
    pl.R = T - q * P;
    pl.I = pl.R * p.Kt;
    pl.Ps = static_cast<int>(min<int64_t>(P, max<int64_t>(1, pl.I / kPkMinSegKt)));
    pl.sk = p.ws && q == 0 && 4 * pl.R <= 3 * static_cast<int64_t>(P) && pl.R > 0 && pl.Ps + pl.R - 1 <= p.pk_slots;
    pl.dp_tiles = pl.sk ? q * P : T;
    return pl;
}
// The worker whose part of the stream-K range holds K tile x of it: parts
// are [floor(w I / Ps), floor((w + 1) I / Ps)), so w = ceil((x + 1) Ps / I) - 1.
__device__ __forceinline__ int pk_worker_of(int64_t x, const PkPlan& pl) {
    return static_cast<int>(((x + 1) * pl.Ps + pl.I - 1) / pl.I - 1);
}

// The bf16 epilogue of one wave's 16 RB x 16 MM_CT block: accumulator
// (i, c) element r is row r0 + 16 i + 4 (lane >> 4) + r, column lane & 15 of
// column tile nt0 + c.  SWI: blocks (c, c + 1) hold a gate tile and its up
// tile (nt0 even), stored as act column tile (nt0 + c) / 2.
template <bool SWI, int RB>
__device__ __forceinline__ void store_bf16_block(const W4Args& p, uint16_t* C, const f32x4_t (&acc)[RB][MM_CT],
                                                 int nt0, int r0, int m_end, int lane) {
    const int col = lane & 15;
#pragma unroll
    for (int c = 0; c < MM_CT; c += SWI ? 2 : 1) {
        const int nt = nt0 + c;
        const int cn = (SWI ? (nt >> 1) : nt) * kW4TileN + col;
        if (nt >= p.Nt || cn >= p.N) continue;
#pragma unroll
        for (int i = 0; i < RB; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = r0 + i * 16 + 4 * (lane >> 4) + r;
                if (row >= m_end) continue;
                if constexpr (SWI)
                    C[static_cast<int64_t>(row) * p.N + cn] = f32_to_bf16(swiglu(acc[i][c][r], acc[i][c + 1][r]));
                else C[static_cast<int64_t>(row) * p.N + cn] = f32_to_bf16(acc[i][c][r]);
            }
    }
}

// A pointer that is the same in every lane, moved to scalar registers.
template <typename T>
__device__ __forceinline__ T* uniform_ptr(T* q) {
    const uint64_t v = reinterpret_cast<uint64_t>(q);
    const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v));
    const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v >> 32));
    return reinterpret_cast<T*>((static_cast<uint64_t>(hi) << 32) | lo);
}

// One output tile of w4_mma_kernel: column group bx, row tile by, batch or
// split bz, K tiles [kb, ke) (a split-K launch takes its range from bz).
// pk_slot >= 0 (persistent grouped launches): [kb, ke) is one K segment of
// a tile split across workgroups, whose fp32 partial sums go to workspace
// slot pk_slot in register order; w4_pk_fixup_kernel adds the segments.
template <int BPS, bool GBIG, bool GR, bool SWI, int L, bool SK, int RB, bool F32, bool PK>
__device__ __forceinline__ void mma_tile(const W4Args& p, uint8_t* mm_lds, int bx, int by, int bz, int kb_in,
                                         int ke_in, int pk_slot) {
    static_assert(RB == 4 || (RB <= 2 && L != 0 && !GR), "16- and 32-row blocks on plain launches, not 128 x 128");
    static_assert(!SK || (!GR && !SWI), "split-K on plain launches only");
    static_assert(!PK || (GR && L == 1 && RB == 4 && !SK && !F32), "persistent launches: grouped 64 x 256 tiles");
    static_assert(L != 4 || SK, "the 8-wave 64 x 256 layout on split-K launches only");
    static_assert(!F32 || (!GR && !SWI && L != 0 && L != 4 && (RB == 4 ? L == 1 : true)),
                  "the fp32 interface: plain launches, 64 x 256 tiles or 16- / 32-row blocks");
    constexpr int SEGS = 4 / BPS;
    constexpr int NW = (L >= 3) ? 8 : 4;                                  // waves
    constexpr int NK = (L == 2 || L == 4) ? 2 : (L == 3) ? 4 : 1;        // K parts
    constexpr int BM = (L == 0) ? 128 : 16 * RB, WN = (L == 1 || L == 4) ? 4 : 2;
    constexpr int RR = (L == 0) ? 64 : 16 * RB;                          // rows per LDS region
    constexpr int EA = F32 ? 4 : 2;                                      // activation bytes
    constexpr int RBYTES = kW4TileK * EA;                                // LDS bytes per row
    constexpr int CPR = RBYTES / 16;                                     // 16-byte chunks per row
    constexpr int A_BYTES = ((L == 0) ? 128 : NK * RR) * RBYTES;
    constexpr int DMA = A_BYTES / 1024 / NW;  // activation DMAs per wave per K tile
    // mm_lds: 2 x A_BYTES (+ the fp32 form's partial sums)
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // this wave's LDS activation region (row group or K part), row group,
    // K part and column group
    const int wr = (L == 1) ? 0 : (L == 4) ? (wave >> 2) : (wave >> 1);
    const int wm = (L == 0) ? wr : 0;
    const int ks = (NK > 1) ? wr : 0;
    const int wn = (L == 1) ? wave : (L == 4) ? (wave & 3) : (wave & 1);
    // K tiles [kb, ke) of this workgroup (its split, or all of K), in NK
    // parts of kh tiles; this wave's part starts at kofs
    const int kb = SK ? bz * p.kps : kb_in;
    const int ke = SK ? min(p.Kt, kb + p.kps) : ke_in;
    const int kh = (ke - kb + NK - 1) / NK;
    const int kofs = kb + ks * kh;
    const int z = SK ? 0 : bz;
    int m0, m_end;
    const uint8_t* qw;
    const uint16_t* sc;
    const uint32_t* zs;
    if constexpr (GR) {
        int e;
        if (!resolve_group<BM>(p, by, e, m0, m_end)) return;  // uniform per workgroup
        qw = p.qws[e];
        sc = static_cast<const uint16_t*>(p.scs[e]);
        zs = p.zss[e];
        if constexpr (PK) {
            // after an earlier tile's stores these table loads are vector
            // loads; their (uniform) results go back to scalar registers,
            // where the buffer descriptors need them
            qw = uniform_ptr(qw);
            sc = uniform_ptr(sc);
            zs = uniform_ptr(zs);
        }
    } else {
        m0 = by * BM;
        m_end = p.M;
        qw = p.qw + z * p.qw_bs;
        sc = static_cast<const uint16_t*>(p.scales) + z * p.s_bs;
        zs = p.zeros + z * p.z_bs;
    }
    const uint16_t* A = static_cast<const uint16_t*>(p.A) + (GR ? 0 : z * p.a_bs);
    const float* Af = static_cast<const float*>(p.A) + (GR ? 0 : z * p.a_bs);
    const float* scf = static_cast<const float*>(p.scales) + (GR ? 0 : z * p.s_bs);
    const int col = lane & 15;

    // activation DMA q of this wave: chunk idx = (DMA*wave + q)*64 + lane is
    // LDS row idx >> 4, LDS slot idx & 15, global chunk slot ^ (row & 15);
    // LDS row r lies in region r / RR, the region of the K part whose waves
    // issue it (DMA*4 rows per wave); offsets are taken from the workgroup's
    // first row (64 rows x K elements at most)
    // (a fixed bound: a bound that depends on a template parameter, with the
    // array captured by the lambdas below, makes hipcc's host pass drop the
    // kernel's launch stub without a diagnostic; entries past DMA are unused)
    static_assert(DMA >= 1 && DMA <= 8, "activation DMAs per wave");
    constexpr int DROWS = 64 * DMA / CPR;  // LDS rows one wave's DMAs fill
    static_assert(NK == 1 || (RR % DROWS == 0 && RR / DROWS == NW / NK),
                  "each wave's DMA rows lie in its own K part's region");
    uint32_t a_voff[8];  // byte offsets from the workgroup's first row
#pragma unroll
    for (int q = 0; q < DMA; ++q) {
        const int idx = (DMA * wave + q) * 64 + lane;
        const int r = idx / CPR, slot = idx % CPR;  // LDS row r: region r / RR (this wave's, wr)
        const int row = min(m0 + ((NK > 1) ? (r % RR) : r), m_end - 1);
        a_voff[q] = (static_cast<uint32_t>(row - m0) * static_cast<uint32_t>(p.K) +
                     static_cast<uint32_t>((slot ^ (r & 15)) * (16 / EA))) * EA;
    }
    const uint32_t s_half = 16u * (col & 1);
    // Buffer resources based at this workgroup's first row and this wave's
    // first column tile: the per-lane part of each address is fixed for the
    // whole K loop (voffset) and the per-tile part is scalar (soffset), so
    // a tile's loads take no vector address arithmetic (and a read past a
    // resource's extent returns zero instead of faulting).
    constexpr int ES = F32 ? 4 : 2;  // scale bytes
    const int nt0 = min(bx * WN * MM_CT + wn * MM_CT, p.Nt - 1);
    int dnt[MM_CT];
#pragma unroll
    for (int c = 0; c < MM_CT; ++c) dnt[c] = min(nt0 + c, p.Nt - 1) - nt0;
    const int nt_left = p.Nt - nt0;
    // extents in bytes, at most 2^32 - 1 (offsets within them are 32-bit)
    auto extent = [](int64_t bytes) {
        return static_cast<int>(static_cast<uint32_t>(bytes < int64_t{0xFFFFFFFF} ? bytes : int64_t{0xFFFFFFFF}));
    };
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(qw) + static_cast<int64_t>(nt0) * p.Kt * kW4TileBytes, 0,
        extent(static_cast<int64_t>(nt_left) * p.Kt * kW4TileBytes), kBufWord3);
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        F32 ? static_cast<void*>(const_cast<float*>(scf) + static_cast<int64_t>(nt0) * p.NG * 16)
            : static_cast<void*>(const_cast<uint16_t*>(sc) + static_cast<int64_t>(nt0) * p.NG * 16),
        0, extent(static_cast<int64_t>(nt_left) * p.NG * 16 * ES), kBufWord3);
    const __amdgpu_buffer_rsrc_t rz = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint32_t*>(zs) + static_cast<int64_t>(nt0) * p.NG8 * 16, 0,
        extent(static_cast<int64_t>(nt_left) * p.NG8 * 16 * 4), kBufWord3);
    const __amdgpu_buffer_rsrc_t ra_ = __builtin_amdgcn_make_buffer_rsrc(
        F32 ? static_cast<void*>(const_cast<float*>(Af) + static_cast<int64_t>(m0) * p.K)
            : static_cast<void*>(const_cast<uint16_t*>(A) + static_cast<int64_t>(m0) * p.K),
        0, extent(static_cast<int64_t>(m_end - m0) * p.K * EA), kBufWord3);
    const int w_voff = lane * 16;
    const int s_voff = (F32 ? col : (col & ~1)) * ES;
    const int z_voff = col * 4;

    struct Regs {
        u32x4_t w[MM_CT];
        uint32_t sw[MM_CT][SEGS];
        uint32_t zw[MM_CT];
    };
    // all loads of K tile kt (clamped) into LDS buffer buf and registers R
    auto issue = [&](uint8_t* buf, Regs& R, int kt_in) {
        const int kt = min(kt_in + kofs, p.Kt - 1);
#pragma unroll
        for (int q = 0; q < DMA; ++q)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(ra_, (LHQ_LDS_AS void*)(buf + (DMA * wave + q) * 1024), 16,
                                                     a_voff[q], kt * kW4TileK * EA, 0, 0);
#pragma unroll
        for (int c = 0; c < MM_CT; ++c) {
            if constexpr (!F32)
                R.zw[c] = __builtin_amdgcn_raw_buffer_load_b32(
                    rz, z_voff, (dnt[c] * p.NG8 + (group_of_c<BPS, GBIG>(kt, 0, p.gmul) >> 3)) * 16 * 4, 0);
#pragma unroll
            for (int s = 0; s < SEGS; ++s)
                R.sw[c][s] = __builtin_amdgcn_raw_buffer_load_b32(
                    rs, s_voff, (dnt[c] * p.NG + group_of_c<BPS, GBIG>(kt, s, p.gmul)) * 16 * ES, 0);
            R.w[c] = __builtin_amdgcn_raw_buffer_load_b128(rw, w_voff, (dnt[c] * p.Kt + kt) * kW4TileBytes, 0);
        }
    };

    f32x4_t acc[RB][MM_CT];
#pragma unroll
    for (int i = 0; i < RB; ++i)
#pragma unroll
        for (int c = 0; c < MM_CT; ++c) acc[i][c] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    const u32x4_t m144 = {kM144Bf16x2, kM144Bf16x2, kM144Bf16x2, kM144Bf16x2};
    // fragment (row block i, k block j): LDS row 64*wr + 16*i + (lane & 15), k
    // chunk 4j + (lane >> 4), stored in slot chunk ^ (lane & 15)
    const uint32_t a_frag = static_cast<uint32_t>((wr * RR + col) * RBYTES);

    // a wave whose 64 rows all lie past the block's last row (a ragged
    // group's tail block, or M <= 64) has nothing to compute; it still
    // takes part in the loads and rendezvous, and its SIMD time goes to
    // the other waves resident there
    const bool live = m0 + 64 * wm < m_end;
    auto compute = [&](const uint8_t* buf, const Regs& R, int kt_in) {
        const int kt = kt_in + kofs;
        // the last K part may be short; the fp32 form has a barrier inside,
        // which every wave of the workgroup reaches with or without work
        const bool active = live && kt < ke;
        if (!F32 && !active) return;
        if constexpr (F32) {
            // Symmetric codes: 16 - 8 in every byte.  The VALU phase decodes
            // the weights and splits the K part's activation rows into bf16
            // hi + lo in place: the RB x 4 (row block, 32-k block) units of
            // the region are dealt out in order to its WPR waves, UPW each,
            // and each lane overwrites the two fp32 chunks it read with their
            // hi and lo halves, so no lane writes what another still reads.
            // Each wave also adds its units' activation sums into partial xs
            // per row block in LDS (one partial per row block where a wave
            // holds whole row blocks, PS per row block otherwise).  After a
            // barrier the matrix phase, at raised priority, reads every row
            // block's hi / lo fragments and adds its partial sums.
            constexpr int WPR = NW / NK;               // waves sharing the region
            constexpr int UPW = 4 * RB / WPR;          // units per wave
            constexpr int PS = UPW >= 4 ? 1 : 4 / UPW; // partial sums per row block
            static_assert(UPW * WPR == 4 * RB && (UPW % 4 == 0 || 4 % UPW == 0), "units per wave");
            f32x4_t* const xs_l = reinterpret_cast<f32x4_t*>(mm_lds + 2 * A_BYTES) + wr * RB * PS * 64;
            u32x4_t b[MM_CT][4];
            float scv[MM_CT];
#pragma unroll
            for (int c = 0; c < MM_CT; ++c) {
#pragma unroll
                for (int j = 0; j < 4; ++j) b[c][j] = w4_operand_z(R.w[c][j], 0x08080808u);
                scv[c] = __uint_as_float(R.sw[c][0]);
            }
            // fp32 chunk c0 = 8j + 2(lane >> 4) of a row and the next hold 8
            // activations; after the split they hold their hi and lo halves
            auto chunk = [&](int i, int j, int h) {
                const int c0 = 8 * j + 2 * (lane >> 4) + h;
                return const_cast<uint8_t*>(buf) + a_frag + i * 16 * RBYTES + ((c0 ^ col) * 16);
            };
            if (active) {
                f32x4_t xs = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int q = 0; q < UPW; ++q) {
                    const int u = wn * UPW + q, i = u / 4, j = u % 4;
                    const f32x4_t x0 = *reinterpret_cast<const f32x4_t*>(chunk(i, j, 0));
                    const f32x4_t x1 = *reinterpret_cast<const f32x4_t*>(chunk(i, j, 1));
                    const float v[8] = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
                    u32x4_t ah, al;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const uint16_t h0 = f32_to_bf16(v[2 * e]), h1 = f32_to_bf16(v[2 * e + 1]);
                        ah[e] = static_cast<uint32_t>(h0) | (static_cast<uint32_t>(h1) << 16);
                        al[e] = pack_bf16x2(v[2 * e] - bf16_to_f32(h0), v[2 * e + 1] - bf16_to_f32(h1));
                    }
                    *reinterpret_cast<u32x4_t*>(chunk(i, j, 0)) = ah;
                    *reinterpret_cast<u32x4_t*>(chunk(i, j, 1)) = al;
                    xs = mfma_bf16_16x16x32(ah, m144, xs);
                    xs = mfma_bf16_16x16x32(al, m144, xs);
                    if (j == 3 || q == UPW - 1) {
                        // row block i's sum over this wave's units: partial
                        // (u % 4) / UPW of PS (0 when the wave holds the block)
                        xs_l[(i * PS + (PS > 1 ? (u % 4) / UPW : 0)) * 64 + lane] = xs;
                        xs = f32x4_t{0.f, 0.f, 0.f, 0.f};
                    }
                }
            }
            // every wave's splits and sums are in LDS (lgkmcnt(0); the next
            // tile's loads stay in flight); the empty asm statements keep the
            // compiler from moving LDS accesses across the barrier
            __builtin_amdgcn_s_waitcnt(0xC07F);
            asm volatile("" ::: "memory");
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
            if (!active) return;
            __builtin_amdgcn_s_setprio(1);
#pragma unroll
            for (int i = 0; i < RB; ++i) {
                u32x4_t ah[4], al[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    ah[j] = *reinterpret_cast<const u32x4_t*>(chunk(i, j, 0));
                    al[j] = *reinterpret_cast<const u32x4_t*>(chunk(i, j, 1));
                }
                f32x4_t xs = xs_l[i * PS * 64 + lane];
#pragma unroll
                for (int q = 1; q < PS; ++q) {
                    const f32x4_t x2 = xs_l[(i * PS + q) * 64 + lane];
#pragma unroll
                    for (int r = 0; r < 4; ++r) xs[r] += x2[r];
                }
#pragma unroll
                for (int c = 0; c < MM_CT; ++c) {
                    f32x4_t t = xs;
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        t = mfma_bf16_16x16x32(ah[j], b[c][j], t);
                        t = mfma_bf16_16x16x32(al[j], b[c][j], t);
                    }
#pragma unroll
                    for (int r = 0; r < 4; ++r) acc[i][c][r] = __builtin_fmaf(scv[c], t[r], acc[i][c][r]);
                }
            }
            __builtin_amdgcn_s_setprio(0);
            return;
        }
        static_assert(SEGS == 1, "one scale segment per K tile");
        const int g = group_of_c<BPS, GBIG>(kt, 0, p.gmul);
        // 16 - z of column tile c in every byte (a byte broadcast, not a
        // multiply: v_mul_lo_u32 issues at a quarter of the VALU rate)
        auto zero_bytes = [&](int c) {
            return __builtin_amdgcn_perm(0u, 16u - ((R.zw[c] >> (4 * (g & 7))) & 15u), 0u);
        };
        auto frag = [&](int i, int j) {
            return *reinterpret_cast<const u32x4_t*>(buf + a_frag + i * 16 * 256 + (((4 * j + (lane >> 4)) ^ col) * 16));
        };
        // The zero point enters the weight operand: each code byte gets
        // 16 - z added before it becomes a bf16 integer, which is then
        // 144 + u - z (exact), so the chain seeded with xs = -144 * sum x
        // (the MFMA against a -144 operand, per row block) yields
        // t = sum_k x * (u - z) and the group's correction is acc += s * t.
        auto correct = [&](int c, int i, const f32x4_t& t, float sc) {
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[i][c][r] = __builtin_fmaf(sc, t[r], acc[i][c][r]);
        };
        if constexpr (RB == 4) {
            // Two phases per K tile.  First the VALU phase: every weight
            // operand of the tile (4 column tiles x 4 k blocks, decoded once
            // per 64 rows).  Then, at raised wave priority, the matrix phase:
            // per row block its fragments (the next block's read ahead), its
            // sums and its four chains, each chain's correction issued behind
            // the next chain.  The two waves sharing a SIMD (two workgroups
            // per CU) drift into opposite phases, and the priority lets the
            // wave in its matrix phase issue first, so one wave's decode runs
            // under the other's MFMAs (measured at M=4096, K=8192, N=28672:
            // 1870-1880 against 2029 us with the interleaved schedule; the
            // same split without the priority change was 3% slower than it).
            u32x4_t b[MM_CT][4];
            float scs[MM_CT];
#pragma unroll
            for (int c = 0; c < MM_CT; ++c) {
                const uint32_t zb = zero_bytes(c);
#pragma unroll
                for (int j = 0; j < 4; ++j) b[c][j] = w4_operand_z(R.w[c][j], zb);
                scs[c] = f16_to_f32(static_cast<uint16_t>(R.sw[c][0] >> s_half));
            }
            u32x4_t a0[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) a0[j] = frag(0, j);
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_s_setprio(1);
            f32x4_t tp = {0.f, 0.f, 0.f, 0.f};
            float sp = 0.f;
#pragma unroll
            for (int i = 0; i < RB; ++i) {
                u32x4_t a1[4];
                if (i + 1 < RB) {
#pragma unroll
                    for (int j = 0; j < 4; ++j) a1[j] = frag(i + 1, j);
                }
                f32x4_t xs = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int j = 0; j < 4; ++j) xs = mfma_bf16_16x16x32(a0[j], m144, xs);
#pragma unroll
                for (int c = 0; c < MM_CT; ++c) {
                    f32x4_t t = xs;
#pragma unroll
                    for (int j = 0; j < 4; ++j) t = mfma_bf16_16x16x32(a0[j], b[c][j], t);
                    if (c > 0 || i > 0) correct(c == 0 ? MM_CT - 1 : c - 1, c == 0 ? i - 1 : i, tp, sp);
                    tp = t;
                    sp = scs[c];
                }
#pragma unroll
                for (int j = 0; j < 4; ++j) a0[j] = a1[j];
            }
            correct(MM_CT - 1, RB - 1, tp, sp);
            __builtin_amdgcn_s_setprio(0);
            return;
        }
        // 16- and 32-row blocks (split-K launches of up to 32 rows): one
        // column tile's operands at a time
        u32x4_t a[RB][4];
#pragma unroll
        for (int i = 0; i < RB; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) a[i][j] = frag(i, j);
        f32x4_t xs[RB];
#pragma unroll
        for (int i = 0; i < RB; ++i) {
            xs[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int j = 0; j < 4; ++j) xs[i] = mfma_bf16_16x16x32(a[i][j], m144, xs[i]);
        }
        // Software pipeline over (column tile, row block) units: the t chain
        // of unit k is issued before the correction of unit k-1, which does
        // not depend on it, so the correction VALU runs while the matrix core
        // works instead of waiting on each chain.
        f32x4_t tp = {0.f, 0.f, 0.f, 0.f};
        float sp = 0.f;
#pragma unroll
        for (int c = 0; c < MM_CT; ++c) {
            const uint32_t zb = zero_bytes(c);
            u32x4_t b[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) b[j] = w4_operand_z(R.w[c][j], zb);
            const float sc = f16_to_f32(static_cast<uint16_t>(R.sw[c][0] >> s_half));
#pragma unroll
            for (int i = 0; i < RB; ++i) {
                f32x4_t t = xs[i];
#pragma unroll
                for (int j = 0; j < 4; ++j) t = mfma_bf16_16x16x32(a[i][j], b[j], t);
                if (c > 0 || i > 0) correct(i == 0 ? c - 1 : c, i == 0 ? RB - 1 : i - 1, tp, sp);
                tp = t;
                sp = sc;
            }
        }
        correct(MM_CT - 1, RB - 1, tp, sp);
    };
    // all of this wave's loads have landed and every wave is done with the
    // buffer the next DMA overwrites.  Builtins, not inline asm: the
    // compiler's wait counting then knows every older load is complete and
    // does not add a drain-everything wait behind the next tile's loads
    // before this tile's registers are used.  0x0F70: vmcnt(0), expcnt and
    // lgkmcnt at their maxima (not waited on).
    auto rendezvous = [&]() {
        __builtin_amdgcn_s_waitcnt(0x0F70);
        __builtin_amdgcn_s_barrier();
    };

    uint8_t* const buf0 = mm_lds;
    uint8_t* const buf1 = mm_lds + A_BYTES;
    Regs ra, rb;
    issue(buf0, ra, 0);
    int kt = 0;
    for (; kt + 2 <= kh; kt += 2) {
        rendezvous();
        issue(buf1, rb, kt + 1);
        compute(buf0, ra, kt);
        rendezvous();
        issue(buf0, ra, kt + 2);  // clamped past the end: never used
        compute(buf1, rb, kt + 1);
    }
    if (kt < kh) {
        rendezvous();
        compute(buf0, ra, kt);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

    if constexpr (NK > 1) {
        // K parts 1.. hand their accumulators to part 0 through LDS, which
        // adds them in part order (deterministic): after the barrier every
        // wave's loads have landed and no wave reads the activation buffers
        // again.  (NK-1) * WN * RB * 4 KiB fits the 2 * A_BYTES of LDS.
        static_assert((NK - 1) * WN * RB * MM_CT * 64 * 16 <= 2 * A_BYTES, "reduction area");
        __syncthreads();
        f32x4_t* const red = reinterpret_cast<f32x4_t*>(mm_lds);
        constexpr int RS = RB * MM_CT * 64;  // f32x4 entries per wave's accumulators
        if (ks > 0) {
            f32x4_t* const mine = red + ((ks - 1) * WN + wn) * RS;
#pragma unroll
            for (int i = 0; i < RB; ++i)
#pragma unroll
                for (int c = 0; c < MM_CT; ++c) mine[(i * MM_CT + c) * 64 + lane] = acc[i][c];
        }
        __syncthreads();
        if (ks > 0) return;
#pragma unroll
        for (int q = 1; q < NK; ++q) {
            const f32x4_t* const part = red + ((q - 1) * WN + wn) * RS;
#pragma unroll
            for (int i = 0; i < RB; ++i)
#pragma unroll
                for (int c = 0; c < MM_CT; ++c) {
                    const f32x4_t h = part[(i * MM_CT + c) * 64 + lane];
#pragma unroll
                    for (int r = 0; r < 4; ++r) acc[i][c][r] += h[r];
                }
        }
    }

    // D element r of block (i, c): row 64*wm + 16*i + 4*(lane >> 4) + r,
    // column of tile (bx*WN*MM_CT + MM_CT*wn + c), lane & 15
    if constexpr (PK) {
        if (pk_slot >= 0) {
            // a K segment of a split tile: its partial sums in register
            // order (coalesced), every row of the tile
            f32x4_t* const W = reinterpret_cast<f32x4_t*>(p.ws) + static_cast<int64_t>(pk_slot) * kPkTileVecs +
                               wn * RB * MM_CT * 64 + lane;
#pragma unroll
            for (int i = 0; i < RB; ++i)
#pragma unroll
                for (int c = 0; c < MM_CT; ++c) W[(i * MM_CT + c) * 64] = acc[i][c];
            return;
        }
    }
    if constexpr (SK) {
        float* const W = p.ws + static_cast<int64_t>(bz) * p.M * p.N;
#pragma unroll
        for (int c = 0; c < MM_CT; ++c) {
            const int nt = bx * WN * MM_CT + wn * MM_CT + c;
            const int cn = nt * kW4TileN + col;
            if (nt >= p.Nt || cn >= p.N) continue;
#pragma unroll
            for (int i = 0; i < RB; ++i)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int row = m0 + wm * 64 + i * 16 + 4 * (lane >> 4) + r;
                    if (row < m_end) W[static_cast<int64_t>(row) * p.N + cn] = acc[i][c][r];
                }
        }
        return;
    }
    if constexpr (!F32) {
        store_bf16_block<SWI, RB>(p, static_cast<uint16_t*>(p.C) + (GR ? 0 : z * p.c_bs), acc,
                                  bx * WN * MM_CT + wn * MM_CT, m0 + wm * 64, m_end, lane);
        return;
    }
#pragma unroll
    for (int c = 0; c < MM_CT; ++c) {
        const int nt = bx * WN * MM_CT + wn * MM_CT + c;
        const int cn = nt * kW4TileN + col;
        if (nt >= p.Nt || cn >= p.N) continue;
#pragma unroll
        for (int i = 0; i < RB; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = m0 + wm * 64 + i * 16 + 4 * (lane >> 4) + r;
                // the reference's alpha / beta epilogue on fp32 C
                if (row < m_end) w4_store<true>(p, z * p.c_bs + static_cast<int64_t>(row) * p.N + cn, acc[i][c][r]);
            }
    }
}

// ---------------------------------------------------------------------------
// The 64 x 256 tile on the 32x32x16 MFMA (W32: layout 1, 64-row blocks;
// bf16 activations and output on plain, batched, grouped, SwiGLU, persistent
// grouped and split-K launches, and the fp32 interface (F32) on plain and
// split-K launches).  Same loads and LDS activation layout as mma_tile; what
// changes is the matrix work per K tile and wave (64 rows x 64 columns x
// 128 k):
//   - the products run as 32 MFMAs of 32x32x16 instead of 64 of 16x16x32.
//     Each MFMA issue takes the SIMD's issue port for about 8 cycles
//     whatever its size, so the 32-cycle form leaves room for ~6 VALU
//     instructions (the weight decode and group corrections) per MFMA where
//     the 16-cycle form leaves ~2: measured with register operands, two
//     waves per SIMD, chains of MFMAs with n VALU instructions between them:
//     16x16x32 17.6 / 27.1 / 35.2 cycles per MFMA at n = 0 / 4 / 6,
//     32x32x16 32.5 / 33.6 / 35.2 / 44.6 at n = 0 / 4 / 6 / 8.  So the
//     weight decode is interleaved with the MFMAs (two operands per k step)
//     instead of running as a phase of its own;
//   - the activation sums xs = -144 * sum_k x seeding the chains are made
//     once per workgroup: each wave sums the 16 rows its own DMAs carry
//     (16 * wave..; 4 MFMAs of 16x16x32 against the -144 operand) as soon as
//     its loads land, before the K tile's rendezvous, whose barrier hands
//     them to every wave through LDS; the 16x16 form has every wave sum all
//     64 rows;
//   - the wave's four column tiles nt0 + c form two 32-column blocks: block
//     cb holds tile cb in lanes with (lane >> 4) & 1 == 0 and tile cb + 2 in
//     the others, so with SwiGLU's interleaved gate / up tiles block 0 holds
//     the gates and block 1 the ups of the same two output tiles, in the
//     same lanes;
//   - MFMA q = (j, s) (k block j of 32, half s) takes in lane l the row /
//     column l & 31 of the block and the 8 k at 32 j + 16 s + 8 (l >> 5):
//     the weight dwords j of the prepacked tile's 16-byte chunk
//     (l & 15) + 16 (l >> 5) + 32 s, and the activations of LDS chunk
//     4 j + 2 s + (l >> 5) of row l & 31;
//   - D element e of block (ib, cb) in lane l: row 32 ib + 8 (e >> 2) +
//     4 (l >> 5) + (e & 3), column (lane & 15) of the lane's tile; the group
//     correction acc += s * t uses one scale per lane and block.
// F32: fp32 activations staged in LDS (512 bytes per row); each wave splits
// its own 16 rows into bf16 hi + lo in place before the rendezvous (with
// their sums), and every product runs twice, hi and lo, as in mma_tile's
// fp32 form; symmetric codes, fp32 scales, the alpha / beta epilogue.
// Everything else (zero point folded into the codes, xs seeding each chain,
// one correction per group, one K tile of loads in flight, unconditional
// clamped loads) is as in mma_tile.
template <bool GBIG, bool GR, bool SWI, bool PK, bool SK, bool F32>
__device__ __forceinline__ void mma_tile32(const W4Args& p, uint8_t* mm_lds, int bx, int by, int bz, int kb_in,
                                           int ke_in, int pk_slot) {
    static_assert(!SK || (!GR && !SWI && !PK), "split-K on plain launches only");
    static_assert(!F32 || (!GR && !SWI && !PK), "the fp32 interface: plain launches");
    constexpr int BPS = 4;
    constexpr int EA = F32 ? 4 : 2;               // activation bytes
    constexpr int RBYTES = kW4TileK * EA;         // LDS bytes per activation row
    constexpr int CPR = RBYTES / 16;              // 16-byte chunks per row
    constexpr int A_BYTES = 64 * RBYTES;          // one activation buffer
    constexpr int DMA = A_BYTES / 1024 / 4;       // activation DMAs per wave per K tile
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int col = lane & 15, h = lane >> 5, u = (lane >> 4) & 1;
    // K tiles [kb, ke): a split-K launch takes its split's range from bz,
    // which is the batch index otherwise
    const int kb = SK ? bz * p.kps : kb_in;
    const int ke = SK ? min(p.Kt, kb + p.kps) : ke_in;
    const int z = SK ? 0 : bz;
    int m0, m_end;
    const uint8_t* qw;
    const uint16_t* sc;
    const uint32_t* zs;
    if constexpr (GR) {
        int e;
        if (!resolve_group<64>(p, by, e, m0, m_end)) return;  // uniform per workgroup
        qw = p.qws[e];
        sc = static_cast<const uint16_t*>(p.scs[e]);
        zs = p.zss[e];
        if constexpr (PK) {
            qw = uniform_ptr(qw);
            sc = uniform_ptr(sc);
            zs = uniform_ptr(zs);
        }
    } else {
        m0 = by * 64;
        m_end = p.M;
        qw = p.qw + z * p.qw_bs;
        sc = static_cast<const uint16_t*>(p.scales) + z * p.s_bs;
        zs = p.zeros + z * p.z_bs;
    }
    const uint16_t* A = static_cast<const uint16_t*>(p.A) + (GR ? 0 : z * p.a_bs);
    const float* Af = static_cast<const float*>(p.A) + z * p.a_bs;
    const float* scf = static_cast<const float*>(p.scales) + z * p.s_bs;
    uint32_t a_voff[DMA];  // as in mma_tile: LDS row idx / CPR, slot idx % CPR
#pragma unroll
    for (int q = 0; q < DMA; ++q) {
        const int idx = (DMA * wave + q) * 64 + lane;
        const int r = idx / CPR, slot = idx % CPR;
        const int row = min(m0 + r, m_end - 1);
        a_voff[q] = (static_cast<uint32_t>(row - m0) * static_cast<uint32_t>(p.K) +
                     static_cast<uint32_t>((slot ^ (r & 15)) * (16 / EA))) * EA;
    }
    const uint32_t s_half = 16u * (col & 1);
    const int nt0 = min(bx * 4 * MM_CT + wave * MM_CT, p.Nt - 1);
    const int nt_left = p.Nt - nt0;
    auto extent = [](int64_t bytes) {
        return static_cast<int>(static_cast<uint32_t>(bytes < int64_t{0xFFFFFFFF} ? bytes : int64_t{0xFFFFFFFF}));
    };
    constexpr int ES = F32 ? 4 : 2;  // scale bytes
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(qw) + static_cast<int64_t>(nt0) * p.Kt * kW4TileBytes, 0,
        extent(static_cast<int64_t>(nt_left) * p.Kt * kW4TileBytes), kBufWord3);
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        F32 ? static_cast<void*>(const_cast<float*>(scf) + static_cast<int64_t>(nt0) * p.NG * 16)
            : static_cast<void*>(const_cast<uint16_t*>(sc) + static_cast<int64_t>(nt0) * p.NG * 16),
        0, extent(static_cast<int64_t>(nt_left) * p.NG * 16 * ES), kBufWord3);
    const __amdgpu_buffer_rsrc_t rz = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint32_t*>(zs) + static_cast<int64_t>(nt0) * p.NG8 * 16, 0,
        extent(F32 ? 0 : static_cast<int64_t>(nt_left) * p.NG8 * 16 * 4), kBufWord3);
    const __amdgpu_buffer_rsrc_t ra_ = __builtin_amdgcn_make_buffer_rsrc(
        F32 ? static_cast<void*>(const_cast<float*>(Af) + static_cast<int64_t>(m0) * p.K)
            : static_cast<void*>(const_cast<uint16_t*>(A) + static_cast<int64_t>(m0) * p.K),
        0, extent(static_cast<int64_t>(m_end - m0) * p.K * EA), kBufWord3);
    // the lane's tile in block cb (tiles past Nt re-read the last one)
    uint32_t w_voff[2], s_voff[2], z_voff[2];
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
        const uint32_t dt = static_cast<uint32_t>(min(nt0 + cb + 2 * u, p.Nt - 1) - nt0);
        w_voff[cb] = dt * static_cast<uint32_t>(p.Kt) * kW4TileBytes + col * 16 + 256 * h;
        s_voff[cb] = (dt * static_cast<uint32_t>(p.NG) * 16 + (F32 ? col : (col & ~1))) * ES;
        z_voff[cb] = (dt * static_cast<uint32_t>(p.NG8) * 16 + col) * 4;
    }

    struct Regs {
        u32x4_t w[2][2];  // block cb, half s
        uint32_t sw[2];
        uint32_t zw[2];
    };
    auto issue = [&](uint8_t* buf, Regs& R, int kt_in) {
        const int kt = min(kt_in + kb, p.Kt - 1);
#pragma unroll
        for (int q = 0; q < DMA; ++q)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(ra_, (LHQ_LDS_AS void*)(buf + (DMA * wave + q) * 1024), 16,
                                                     a_voff[q], kt * kW4TileK * EA, 0, 0);
        const int g = group_of_c<BPS, GBIG>(kt, 0, p.gmul);
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) {
            if constexpr (!F32) R.zw[cb] = __builtin_amdgcn_raw_buffer_load_b32(rz, z_voff[cb], (g >> 3) * 16 * 4, 0);
            R.sw[cb] = __builtin_amdgcn_raw_buffer_load_b32(rs, s_voff[cb], g * 16 * ES, 0);
#pragma unroll
            for (int s = 0; s < 2; ++s)
                R.w[cb][s] = __builtin_amdgcn_raw_buffer_load_b128(rw, w_voff[cb] + 512 * s, kt * kW4TileBytes, 0);
        }
    };

    f32x16_t acc[2][2];
#pragma unroll
    for (int ib = 0; ib < 2; ++ib)
#pragma unroll
        for (int cb = 0; cb < 2; ++cb)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[ib][cb][e] = 0.f;
    const u32x4_t m144 = {kM144Bf16x2, kM144Bf16x2, kM144Bf16x2, kM144Bf16x2};
    float* const xs_l = reinterpret_cast<float*>(mm_lds + 2 * A_BYTES);  // 64 rows' sums, two tiles
    // rows past the end read the last row; a tile with no live row (m0 >=
    // m_end) skips the arithmetic in every wave alike
    const bool live = m0 < m_end;
    // activation chunk of row `row` of the tile (LDS slot chunk ^ (row & 15));
    // fp32 rows after the split: chunk 8 j + 2 g holds the bf16 hi halves and
    // chunk 8 j + 2 g + 1 the lo halves of k = 32 j + 8 g .. + 7
    auto chunk_at = [&](const uint8_t* buf, int row, int c) {
        return const_cast<uint8_t*>(buf) + row * RBYTES + ((c ^ (row & 15)) * 16);
    };
    // The activation sums of a K tile, made before the rendezvous that
    // opens it: each wave's own DMAs carry its 16 rows (16 * wave..) of every
    // tile, so once its loads have landed the wave sums them (4 MFMAs against
    // the -144 operand, 16x16 D layout: rows 4 (lane >> 4) + r, every column
    // alike) and column 0 writes them to the tile's half of xs_l; the
    // rendezvous barrier then publishes them to every wave.  Two halves: a
    // tile's sums are written while the waves may still read the previous
    // tile's.  F32: the wave first splits its rows' fp32 activations into
    // bf16 hi + lo in place (each lane rewrites the two chunks it read) and
    // sums both halves (8 MFMAs).
    auto sums = [&](const uint8_t* buf, int kt_in) {
        // vmcnt(0) (expcnt and lgkmcnt at their maxima), as a builtin so the
        // compiler's wait counting knows the tile's loads are complete
        __builtin_amdgcn_s_waitcnt(0x0F70);
        asm volatile("" ::: "memory");
        if (!live) return;
        const int row = 16 * wave + col;
        f32x4_t xs = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if constexpr (F32) {
                uint8_t* const c_hi = chunk_at(buf, row, 8 * j + 2 * (lane >> 4));
                uint8_t* const c_lo = chunk_at(buf, row, 8 * j + 2 * (lane >> 4) + 1);
                const f32x4_t x0 = *reinterpret_cast<const f32x4_t*>(c_hi);
                const f32x4_t x1 = *reinterpret_cast<const f32x4_t*>(c_lo);
                const float v[8] = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
                u32x4_t ah, al;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const uint16_t h0 = f32_to_bf16(v[2 * e]), h1 = f32_to_bf16(v[2 * e + 1]);
                    ah[e] = static_cast<uint32_t>(h0) | (static_cast<uint32_t>(h1) << 16);
                    al[e] = pack_bf16x2(v[2 * e] - bf16_to_f32(h0), v[2 * e + 1] - bf16_to_f32(h1));
                }
                *reinterpret_cast<u32x4_t*>(c_hi) = ah;
                *reinterpret_cast<u32x4_t*>(c_lo) = al;
                xs = mfma_bf16_16x16x32(ah, m144, xs);
                xs = mfma_bf16_16x16x32(al, m144, xs);
            } else {
                xs = mfma_bf16_16x16x32(
                    *reinterpret_cast<const u32x4_t*>(chunk_at(buf, row, 4 * j + (lane >> 4))), m144, xs);
            }
        }
        if (col == 0) *reinterpret_cast<f32x4_t*>(xs_l + 64 * (kt_in & 1) + 16 * wave + 4 * (lane >> 4)) = xs;
    };
    auto compute = [&](const uint8_t* buf, const Regs& R, int kt_in) {
        if (!live) return;
        const int g = group_of_c<BPS, GBIG>(kb + kt_in, 0, p.gmul);
        const float* const xs_t = xs_l + 64 * (kt_in & 1);
        uint32_t zb[2];
        float scs[2];
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) {
            if constexpr (F32) {
                zb[cb] = 0x08080808u;  // symmetric codes: 16 - 8 in every byte
                scs[cb] = __uint_as_float(R.sw[cb]);
            } else {
                zb[cb] = __builtin_amdgcn_perm(0u, 16u - ((R.zw[cb] >> (4 * (g & 7))) & 15u), 0u);
                scs[cb] = f16_to_f32(static_cast<uint16_t>(R.sw[cb] >> s_half));
            }
        }
        // activation fragment(s) of row block ib for k step q (F32: the hi
        // and the lo halves), read ahead of their use
        constexpr int NH = F32 ? 2 : 1;  // fragments per row block and k step
        constexpr int RING = F32 ? 2 : 3;
        auto frag32 = [&](int q, int ib, int hh) {
            const int j = q >> 1, s = q & 1;
            const int c = F32 ? 8 * j + 2 * (2 * s + h) + hh : 4 * j + 2 * s + h;
            return *reinterpret_cast<const u32x4_t*>(chunk_at(buf, 32 * ib + (lane & 31), c));
        };
        u32x4_t af[RING][2][NH];
#pragma unroll
        for (int q = 0; q < RING - 1; ++q)
#pragma unroll
            for (int ib = 0; ib < 2; ++ib)
#pragma unroll
                for (int hh = 0; hh < NH; ++hh) af[q][ib][hh] = frag32(q, ib, hh);
        // four chains (ib, cb) seeded with their row block's sums; per k
        // step q the two weight operands are decoded just before their
        // MFMAs (the VALU work runs under the 32-cycle MFMAs), and the
        // activation fragments serve both column blocks
        f32x16_t t[2][2];
#pragma unroll
        for (int ib = 0; ib < 2; ++ib) {
#pragma unroll
            for (int i4 = 0; i4 < 4; ++i4) {
                const f32x4_t x = *reinterpret_cast<const f32x4_t*>(xs_t + 32 * ib + 8 * i4 + 4 * h);
#pragma unroll
                for (int r = 0; r < 4; ++r) t[ib][0][4 * i4 + r] = x[r];
            }
            t[ib][1] = t[ib][0];
        }
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const int j = q >> 1, s = q & 1;
            if (q + RING - 1 < 8)
#pragma unroll
                for (int ib = 0; ib < 2; ++ib)
#pragma unroll
                    for (int hh = 0; hh < NH; ++hh) af[(q + RING - 1) % RING][ib][hh] = frag32(q + RING - 1, ib, hh);
            u32x4_t bq[2];
#pragma unroll
            for (int cb = 0; cb < 2; ++cb) bq[cb] = w4_operand_z(R.w[cb][s][j], zb[cb]);
#pragma unroll
            for (int ib = 0; ib < 2; ++ib)
#pragma unroll
                for (int cb = 0; cb < 2; ++cb)
#pragma unroll
                    for (int hh = 0; hh < NH; ++hh)
                        t[ib][cb] = mfma_bf16_32x32x16(af[q % RING][ib][hh], bq[cb], t[ib][cb]);
            // keeps each k step's fragment reads ahead of their use
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int ib = 0; ib < 2; ++ib)
#pragma unroll
            for (int cb = 0; cb < 2; ++cb)
#pragma unroll
                for (int e = 0; e < 16; ++e) acc[ib][cb][e] = __builtin_fmaf(scs[cb], t[ib][cb][e], acc[ib][cb][e]);
    };
    // every wave's loads of the tile have landed (waited in sums), its sums
    // are in LDS, and every wave is done with the buffers the next loads
    // overwrite.  0xC07F: lgkmcnt(0), vmcnt and expcnt at their maxima; the
    // empty asm statements keep the compiler from moving LDS accesses across
    // the barrier
    auto rendezvous = [&]() {
        __builtin_amdgcn_s_waitcnt(0xC07F);
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
    };

    uint8_t* const buf0 = mm_lds;
    uint8_t* const buf1 = mm_lds + A_BYTES;
    const int kh = ke - kb;
    Regs ra, rb;
    issue(buf0, ra, 0);
    sums(buf0, 0);
    int kt = 0;
    for (; kt + 2 <= kh; kt += 2) {
        rendezvous();
        issue(buf1, rb, kt + 1);
        compute(buf0, ra, kt);
        sums(buf1, kt + 1);
        rendezvous();
        issue(buf0, ra, kt + 2);  // clamped past the end: never used
        compute(buf1, rb, kt + 1);
        if (kt + 2 < kh) sums(buf0, kt + 2);
    }
    if (kt < kh) {
        rendezvous();
        compute(buf0, ra, kt);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

    const int ntw = bx * 4 * MM_CT + wave * MM_CT;  // the wave's first column tile
    if constexpr (PK) {
        if (pk_slot >= 0) {
            // a K segment of a split tile: its partial sums in register
            // order (f32x4 (ib, cb, e >> 2) of each lane), every row
            f32x4_t* const W = reinterpret_cast<f32x4_t*>(p.ws) + static_cast<int64_t>(pk_slot) * kPkTileVecs +
                               wave * 16 * 64 + lane;
#pragma unroll
            for (int ib = 0; ib < 2; ++ib)
#pragma unroll
                for (int cb = 0; cb < 2; ++cb)
#pragma unroll
                    for (int i4 = 0; i4 < 4; ++i4)
                        W[((ib * 2 + cb) * 4 + i4) * 64] =
                            f32x4_t{acc[ib][cb][4 * i4], acc[ib][cb][4 * i4 + 1], acc[ib][cb][4 * i4 + 2],
                                    acc[ib][cb][4 * i4 + 3]};
            return;
        }
    }
    if constexpr (SK) {
        // the split's fp32 partial sums, ws[split][M][N]
        float* const W = p.ws + static_cast<int64_t>(bz) * p.M * p.N;
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) {
            const int nt = ntw + cb + 2 * u;
            const int cn = nt * kW4TileN + col;
            if (nt >= p.Nt || cn >= p.N) continue;
#pragma unroll
            for (int ib = 0; ib < 2; ++ib)
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int row = m0 + 32 * ib + 8 * (e >> 2) + 4 * h + (e & 3);
                    if (row < m_end) W[static_cast<int64_t>(row) * p.N + cn] = acc[ib][cb][e];
                }
        }
        return;
    }
    if constexpr (F32) {
        // the reference's alpha / beta epilogue on fp32 C
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) {
            const int nt = ntw + cb + 2 * u;
            const int cn = nt * kW4TileN + col;
            if (nt >= p.Nt || cn >= p.N) continue;
#pragma unroll
            for (int ib = 0; ib < 2; ++ib)
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int row = m0 + 32 * ib + 8 * (e >> 2) + 4 * h + (e & 3);
                    if (row < m_end)
                        w4_store<true>(p, z * p.c_bs + static_cast<int64_t>(row) * p.N + cn, acc[ib][cb][e]);
                }
        }
    } else {
        uint16_t* const C = static_cast<uint16_t*>(p.C) + (GR ? 0 : z * p.c_bs);
#pragma unroll
        for (int cb = 0; cb < (SWI ? 1 : 2); ++cb) {
            // SwiGLU: block 0 holds the gates, block 1 the ups of output tile
            // ntw / 2 + u
            const int nt = ntw + cb + 2 * u;
            const int cn = (SWI ? (ntw >> 1) + u : nt) * kW4TileN + col;
            if (nt >= p.Nt || cn >= p.N) continue;
#pragma unroll
            for (int ib = 0; ib < 2; ++ib)
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int row = m0 + 32 * ib + 8 * (e >> 2) + 4 * h + (e & 3);
                    if (row >= m_end) continue;
                    if constexpr (SWI)
                        C[static_cast<int64_t>(row) * p.N + cn] = f32_to_bf16(swiglu(acc[ib][0][e], acc[ib][1][e]));
                    else C[static_cast<int64_t>(row) * p.N + cn] = f32_to_bf16(acc[ib][cb][e]);
                }
        }
    }
}

// The tile kernel: one output tile per workgroup (grid: column groups x row
// tiles x batch or K splits), or with PK a persistent grouped launch.
//
// PK: gridDim.x workers (two per CU, all resident) share the T = X * Y
// tiles of a ragged grouped launch, X column groups of 256 and Y row tiles
// of 64 (counted from the device-side group table), tile t to worker t % P.
// Where the tiles do not fill one round (T < P) and leave at least a quarter
// of the workers idle, they are spread evenly along K instead (stream-K):
// their T * Kt K tiles form one range cut into Ps equal parts (at least 4 K
// tiles each), and each worker runs its part tile by tile -- a whole tile
// writes its output, a K segment of a tile writes fp32 partial sums to
// workspace slot (worker + tile), and w4_pk_fixup_kernel, next on the
// stream, adds each split tile's segments in K order (deterministic) and
// writes the output.  Measured on MI355X (us; one-workgroup-per-tile grid /
// persistent, whole tiles / persistent, split): config 4's grouped GEMM
// (1,120 tiles, K = 4096) 197.7 / 183.2 / 182.4, its SwiGLU gate / up launch
// (2,240 tiles) 349.9 / 342.2 / 347.8, its down projection (320 tiles, K =
// 14336) 199.9 / 195.8 / 185.4: with whole rounds to run, the split's
// partial sums and fixup cost what balancing the last round saves.
template <int BPS, bool GBIG, bool GR, bool SWI, int L, bool SK = false, int RB = 4, bool F32 = false, bool PK = false,
          bool W32 = false>
__global__ __launch_bounds__(L >= 3 ? 512 : 256, L == 3 ? 1 : 2) void w4_mma_kernel(W4Args p) {
    static_assert(!W32 || (BPS == 4 && L == 1 && RB == 4), "the 32x32x16 tile: 64 x 256 tiles");
    extern __shared__ __attribute__((aligned(1024))) uint8_t mm_lds[];
    auto tile = [&](int bx, int by, int bz, int k0, int k1, int slot) {
        if constexpr (W32) mma_tile32<GBIG, GR, SWI, PK, SK, F32>(p, mm_lds, bx, by, bz, k0, k1, slot);
        else mma_tile<BPS, GBIG, GR, SWI, L, SK, RB, F32, PK>(p, mm_lds, bx, by, bz, k0, k1, slot);
    };
    if constexpr (!PK) {
        tile(blockIdx.x, blockIdx.y, blockIdx.z, 0, p.Kt, -1);
    } else {
        const PkPlan pl = pk_plan(p, gridDim.x);
        const int w = blockIdx.x;
        // Tile coordinates pass through readfirstlane: they are uniform, and
        // the buffer descriptors built from them must sit in scalar
        // registers (a value the compiler cannot prove uniform puts every
        // buffer load of the K loop in a waterfall loop).
        auto uni = [](int64_t v) { return __builtin_amdgcn_readfirstlane(static_cast<int>(v)); };
        // one loop and one tile call site for both parts (whole tiles
        // t = w, w + P, ..., then this worker's stream-K range [lo, hi)), so
        // the tile is inlined once; a barrier between tiles: the next
        // tile's first DMA overwrites LDS that other waves may still read
        // for the last one
        int64_t t = w, lo = 0, hi = 0;
        bool split = false, first = true;
        while (true) {
            int64_t tt;
            int k0 = 0, k1 = p.Kt, slot = -1;
            if (!split) {
                if (t < pl.dp_tiles) {
                    tt = t;
                    t += gridDim.x;
                } else {
                    if (!pl.sk || w >= pl.Ps) break;
                    split = true;
                    lo = w * pl.I / pl.Ps;
                    hi = (w + 1) * pl.I / pl.Ps;
                    continue;
                }
            } else {
                if (lo >= hi) break;
                const int64_t tr = lo / p.Kt;  // split tile, counted from the first one
                k0 = static_cast<int>(lo - tr * p.Kt);
                k1 = static_cast<int>(min<int64_t>(p.Kt, k0 + (hi - lo)));
                tt = pl.dp_tiles + tr;
                slot = (k0 == 0 && k1 == p.Kt) ? -1 : static_cast<int>(w + tr);
                lo += k1 - k0;
            }
            if (!first) __syncthreads();
            first = false;
            tile(uni(tt % pl.X), uni(tt / pl.X), 0, uni(k0), uni(k1), uni(slot));
        }
    }
}

// The split tiles of a persistent grouped launch (w4_mma_kernel with PK,
// same W4Args, p.pk_workers = its grid): split tile tr's K segments are
// the partial sums of workers wa..wb in slots wa + tr .. wb + tr, added in
// that (K) order and written as the tile kernel writes a tile.  Workgroup
// 4 tr + qn takes column quarter qn of the tile (the 16 KiB a slot holds for
// wave qn): thread t holds lane t & 63 of column tile t >> 6 at row blocks
// 0..3, or with SWI the gate / up pair (2 (t >> 6 & 1), + 1) at row blocks
// 2 (t >> 7) and + 1; each segment's loads are issued four segments at a
// time before they are added.  W32 (slots written by mma_tile32): thread t
// holds lane t & 63 of blocks (ib, cb) at the D rows 8 i4 .. of the (ib, i4)
// pairs 2 (t >> 6) and + 1, cb = 0 and 1 of each (a gate / up pair with SWI).
template <bool SWI, bool W32 = false>
__global__ __launch_bounds__(256) void w4_pk_fixup_kernel(W4Args p) {
    const PkPlan pl = pk_plan(p, p.pk_workers);
    const int64_t tr = blockIdx.x >> 2;
    const int qn = blockIdx.x & 3;
    if (!pl.sk || tr >= pl.R) return;
    const int wa = pk_worker_of(tr * p.Kt, pl), wb = pk_worker_of((tr + 1) * p.Kt - 1, pl);
    if (wa == wb) return;  // one worker ran the whole tile
    const int64_t t = pl.dp_tiles + tr;
    int e, m0, m_end;
    if (!resolve_group<64>(p, static_cast<int>(t / pl.X), e, m0, m_end)) return;
    const int lane = threadIdx.x & 63, cp = threadIdx.x >> 6;
    // this thread's four slot entries: (row block, column tile) of the
    // 16x16 layout, or (ib, cb, i4) of the 32x32 one
    int ib[4], cb[4], ent[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        if constexpr (W32) {
            const int c = 2 * cp + (k >> 1);
            ib[k] = c >> 2;  // 32-row block
            cb[k] = k & 1;
            ent[k] = (ib[k] * 2 + cb[k]) * 4 + (c & 3);
        } else {
            ib[k] = SWI ? 2 * (cp >> 1) + (k >> 1) : k;
            cb[k] = SWI ? 2 * (cp & 1) + (k & 1) : cp;
            ent[k] = ib[k] * MM_CT + cb[k];
        }
    }
    const f32x4_t* const W = reinterpret_cast<const f32x4_t*>(p.ws) + qn * 4 * MM_CT * 64 + lane;
    f32x4_t acc[4];
    for (int w0 = wa; w0 <= wb; w0 += 4) {
        f32x4_t v[4][4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const f32x4_t* const S = W + (min(w0 + u, wb) + tr) * kPkTileVecs;
#pragma unroll
            for (int k = 0; k < 4; ++k) v[u][k] = S[ent[k] * 64];
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            if (w0 + u > wb) break;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                if (w0 + u == wa) acc[k] = v[u][k];
                else
#pragma unroll
                    for (int r = 0; r < 4; ++r) acc[k][r] += v[u][k][r];
            }
        }
    }
    uint16_t* const C = static_cast<uint16_t*>(p.C);
    const int nt0 = static_cast<int>(t % pl.X) * 4 * MM_CT + qn * MM_CT;
    const int col = lane & 15;
#pragma unroll
    for (int k = 0; k < 4; k += SWI ? 2 : 1) {
        int nt, cn, row0;
        if constexpr (W32) {
            const int u = (lane >> 4) & 1;
            nt = nt0 + cb[k] + 2 * u;
            cn = (SWI ? (nt0 >> 1) + u : nt) * kW4TileN + col;
            row0 = m0 + 32 * ib[k] + 8 * (ent[k] & 3) + 4 * (lane >> 5);
        } else {
            nt = nt0 + cb[k];
            cn = (SWI ? (nt >> 1) : nt) * kW4TileN + col;
            row0 = m0 + ib[k] * 16 + 4 * (lane >> 4);
        }
        if (nt >= p.Nt || cn >= p.N) continue;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = row0 + r;
            if (row >= m_end) continue;
            if constexpr (SWI) C[static_cast<int64_t>(row) * p.N + cn] = f32_to_bf16(swiglu(acc[k][r], acc[k + 1][r]));
            else C[static_cast<int64_t>(row) * p.N + cn] = f32_to_bf16(acc[k][r]);
        }
    }
}

// C[m][n] = bf16(sum over s < S of ws[s][m][n]), the splits added in order
// (deterministic); four consecutive elements per thread where 4 | MN.  The
// loads of eight splits are issued before any is added: a thread's loads
// are independent, so it waits for the memory system once per eight splits
// instead of once per split.
template <bool VEC>
__global__ void w4_splitk_reduce_kernel(const float* __restrict__ ws, uint16_t* __restrict__ C, int64_t mn, int S) {
    constexpr int U = 8;
    using V = std::conditional_t<VEC, f32x4_t, float>;
    const int64_t i = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) * (VEC ? 4 : 1);
    if (i >= mn) return;
    V v{};
    for (int s0 = 0; s0 < S; s0 += U) {
        V w[U];
#pragma unroll
        for (int u = 0; u < U; ++u)  // splits past S re-read the last one (not added)
            w[u] = *reinterpret_cast<const V*>(ws + static_cast<int64_t>(min(s0 + u, S - 1)) * mn + i);
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (s0 + u >= S) break;
            if (s0 + u == 0) v = w[u];
            else v += w[u];
        }
    }
    if constexpr (VEC) *reinterpret_cast<u32x2_t*>(C + i) = u32x2_t{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
    else C[i] = f32_to_bf16(v);
}

// The fp32 interface's split-K sum: C[i] = alpha * (sum over s < S of
// ws[s][i], in split order), then the reference's beta (beta == 0 never
// reads C, gemm_quant.cpp:12-21), as w4_store<true> does for an unsplit
// tile.  Four consecutive elements per thread where 4 | MN.
template <bool VEC>
__global__ void w4_splitk_reduce_f32_kernel(const float* __restrict__ ws, float* __restrict__ C, int64_t mn, int S,
                                            float alpha, float beta) {
    constexpr int U = 8;
    using V = std::conditional_t<VEC, f32x4_t, float>;
    const int64_t i = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) * (VEC ? 4 : 1);
    if (i >= mn) return;
    V v{};
    for (int s0 = 0; s0 < S; s0 += U) {
        V w[U];
#pragma unroll
        for (int u = 0; u < U; ++u)  // splits past S re-read the last one (not added)
            w[u] = *reinterpret_cast<const V*>(ws + static_cast<int64_t>(min(s0 + u, S - 1)) * mn + i);
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (s0 + u >= S) break;
            if (s0 + u == 0) v = w[u];
            else v += w[u];
        }
    }
    V out = alpha * v;
    if (beta != 0.0f) out = beta * *reinterpret_cast<const V*>(C + i) + out;
    *reinterpret_cast<V*>(C + i) = out;
}

// ---------------------------------------------------------------------------
// Launch selection
// ---------------------------------------------------------------------------

constexpr int kDecodeMaxLds = 64 * 1024;  // activation bytes a decode workgroup may stage
constexpr int kDecodeBigLds = 96 * 1024;   // ... when its workgroups fit one per CU
constexpr int kCuLds = 160 * 1024;         // LDS of one CU (gfx950)

// Lets a kernel take more than the default 64 KiB of dynamic LDS (set once
// per kernel, to the CU's whole LDS).
template <auto Kern>
void allow_cu_lds() {
    static const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(Kern),
                                                    hipFuncAttributeMaxDynamicSharedMemorySize, kCuLds);
    (void)e;
}

// Tuning knobs (tuning_knob: read only in a -DLHQ_TUNING_KNOBS build; unset
// or product build = heuristic):
//   LHQ_W4_I8=-1 disables the integer decode kernel (M == 1);
//   LHQ_W4_DECODE=-1 disables the bf16 decode kernel (plain and grouped);
//   LHQ_W4_DEC_T (1|2), LHQ_W4_DEC_NPW (4|8 tiles per wave per pass) and
//   LHQ_W4_DEC_S (waves per workgroup, 1..16) shape it;
//   LHQ_W4_GRB (rows per block, 1..16) forces the grouped decode kernel
//   with that row block on every grouped launch it can stage;
//   LHQ_W4_TILES (1|2), LHQ_W4_WAVES (1|2|4|8) shape the generic kernel;
//   LHQ_W4_MMA (0|1) and LHQ_W4_MMA_L (0..3) force the tile kernel off / on
//   and its layout.
int env_int(const char* name) { return tuning_knob(name, 0); }

template <bool F32A, bool ASYM, bool F32C, int T, int NPW, int MR>
void launch_decode_mr(const W4Args& a, dim3 grid, int S, int bps, size_t lds, hipStream_t s) {
    lds = std::max(lds, static_cast<size_t>(S) * T * MR * 64 * sizeof(float));  // the reduction reuses it
    switch (bps) {
        case 1:
            allow_cu_lds<&w4_decode_kernel<F32A, ASYM, F32C, T, NPW, 1, false, MR>>();
            w4_decode_kernel<F32A, ASYM, F32C, T, NPW, 1, false, MR><<<grid, 64 * S, lds, s>>>(a);
            break;
        case 2:
            allow_cu_lds<&w4_decode_kernel<F32A, ASYM, F32C, T, NPW, 2, false, MR>>();
            w4_decode_kernel<F32A, ASYM, F32C, T, NPW, 2, false, MR><<<grid, 64 * S, lds, s>>>(a);
            break;
        default:
            if (a.gmul) {
                allow_cu_lds<&w4_decode_kernel<F32A, ASYM, F32C, T, NPW, 4, true, MR>>();
                w4_decode_kernel<F32A, ASYM, F32C, T, NPW, 4, true, MR><<<grid, 64 * S, lds, s>>>(a);
            } else {
                allow_cu_lds<&w4_decode_kernel<F32A, ASYM, F32C, T, NPW, 4, false, MR>>();
                w4_decode_kernel<F32A, ASYM, F32C, T, NPW, 4, false, MR><<<grid, 64 * S, lds, s>>>(a);
            }
            break;
    }
}

// Grouped decode (bf16, fp16 scales, four K tiles per wave per pass).
template <int T, bool SWI>
void launch_decode_grouped(const W4Args& a, dim3 grid, int S, int bps, size_t lds, hipStream_t s) {
    lds = std::max(lds, static_cast<size_t>(S) * T * 4 * 64 * sizeof(float));  // the reduction reuses it
    switch (bps) {
        case 1:
            allow_cu_lds<&w4_decode_kernel<false, true, false, T, 4, 1, false, 4, true, SWI>>();
            w4_decode_kernel<false, true, false, T, 4, 1, false, 4, true, SWI><<<grid, 64 * S, lds, s>>>(a);
            break;
        case 2:
            allow_cu_lds<&w4_decode_kernel<false, true, false, T, 4, 2, false, 4, true, SWI>>();
            w4_decode_kernel<false, true, false, T, 4, 2, false, 4, true, SWI><<<grid, 64 * S, lds, s>>>(a);
            break;
        default:
            if (a.gmul) {
                allow_cu_lds<&w4_decode_kernel<false, true, false, T, 4, 4, true, 4, true, SWI>>();
                w4_decode_kernel<false, true, false, T, 4, 4, true, 4, true, SWI><<<grid, 64 * S, lds, s>>>(a);
            } else {
                allow_cu_lds<&w4_decode_kernel<false, true, false, T, 4, 4, false, 4, true, SWI>>();
                w4_decode_kernel<false, true, false, T, 4, 4, false, 4, true, SWI><<<grid, 64 * S, lds, s>>>(a);
            }
            break;
    }
}

template <bool F32A, bool ASYM, bool F32C, int T, int NPW>
void launch_decode_bps(const W4Args& a, dim3 grid, int S, int bps, size_t lds, hipStream_t s) {
    if (a.M == 1) launch_decode_mr<F32A, ASYM, F32C, T, NPW, 1>(a, grid, S, bps, lds, s);
    else launch_decode_mr<F32A, ASYM, F32C, T, NPW, 4>(a, grid, S, bps, lds, s);
}

template <bool F32A, bool ASYM, bool F32C, int T, int WAVES, bool GR, bool SWI>
void launch_gemv_bps(const W4Args& a, dim3 grid, int bps, hipStream_t s) {
    constexpr bool PIPE = !F32A && !GR && !SWI && T <= 2;
    switch (bps) {
        case 1: w4_gemv_kernel<F32A, ASYM, F32C, T, WAVES, 1, GR, SWI, PIPE><<<grid, 64 * WAVES, 0, s>>>(a); break;
        case 2: w4_gemv_kernel<F32A, ASYM, F32C, T, WAVES, 2, GR, SWI, PIPE><<<grid, 64 * WAVES, 0, s>>>(a); break;
        default: w4_gemv_kernel<F32A, ASYM, F32C, T, WAVES, 4, GR, SWI, PIPE><<<grid, 64 * WAVES, 0, s>>>(a); break;
    }
}

template <bool F32A, bool ASYM, bool F32C, int T, int NPW, int MR>
void launch_i8_mr(const W4Args& a, dim3 grid, int S, size_t lds, hipStream_t s) {
    lds = std::max(lds, static_cast<size_t>(S) * T * MR * 64 * sizeof(float));  // the reduction reuses it
    const bool big = lds > 64 * 1024;  // one workgroup per CU (the launch checks the grid)
    if (a.G == 64) {
        if (big) allow_cu_lds<&w4_decode_i8_kernel<F32A, ASYM, F32C, T, NPW, 2, false, MR>>();
        w4_decode_i8_kernel<F32A, ASYM, F32C, T, NPW, 2, false, MR><<<grid, 64 * S, lds, s>>>(a);
    } else if (a.gmul) {
        if (big) allow_cu_lds<&w4_decode_i8_kernel<F32A, ASYM, F32C, T, NPW, 4, true, MR>>();
        w4_decode_i8_kernel<F32A, ASYM, F32C, T, NPW, 4, true, MR><<<grid, 64 * S, lds, s>>>(a);
    } else {
        if (big) allow_cu_lds<&w4_decode_i8_kernel<F32A, ASYM, F32C, T, NPW, 4, false, MR>>();
        w4_decode_i8_kernel<F32A, ASYM, F32C, T, NPW, 4, false, MR><<<grid, 64 * S, lds, s>>>(a);
    }
}

// The grouped integer decode (one row per workgroup, G = 128).
template <int T, bool SWI>
void launch_i8_grouped(const W4Args& a, dim3 grid, int S, size_t lds, hipStream_t s) {
    lds = std::max(lds, static_cast<size_t>(S) * T * 64 * sizeof(float));  // the reduction reuses it
    w4_decode_i8_kernel<false, true, false, T, 4, 4, false, 1, true, SWI><<<grid, 64 * S, lds, s>>>(a);
}

template <bool F32A, bool ASYM, bool F32C, int T, bool GR, bool SWI = false>
void launch_gemv_waves(const W4Args& a, dim3 grid, int W, int bps, hipStream_t s) {
    switch (W) {
        case 1: launch_gemv_bps<F32A, ASYM, F32C, T, 1, GR, SWI>(a, grid, bps, s); break;
        case 2: launch_gemv_bps<F32A, ASYM, F32C, T, 2, GR, SWI>(a, grid, bps, s); break;
        case 4: launch_gemv_bps<F32A, ASYM, F32C, T, 4, GR, SWI>(a, grid, bps, s); break;
        default: launch_gemv_bps<F32A, ASYM, F32C, T, 8, GR, SWI>(a, grid, bps, s); break;
    }
}

// G >= 128 only (one scale group per K tile segment); smaller groups would
// need four times the activation-sum registers and spill.
// LDS of the 32x32x16 tile: two activation buffers and two tiles' row sums
// (bf16 activations; fp32 for the reference interface)
constexpr size_t kMma32Lds = 2 * 64 * kW4TileK * 2 + 2 * 64 * 4;
constexpr size_t kMma32F32Lds = 2 * 64 * kW4TileK * 4 + 2 * 64 * 4;
// the 32x32x16 form of the 64 x 256 bf16 tile (LHQ_W4_W32=0 in a tuning
// build keeps the 16x16x32 form)
bool use_w32() {
    static const bool on = tuning_knob("LHQ_W4_W32", 1) != 0;
    return on;
}
template <bool GBIG, bool GR, bool SWI, bool PK>
void launch_mma32(const W4Args& a, dim3 grid, hipStream_t s) {
    w4_mma_kernel<4, GBIG, GR, SWI, 1, false, 4, false, PK, true><<<grid, 256, kMma32Lds, s>>>(a);
}

template <bool GR, bool SWI, int L>
void launch_mma_l(const W4Args& a, unsigned row_tiles, unsigned batch, hipStream_t s) {
    constexpr size_t lds = 2 * ((L == 1) ? 64 : (L == 3) ? 256 : 128) * kW4TileK * 2;
    constexpr int threads = (L == 3) ? 512 : 256;
    const dim3 grid(ceil_div(a.Nt, ((L == 1) ? 4 : 2) * MM_CT), row_tiles, batch);
    if constexpr (L == 1) {
        if (use_w32()) {
            if (a.gmul) launch_mma32<true, GR, SWI, false>(a, grid, s);
            else launch_mma32<false, GR, SWI, false>(a, grid, s);
            return;
        }
    }
    if (a.gmul) {
        if constexpr (lds > 64 * 1024) allow_cu_lds<&w4_mma_kernel<4, true, GR, SWI, L>>();
        w4_mma_kernel<4, true, GR, SWI, L><<<grid, threads, lds, s>>>(a);
    } else {
        if constexpr (lds > 64 * 1024) allow_cu_lds<&w4_mma_kernel<4, false, GR, SWI, L>>();
        w4_mma_kernel<4, false, GR, SWI, L><<<grid, threads, lds, s>>>(a);
    }
}

int device_cus() {
    static const int cus = [] {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            return 0;
        return n;
    }();
    return cus;
}

// The tile kernel over `rows` rows (dense / batched), or over a ragged group
// table of `groups` groups holding `rows` rows in all: each group adds at
// most one partial row tile.  Layout 1 (64 x 256) unless its grid holds at
// most one workgroup per CU (two fit, by LDS and registers) and K is long:
// then layout 2 splits K for twice the workgroups, and where even its grid
// holds at most one workgroup per CU, layout 3 (eight waves, K in four
// parts, 128 KiB of LDS) doubles the waves again.  Measured on MI355X:
// 64 x 256 beat 128 x 128 on every shape tried (M=4096 K=8192 N=28672 2104
// vs 2215 us; config 4's grouped GEMM 196 vs 229 us).  Between one and two
// workgroups per CU layout 1 beats layout 2 (us, layout 1 vs 2): K=8192
// N=28672 M=192 118-120 vs 127-128, M=256 132 vs 144-146; M=320 K=4096
// N=14336 59 vs 66; config 4's grouped down projection (K=14336, N=4096,
// 384 workgroups) 195 vs 215.  At or below one per CU layout 2 wins: M=128
// K=8192 N=28672 83 vs 102, M=448 K=N=8192 74 vs 95.  LHQ_W4_MMA_L (0..3)
// forces a layout.
template <bool GR, bool SWI = false>
int launch_mma(const W4Args& a, int64_t rows, int groups, int batch, hipStream_t s, const char* who) {
    static const int env_l = tuning_knob("LHQ_W4_MMA_L", -1);
    int l = 1;
    const int64_t wgs1 = static_cast<int64_t>(ceil_div(a.Nt, 4 * MM_CT)) * (ceil_div64(rows, 64) + groups) * batch;
    if (wgs1 <= static_cast<int64_t>(device_cus()) && a.Kt >= 16) l = 2;
    if (2 * wgs1 <= static_cast<int64_t>(device_cus()) && a.Kt >= 32) l = 3;
    if (env_l >= 0 && env_l <= 3) l = env_l;
    const int64_t tiles = ceil_div64(rows, l == 0 ? 128 : 64) + groups;
    LHQ_SUPPORTED(tiles <= 65535, "%s: %lld row tiles exceed the grid limit", who, static_cast<long long>(tiles));
    const unsigned t = static_cast<unsigned>(tiles), b = static_cast<unsigned>(batch);
    if (l == 0) launch_mma_l<GR, SWI, 0>(a, t, b, s);
    else if (l == 1) launch_mma_l<GR, SWI, 1>(a, t, b, s);
    else if (l == 2) launch_mma_l<GR, SWI, 2>(a, t, b, s);
    else launch_mma_l<GR, SWI, 3>(a, t, b, s);
    return check_launch(who);
}

// The fp32 interface on the tile kernel (64 x 256 tiles, plain launches).
// The fp32 interface on the tile kernel: L = 1 with 64-row blocks (64 x 256
// tiles), or 16- / 32-row blocks (RB = 1, 2) with K split across the waves
// of the workgroup (L = 2: two K halves, 16/32 x 128 tiles, 4 waves; L = 3:
// four K quarters, 8 waves) for launches of up to 32 rows, which have few
// output tiles and take no workspace for a K split across workgroups.
template <int L, int RB>
int launch_mma_f32_rb(const W4Args& a, hipStream_t s, const char* who) {
    constexpr int NW = L >= 3 ? 8 : 4, NK = L == 2 ? 2 : L == 3 ? 4 : 1, WN = L == 1 ? 4 : 2;
    constexpr size_t a_bytes = static_cast<size_t>(NK) * 16 * RB * kW4TileK * 4;
    constexpr int UPW = 4 * RB / (NW / NK), PS = UPW >= 4 ? 1 : 4 / UPW;
    constexpr size_t lds = 2 * a_bytes + static_cast<size_t>(NK) * RB * PS * 64 * 16;  // tiles, partial sums
    const int64_t tiles = ceil_div64(a.M, 16 * RB);
    LHQ_SUPPORTED(tiles <= 65535, "%s: %lld row tiles exceed the grid limit", who, static_cast<long long>(tiles));
    const dim3 grid(ceil_div(a.Nt, WN * MM_CT), static_cast<unsigned>(tiles), 1);
    if constexpr (L == 1 && RB == 4) {
        if (use_w32()) {
            if (a.gmul) {
                allow_cu_lds<&w4_mma_kernel<4, true, false, false, 1, false, 4, true, false, true>>();
                w4_mma_kernel<4, true, false, false, 1, false, 4, true, false, true><<<grid, 256, kMma32F32Lds, s>>>(a);
            } else {
                allow_cu_lds<&w4_mma_kernel<4, false, false, false, 1, false, 4, true, false, true>>();
                w4_mma_kernel<4, false, false, false, 1, false, 4, true, false, true><<<grid, 256, kMma32F32Lds, s>>>(a);
            }
            return check_launch(who);
        }
    }
    if (a.gmul) {
        allow_cu_lds<&w4_mma_kernel<4, true, false, false, L, false, RB, true>>();
        w4_mma_kernel<4, true, false, false, L, false, RB, true><<<grid, 64 * NW, lds, s>>>(a);
    } else {
        allow_cu_lds<&w4_mma_kernel<4, false, false, false, L, false, RB, true>>();
        w4_mma_kernel<4, false, false, false, L, false, RB, true><<<grid, 64 * NW, lds, s>>>(a);
    }
    return check_launch(who);
}
int launch_mma_f32(const W4Args& a, hipStream_t s, const char* who) { return launch_mma_f32_rb<1, 4>(a, s, who); }

// fp32 interface at 2..47 rows: 0 = the ordinary choice (the 64-row tile
// where mma_applies, else the 16-row kernel), L = 2, 3 = the tile kernel
// with 16-row blocks (M <= 16) or 32-row blocks (ceil(M/32) row tiles),
// K split in halves / quarters across the waves of the workgroup.  Measured
// on MI355X at K = 8192 (us; ordinary / L = 2 / L = 3):
//   M = 4..16, N = 28672: 55-75 / 50 / 44-48; N <= 11008: the ordinary
//     kernel wins (M = 16, N = 8192: 27 / 46 / 40);
//   M = 24, 32: N = 57344 180 / 110 / 127-134; N = 28672 176 / 74 / 68-71;
//     N = 14336 (K = 4096) 38-43 / 37-38 / 32-34; N = 10240 48-53 / 67 / 58-61;
//   M = 40, 47: N = 57344 184-185 / 191 / 233; N = 28672 178-179 / 103-105 /
//     122-123; N = 14336 59-64 / 38-39 / 34; N = 10240 75-76 / 70 / 61-62.
// The 64-row tile at 17..47 rows and N >= 16384 walks all of K in one row
// tile of 112 workgroups (N = 28672), which the K-split layouts quadruple.
int f32_thin_layout(const W4Args& a, int M) {
    static const int env = tuning_knob("LHQ_W4_F32_THIN", -1);
    if (M < 2 || M > 47 || a.G < kW4TileK || a.K % kW4TileK != 0) return 0;
    if (env >= 0) return env;
    const int N = a.N;
    if (M <= 3) return 0;
    if (M <= 16) return N >= 16384 ? 3 : 0;
    if (M <= 32) return N >= 40000 ? 2 : N >= 12288 ? 3 : 0;
    return N >= 40000 ? 0 : N >= 16384 ? 2 : N >= 10240 ? 3 : 0;
}

bool mma_applies(const W4Args& a, int64_t rows, double rows_per_block) {
    static const int env = tuning_knob("LHQ_W4_MMA", -1);
    if (env == 0) return false;
    if (a.G < kW4TileK || a.K % kW4TileK != 0 || rows * a.K >= (int64_t{1} << 31)) return false;
    // The 16-row kernel re-reads the activation rows for every column tile
    // (rows * K * 2 bytes per 16 columns, from L2), the tile kernel once per
    // 256 columns through LDS; the tile kernel has fewer workgroups.
    // Measured on MI355X (us, 16-row kernel vs tile kernel):
    //   rows 16: K=8192 N=8192 20 vs 48, N=57344 74 vs 87;
    //   rows 32: N=8192 35 vs 48, N=28672 112 vs 55, N=57344 214 vs 90,
    //            K=28672 N=8192 114 vs 155;
    //   rows 48: N=8192 58 vs 50, N=28672 184 vs 57.
    // (columns counted as the launch sees them: 2 x I for the SwiGLU launch)
    return env == 1 || rows_per_block >= 48.0 || (rows_per_block > 16.0 && a.Nt * kW4TileN >= 16384);
}

// mblocks: 16-row blocks along grid.y (for a grouped launch, an upper bound
// on the sum over groups of ceil(rows_e / 16)).
// SWI (grouped bf16 only): the SwiGLU epilogue, two column tiles per
// workgroup on the generic kernel.
template <bool F32A, bool ASYM, bool F32C, bool GR = false, bool SWI = false>
int launch_w4(W4Args a, int batch, hipStream_t s, int mblocks = -1) {
    static const int env_dec = env_int("LHQ_W4_DECODE");
    static const int env_dt = env_int("LHQ_W4_DEC_T");
    static const int env_ds = env_int("LHQ_W4_DEC_S");
    static const int env_np = env_int("LHQ_W4_DEC_NPW");
    static const int env_t = env_int("LHQ_W4_TILES");
    static const int env_w = env_int("LHQ_W4_WAVES");
    static const int env_i8 = env_int("LHQ_W4_I8");
    if (mblocks < 0) mblocks = ceil_div(a.M, 16);
    const int bps = a.G >= 128 ? 4 : a.G / 32;

    // Integer-MFMA decode: one row (the kernel handles up to 4, but each
    // workgroup converts its rows' activations, and measured at M = 4 that
    // costs more than the bf16 kernel's decode: 11.9 vs 8.9 us at K=4096,
    // N=11008), G = 64 or a multiple of 128, digit planes and block table
    // within the LDS budget (LHQ_W4_I8=-1 disables).
    const size_t i8_lds = static_cast<size_t>(a.Kt) * (3 * kW4TileK + 16);
    // Up to 64 KiB of digit planes always; up to 96 KiB (K up to 31,488) with
    // two column tiles per wave where the workgroups then fit one per CU
    // (K=28672, N=8192: 256 workgroups)
    const bool i8_big = i8_lds > static_cast<size_t>(kDecodeMaxLds) && i8_lds <= static_cast<size_t>(kDecodeBigLds) &&
                        static_cast<int64_t>(ceil_div(a.Nt, 2)) * batch <= device_cus();
    if (!GR && mblocks == 1 && a.M == 1 && env_i8 >= 0 && (a.G == 64 || a.G % kW4TileK == 0) &&
        (i8_lds <= static_cast<size_t>(kDecodeMaxLds) || i8_big)) {
        // one column tile per wave: measured at K=8192, N=28672 (1792 column
        // tiles) 21.7 us against 22.4 us with two; with fp32 activations and
        // output 21.3 against 22.6 us (N=11008: 7.5 against 8.6 us), and
        // 26.3 us with eight waves per workgroup instead of four
        int T = i8_big ? 2 : 1;
        if (!i8_big && (env_dt == 1 || env_dt == 2)) T = env_dt;
        const int smax = (T == 1) ? 16 : 8;  // the kernel's launch bounds
        const int64_t cols = static_cast<int64_t>(ceil_div(a.Nt, T)) * batch;
        // and at most 32 K tiles per wave (K = 20480, N = 8192: 8 waves
        // 17.5 us against 18.3 with 4)
        int S = 4;
        while (S < smax && (cols * S < 2048 || a.Kt > 32 * S)) S *= 2;
        // two waves where K is at most 32 tiles and two still give 7 waves
        // per CU (us, 4 waves -> 2: K=4096, N=28672 12.8 -> 12.1; N=14336
        // 8.2 -> 7.8; K=2048, N=16384 6.3 -> 5.5; fewer columns lose:
        // K=4096, N=11008 6.8 -> 7.2, N=8192 5.5 -> 6.9)
        if (a.Kt <= 32 && cols * 2 >= int64_t{7} * device_cus()) S = 2;
        S = max(1, min(S, ceil_div(a.Kt, 4)));
        if (env_ds >= 1 && env_ds <= smax) S = env_ds;
        dim3 grid(ceil_div(a.Nt, T), 1, batch);
        if (T == 1) launch_i8_mr<F32A, ASYM, F32C, 1, 4, 1>(a, grid, S, i8_lds, s);
        else launch_i8_mr<F32A, ASYM, F32C, 2, 4, 1>(a, grid, S, i8_lds, s);
        return check_launch("w4a16 decode (int8 MFMA)");
    }

    const size_t dec_lds = static_cast<size_t>(min(a.M, 16)) * a.Kt * kW4TileK * (F32A ? 4 : 2);
    // Up to 64 KiB of staged activations always; up to 96 KiB when the
    // workgroups fit one per CU (measured: M=4, K=11008, N=4096 12.1 -> 9.1 us
    // against the generic kernel; at 128 KiB, or with more workgroups than
    // CUs, the generic kernel stays faster).
    const int cus = device_cus();
    const int64_t dec_wgs = static_cast<int64_t>(ceil_div(a.Nt, a.Nt >= 1024 ? 2 : 1)) * batch;
    const bool dec_fits = dec_lds <= static_cast<size_t>(kDecodeMaxLds) ||
                          (dec_lds <= static_cast<size_t>(kDecodeBigLds) && dec_wgs <= cus);
    if (!GR && mblocks == 1 && env_dec >= 0 && dec_fits) {
        // Measured on MI355X at K=8192, N=28672: two column tiles per wave
        // when there are many, four K tiles per wave per pass, four waves per
        // workgroup; small launches split K over more waves so the grid still
        // holds ~8 waves per CU.
        int T = (a.Nt >= 1024) ? 2 : 1;
        if (env_dt == 1 || env_dt == 2) T = env_dt;
        int npw = 4;
        if (env_np == 4 || env_np == 8) npw = env_np;
        const int smax = (T == 1) ? 16 : 8;  // the kernel's launch bounds
        const int64_t cols = static_cast<int64_t>(ceil_div(a.Nt, T)) * batch;
        // (and at most 32 K tiles per wave: K = 28672, N = 8192 23.1 us with
        // 8 waves against 24.1 with 4)
        int S = 4;
        while (S < smax && (cols * S < 2048 || a.Kt > 32 * S)) S *= 2;
        S = max(1, min(S, ceil_div(a.Kt, npw)));
        if (env_ds >= 1 && env_ds <= smax) S = env_ds;
        dim3 grid(ceil_div(a.Nt, T), 1, batch);
        if (T == 1) {
            if (npw == 4) launch_decode_bps<F32A, ASYM, F32C, 1, 4>(a, grid, S, bps, dec_lds, s);
            else launch_decode_bps<F32A, ASYM, F32C, 1, 8>(a, grid, S, bps, dec_lds, s);
        } else {
            if (npw == 4) launch_decode_bps<F32A, ASYM, F32C, 2, 4>(a, grid, S, bps, dec_lds, s);
            else launch_decode_bps<F32A, ASYM, F32C, 2, 8>(a, grid, S, bps, dec_lds, s);
        }
        return check_launch("w4a16 decode");
    }

    // Grouped decode: few rows per group (decode-time MoE), each group's
    // rows staged in LDS in blocks of rb rows.  Taken when the groups average
    // at most one row; rb = 4 (or as many rows as 64 KiB holds, if fewer)
    // keeps a workgroup's LDS small enough for three per CU at K = 4096
    // while a group of up to four rows still streams its weights once.
    if constexpr (GR && !F32A && ASYM && !F32C) {
        // At most max(2, groups / 2) rows in all: the integer decode, one row
        // per workgroup, each streaming its group's weights, so rows * (one
        // group's weights) are read however the rows spread.  The bf16 form
        // below streams a group's weights once per block of rb rows.
        // Measured, 8 experts of Mixtral shapes, gate/up + down: 1 token
        // (2 rows) 23.1 + 11.9 us against 27.4 + 15.0; 2 tokens 42.7 + 21.9
        // against 48.3 + 26.1; 4 tokens (8 rows) 76.9 + 39.9 against
        // 72.5 + 44.9.
        static const int env_gi8 = env_int("LHQ_W4_GI8");
        static const int env_gmax = tuning_knob("LHQ_W4_GI8_MMAX", 0);
        const int gi8_mmax = (env_gmax >= 1) ? env_gmax : std::max(2, a.num_groups / 2);
        const size_t gi8_lds = static_cast<size_t>(a.Kt) * (3 * kW4TileK + 16);
        if (env_gi8 >= 0 && env_dec >= 0 && a.M <= gi8_mmax && a.G == kW4TileK && gi8_lds <= static_cast<size_t>(kDecodeMaxLds)) {
            static const int env_gt = tuning_knob("LHQ_W4_GI8_T", 0);
            const int T = (SWI || (env_gt == 0 ? a.Nt >= 1024 : env_gt == 2)) ? 2 : 1;
            const int smax = (T == 1) ? 16 : 8;
            const int64_t cols = static_cast<int64_t>(ceil_div(a.Nt, T)) * a.M;
            // at most 16 K tiles per wave, as the bf16 grouped decode, from
            // 2 waves (gate/up at one token, K = 4096: 21.0-21.5 us with 2
            // waves, 22.4 with 4)
            int S = 2;
            while (S < smax && (cols * S < 2048 || a.Kt > 16 * S)) S *= 2;
            S = max(1, min(S, ceil_div(a.Kt, 4)));
            if (env_ds >= 1 && env_ds <= smax) S = env_ds;
            // one-row blocks: exactly a.M of them, however the rows spread
            dim3 grid(ceil_div(a.Nt, T), static_cast<unsigned>(a.M), 1);
            if constexpr (SWI) launch_i8_grouped<2, true>(a, grid, S, gi8_lds, s);
            else if (T == 1) launch_i8_grouped<1, false>(a, grid, S, gi8_lds, s);
            else launch_i8_grouped<2, false>(a, grid, S, gi8_lds, s);
            return check_launch("w4a16 grouped decode (int8 MFMA)");
        }
        static const int env_grb = env_int("LHQ_W4_GRB");
        const int64_t row_bytes = static_cast<int64_t>(a.Kt) * kW4TileK * 2;
        const int rb_max = static_cast<int>(std::min<int64_t>(16, kDecodeMaxLds / row_bytes));
        const int rb = (env_grb >= 1) ? std::min(env_grb, rb_max) : std::min(4, rb_max);
        if (env_dec >= 0 && rb >= 1 && (a.M <= a.num_groups || env_grb >= 1)) {
            a.group_rb = rb;
            const int T = (SWI || a.Nt >= 1024) ? 2 : 1;
            // at most min(groups, rows) groups hold rows: sum_e ceil(rows_e / rb)
            // <= ceil(rows / rb) + min(groups, rows)
            const int64_t blocks = ceil_div64(a.M, rb) + std::min(a.num_groups, a.M);
            const int smax = (T == 1) ? 16 : 8;  // the kernel's launch bounds
            const int64_t cols = static_cast<int64_t>(ceil_div(a.Nt, T)) * blocks;
            // as the ungrouped decode, and at most 16 K tiles per wave
            // (measured at K=14336, N=4096, 2 rows over 8 groups: 16.8 us
            // with 4 waves, 14.2 with 8)
            int S = 4;
            while (S < smax && (cols * S < 2048 || a.Kt > 16 * S)) S *= 2;
            S = max(1, min(S, ceil_div(a.Kt, 4)));
            if (env_ds >= 1 && env_ds <= smax) S = env_ds;
            if (blocks <= 65535) {
                const size_t lds = static_cast<size_t>(std::min(a.M, rb)) * row_bytes;
                dim3 grid(ceil_div(a.Nt, T), static_cast<unsigned>(blocks), 1);
                if constexpr (SWI) launch_decode_grouped<2, true>(a, grid, S, bps, lds, s);
                else if (T == 1) launch_decode_grouped<1, false>(a, grid, S, bps, lds, s);
                else launch_decode_grouped<2, false>(a, grid, S, bps, lds, s);
                return check_launch("w4a16 grouped decode");
            }
        }
    }

    // A grouped launch counts the row blocks that can hold rows, ceil(rows
    // / 16) plus one partial block per group that has rows, not its grid
    // bound (with a few tokens over many experts most of the grid exits at
    // once).
    const int64_t live_blocks = GR ? std::min<int64_t>(mblocks, ceil_div(a.M, 16) + std::min(a.num_groups, a.M))
                                   : mblocks;
    // Column tiles per workgroup: the most (4, 2 or 1) that leave 256
    // workgroups, or 8 where 384 remain (MoE down projection at 128 tokens
    // 146.9 -> 136.6 us, M=8 K=8192 N=57344 58.5 -> 51.9 us; at 320, 16
    // tokens' down projection, it lost: 52.3 -> 59.1 us).  The 16-row kernel is bound by the CU's vector memory path
    // (each activation load touches its 16 rows' cache lines), and a
    // workgroup shares those loads across its column tiles; below 256
    // workgroups the lost parallelism costs more.  Four tiles are bf16
    // only, and the SwiGLU form takes them only at 8 rows per row block (with
    // 2-3, 8-16 tokens over 8 experts, its activation loads are few).
    // Measured on MI355X (us, T = 1 / 2 / 4): M=8 K=28672 N=8192 46.4 / 42.8 /
    // 61.3; M=32 K=8192 N=8192 35.9 / 23.5 / 21.3; M=16 K=11008 N=4096 13.9 /
    // 19.7 / 27.5; M=8 K=8192 N=57344 80.5 / 61.4 / 58.5; MoE down projection
    // at 64 tokens (K=14336, N=4096) 144 / 108 / 95.
    const bool bf16a = !F32A && ASYM && !F32C;
    auto wgs_t = [&](int t) { return static_cast<int64_t>(ceil_div(a.Nt, t)) * live_blocks * batch; };
    const bool rows8 = !SWI || a.M >= 8 * live_blocks;
    int T = 1;
    if (bf16a && wgs_t(8) >= 384 && rows8) T = 8;
    else if (bf16a && wgs_t(4) >= 256 && rows8) T = 4;
    else if (wgs_t(2) >= 256) T = 2;
    if (env_t == 1 || env_t == 2) T = env_t;
    if ((env_t == 4 || env_t == 8) && bf16a) T = env_t;
    if constexpr (SWI) T = (T >= 4) ? T : 2;
    // Enough waves to cover 256 CUs several times over, but at least four
    // K tiles per wave so each wave keeps loads in flight, sized by the live
    // row blocks (measured at 2 rows over 8 experts, K=14336, N=4096: sized
    // by the grid bound, 2 waves walking 56 K tiles each took 46.6 us).
    const int64_t wgs = static_cast<int64_t>(ceil_div(a.Nt, T)) * live_blocks * batch;
    // Also split K further while a wave would walk more than 16 K tiles:
    // the kernel does not prefetch across its K loop, so a long walk by a
    // few waves waits out the memory latency once per tile.
    int W = 2;
    while (W < 8 && (wgs * W < 4096 || a.Kt > 16 * W) && a.Kt / (2 * W) >= 4) W *= 2;
    if (env_w == 1 || env_w == 2 || env_w == 4 || env_w == 8) W = env_w;
    dim3 grid(ceil_div(a.Nt, T), mblocks, batch);
    if constexpr (SWI) {
        if (T == 8) launch_gemv_waves<F32A, ASYM, F32C, 8, GR, true>(a, grid, W, bps, s);
        else if (T == 4) launch_gemv_waves<F32A, ASYM, F32C, 4, GR, true>(a, grid, W, bps, s);
        else launch_gemv_waves<F32A, ASYM, F32C, 2, GR, true>(a, grid, W, bps, s);
    }
    else if (T == 1) launch_gemv_waves<F32A, ASYM, F32C, 1, GR>(a, grid, W, bps, s);
    else if constexpr (!F32A && ASYM && !F32C) {
        if (T == 8) launch_gemv_waves<F32A, ASYM, F32C, 8, GR>(a, grid, W, bps, s);
        else if (T == 4) launch_gemv_waves<F32A, ASYM, F32C, 4, GR>(a, grid, W, bps, s);
        else launch_gemv_waves<F32A, ASYM, F32C, 2, GR>(a, grid, W, bps, s);
    } else {
        launch_gemv_waves<F32A, ASYM, F32C, 2, GR>(a, grid, W, bps, s);
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
    // G > 128 is a multiple of 128 (check_w4_shape): tile kt is in group
    // kt / (G/128), computed as __umulhi(kt, ceil(2^32 / (G/128)))
    a.gmul = (G > kW4TileK) ? static_cast<uint32_t>(((1ull << 32) + G / kW4TileK - 1) / (G / kW4TileK)) : 0u;
    a.alpha = alpha; a.beta = beta;
    return a;
}

// Workers of a persistent grouped launch: two 64 x 256 tile workgroups per
// CU (the tile kernel's occupancy), all resident at once.
int pk_workers() { return 2 * std::max(device_cus(), 1); }

// Tiles of a grouped launch at most: X (ceil(rows / 64) + live groups).
int64_t pk_max_tiles(const W4Args& a) {
    const int64_t X = ceil_div(a.Nt, 4 * MM_CT);
    return X * (ceil_div64(a.row_capacity, 64) + std::min(a.num_groups, a.row_capacity));
}

// The persistent grouped launch (w4_mma_kernel with PK) and its fixup, with
// ws_slots 64 KiB partial-sum slots at ws.
template <bool SWI>
int launch_mma_pk(W4Args a, void* ws, int64_t ws_slots, hipStream_t s, const char* who) {
    constexpr size_t lds = 2 * 64 * kW4TileK * 2;
    const int P = pk_workers();
    // The split needs T <= 3P/4; T is counted on the device, but its bound
    // from row_capacity tells when no table can give a split, and then no
    // slot is offered and the fixup kernel (~4 us for nothing) not launched.
    const int64_t t_max = pk_max_tiles(a);
    const bool may_split = 4 * t_max <= 3 * static_cast<int64_t>(P);
    a.ws = static_cast<float*>(ws);
    a.pk_slots = may_split ? ws_slots : 0;
    a.pk_workers = P;
    const bool w32 = use_w32();
    if (w32) {
        if (a.gmul) launch_mma32<true, true, SWI, true>(a, dim3(P), s);
        else launch_mma32<false, true, SWI, true>(a, dim3(P), s);
    } else if (a.gmul) {
        w4_mma_kernel<4, true, true, SWI, 1, false, 4, false, true><<<P, 256, lds, s>>>(a);
    } else {
        w4_mma_kernel<4, false, true, SWI, 1, false, 4, false, true><<<P, 256, lds, s>>>(a);
    }
    if (int st = check_launch(who)) return st;
    if (!may_split) return LHQ_OK;
    // four workgroups per split tile (every tile when the split runs)
    const unsigned fix_wgs = static_cast<unsigned>(4 * std::max<int64_t>(1, t_max));
    if (w32) w4_pk_fixup_kernel<SWI, true><<<fix_wgs, 256, 0, s>>>(a);
    else w4_pk_fixup_kernel<SWI><<<fix_wgs, 256, 0, s>>>(a);
    return check_launch(who);
}

// The grouped launch's arguments (SWI: N is the intermediate width I, the
// weights hold 2 ceil(I/16) interleaved gate / up column tiles).
template <bool SWI>
W4Args grouped_args(const uint16_t* A, const int32_t* offsets, const uint8_t* const* qweights,
                    const uint16_t* const* scales, const uint32_t* const* zeros, uint16_t* C, int num_groups,
                    int row_capacity, int N, int K, int G) {
    W4Args a = make_args(A, nullptr, nullptr, nullptr, C, row_capacity, N, K, G, 1.0f, 0.0f);
    if constexpr (SWI) a.Nt = 2 * ceil_div(N, kW4TileN);
    a.offsets = offsets;
    a.qws = qweights;
    a.scs = reinterpret_cast<const void* const*>(scales);
    a.zss = zeros;
    a.num_groups = num_groups;
    a.row_capacity = row_capacity;
    return a;
}
bool grouped_uses_tiles(const W4Args& a) {
    return mma_applies(a, a.row_capacity, static_cast<double>(a.row_capacity) / a.num_groups);
}

// Partial-sum slots a persistent grouped launch can use: a split of R = T
// <= 3P/4 tiles over Ps <= P workers touches slots up to (Ps - 1) + (R - 1);
// none where the tile bound rules the split out.
int64_t grouped_pk_slots(const W4Args& a) {
    const int64_t P = pk_workers(), t_max = pk_max_tiles(a);
    return 4 * t_max <= 3 * P ? P + t_max - 1 : 0;
}

// Ragged grouped launch (device-side group table); ws / ws_bytes: the
// persistent launch's workspace (none: one workgroup per tile).
template <bool SWI>
int grouped_w4(const char* who, const uint16_t* A, const int32_t* offsets, const uint8_t* const* qweights,
               const uint16_t* const* scales, const uint32_t* const* zeros, uint16_t* C, int num_groups,
               int row_capacity, int N, int K, int G, void* ws, int64_t ws_bytes, void* stream) {
    if (int st = check_w4_shape(who, row_capacity, N, K, G)) return st;
    LHQ_REQUIRE(num_groups >= 0, "%s: negative num_groups", who);
    LHQ_REQUIRE(offsets && qweights && scales && zeros && C && (A || row_capacity == 0), "%s: null pointer", who);
    LHQ_REQUIRE(ws_bytes >= 0, "%s: negative workspace_bytes", who);
    if (num_groups == 0 || row_capacity == 0) return LHQ_OK;
    const W4Args a =
        grouped_args<SWI>(A, offsets, qweights, scales, zeros, C, num_groups, row_capacity, N, K, G);
    // at most min(num_groups, row_capacity) groups hold rows, so
    // sum_e ceil(rows_e / B) <= ceil(row_capacity / B) + live_groups for row blocks of B
    const int live_groups = std::min(num_groups, row_capacity);
    if (grouped_uses_tiles(a)) {
        if (ws && ws_bytes >= kPkSlotBytes) {
            LHQ_REQUIRE((reinterpret_cast<uintptr_t>(ws) & 15) == 0, "%s: workspace not 16-byte aligned", who);
            return launch_mma_pk<SWI>(a, ws, ws_bytes / kPkSlotBytes, as_stream(stream), who);
        }
        return launch_mma<true, SWI>(a, row_capacity, live_groups, 1, as_stream(stream), who);
    }
    const int64_t mblocks = ceil_div64(row_capacity, 16) + live_groups;
    LHQ_SUPPORTED(mblocks <= 65535, "%s: %lld row blocks exceed the grid limit", who, static_cast<long long>(mblocks));
    return launch_w4<false, true, false, true, SWI>(a, 1, as_stream(stream), static_cast<int>(mblocks));
}

// ---------------------------------------------------------------------------
// Thin grids: the tile kernel with K split across workgroups.
//
// At 2..64 rows the tile kernel's grid has ceil(N / 256) column groups --
// 32 for N = 8192, far short of 256 CUs -- and each workgroup walks all of
// K.  A plan here spreads K over S workgroups per output tile: each writes
// fp32 partial sums of its K range to a workspace [S][M][N], and
// w4_splitk_reduce_kernel adds them in split order into the bf16 output
// (deterministic, whatever the schedule).  Up to 16 or 32 rows use 16- or
// 32-row blocks (RB = 1, 2), so they do not pay for the MFMAs of 64.
// 2..16 rows run 16 x 128 tiles with K in two halves inside the workgroup
// (L = 2).  Measured on MI355X (us, ordinary launch / split), (K, N) at 16
// rows: (28672, 8192) 40.4 / 28.9, (8192, 10240) 21.4 / 17.5, (16384, 4096)
// 19.4 / 15.3, (8192, 28672) 34.9 / 31.7, but (8192, 8192) 13.2 / 14.3; at
// 12 rows (4096, 11008) 11.5 / 12.5; at 8 rows (28672, 8192) 33.4 / 29.3;
// at 2 rows (28672, 8192) 28.7 / 29.3.
// ---------------------------------------------------------------------------
struct TilePlan {
    bool split = false;  // false: the entry point's ordinary launch
    int L = 1;           // tile kernel layout
    int RB = 4;          // 16-row blocks per wave
    int S = 1;           // K splits
    int kps = 0;         // K tiles per split
    int64_t ws_bytes = 0;
};

constexpr int kSplitMinKt = 4;  // K tiles per split at least
constexpr int kThinMaxRows = 512;  // rows a split launch takes at most

// Above 64 rows the split count is capped so that the partial sums (S M N
// fp32, written and read back) are no larger than the weights' codes
// (K N / 2 bytes), i.e. 8 S M <= K: measured (us, unsplit / split, bf16)
// M = 128, K = N = 8192 (8 splits) 50.4 / 33.6; M = 256, K = 8192, N =
// 4096 (4) 50.8 / 33.0; M = 128, K = 28672, N = 8192 (4) 155 / 83.6; but
// M = 512, K = N = 4096 (4 splits, partial sums four times the codes)
// 32.2 / 33.0.
int cap_split_rows(const W4Args& a, int S, int env_s) {
    if (a.M <= 64 || env_s >= 1) return S;
    return static_cast<int>(std::min<int64_t>(S, a.K / (int64_t{8} * a.M)));
}

// ws_cap: the workspace bytes available (-1: as much as the plan wants).
// A split applies to 2..64 rows where the tile kernel runs (G >= 128) (and
// to 65..512 rows of 64-row blocks whose grid fills at most half the CUs,
// cap_split_rows), and
// where the ordinary launch would be the tile kernel or the weights are
// large enough (K * N >= 32 Mi) that the 16-row kernel loses to it: measured
// at M = 32, (K, N) = (4096, 4096) 9.2 us on the 16-row kernel against 12.5
// split, but (4096, 11008) 19.9 against 15.6 and (8192, 8192) 22.0 against
// 17.0.  S brings the grid to about one workgroup per CU, with at least 4 K
// tiles per split (M = 64, K = N = 8192: 48.5 us unsplit, 24.5 with 8
// splits, 27.3 with 16).  At K < 16384 the plain 64 x 256 layout with a K
// split matched or beat the in-workgroup split layouts with a K split (M =
// 64, K = N = 8192: 24.3 us against 24.3 and 25.1; M = 32, K = 8192, N =
// 57344: 69.5 against 97.2 and 112.2); from K = 16384 on, K halves inside
// the workgroup win (below).
TilePlan plan_thin(const W4Args& a, int64_t ws_cap) {
    TilePlan t;
    // (read on every call in a tuning build, so one process can sweep them)
    const int env_thin = tuning_knob("LHQ_W4_THIN", -1);   // 0: never split
    const int env_s = tuning_knob("LHQ_W4_THIN_S", 0);     // force the split count
    const int env_l = tuning_knob("LHQ_W4_THIN_L", 0);     // force the layout (1..4)
    // (more than 64 rows: 64-row blocks, split only where the unsplit grid
    // fills at most half the CUs; the rule below)
    if (env_thin == 0 || a.M < 2 || a.M > tuning_knob("LHQ_W4_THIN_MMAX", kThinMaxRows)) return t;
    if (a.G < kW4TileK || a.K % kW4TileK != 0 || static_cast<int64_t>(a.M) * a.K >= (int64_t{1} << 31)) return t;
    const bool tile = mma_applies(a, a.M, a.M);
    if (!tile && static_cast<int64_t>(a.K) * a.N < (int64_t{32} << 20)) return t;
    t.RB = a.M <= 16 ? 1 : a.M <= 32 ? 2 : 4;
    // 2..16 rows: 16 x 128 tiles with K in two halves inside the workgroup
    // (L = 2), which reach the same grid as 16 x 256 tiles with half the
    // splits, so half the partial-sum traffic
    if (t.RB == 1) t.L = 2;
    if (env_l >= 1 && env_l <= 4) t.L = env_l;
    const int64_t wgs =
        static_cast<int64_t>(ceil_div(a.Nt, (t.L == 1 || t.L == 4 ? 4 : 2) * MM_CT)) * ceil_div(a.M, 16 * t.RB);
    const int cus = std::max(device_cus(), 1);
    // 64-row blocks with more than half a CU's worth of column groups: the
    // ordinary launch (64 x 128 tiles with K halves in the workgroup) does
    // as well or better (M = 64, K = 8192, N = 57344: 88.2-89.9 us against
    // 92.1-92.4 with 2 splits, 104.9-107.1 with 3)
    if (env_s == 0 && env_l == 0 && tile && t.RB == 4 && 2 * wgs > cus) return t;
    // about one workgroup per CU, and for 16-row blocks at most 28 K tiles
    // per split (16 rows, K = 28672: 8 splits 30.8 us, 6 34.3, 4 37.4)
    const int64_t fill = ceil_div64(cus, wgs);
    const int64_t want = (t.RB == 1) ? std::max<int64_t>(fill, ceil_div(a.Kt, 28)) : fill;
    int S = static_cast<int>(std::min<int64_t>(want, std::max(1, a.Kt / kSplitMinKt)));
    // 2..16 rows: the split costs about the same at any row count, while
    // the ordinary launch (decode or 16-row kernel) grows with the rows and
    // with K per wave, and loses most where its workgroups need more than
    // one round of the CUs (N > 8192).  So a split takes a grid at most half
    // full unsplit, three splits or more, and either K >= 16384 (from 4
    // rows; up to 8 rows with N >= 8192) or, from 9 rows, K >= 8192 with
    // N > 8192.
    if (env_s == 0 && t.RB == 1) {
        const bool long_k = a.K >= 16384 && a.M >= 4 && (a.M >= 9 || a.N >= 8192);
        const bool wide = a.M >= 9 && a.K >= 8192 && a.N > 8192;
        if (fill < 2 || S < 3 || !(long_k || wide)) return t;
    }
    // 64-row blocks: about two workgroups per CU, so the two-phase K loop
    // has a second workgroup's wave on every SIMD to alternate with -- by
    // splitting further (at least 8 K tiles per split, and at most two
    // workgroups per CU: a third round costs more than it saves), unless K
    // is long enough for K halves inside the workgroup at one split per CU
    // (the layout switch below).  Measured (us, M = 64, one split per CU or
    // unsplit / this rule): K = 8192, N = 28672 61.1-62.4 / 51.9-52.7 (4
    // splits; 5 splits, 560 workgroups, 63.4-65.3); N = 14336 34.6-35.2 /
    // 33.0-33.4 (8); K = 4096, N = 28672 34.4-34.7 / 32.0-33.1 (4); K =
    // 28672, N = 28672 179.9-181.1 / 148.3-150.0 (4); 48 rows, K = 8192,
    // N = 28672 53.3-53.7 / 46.4-48.4 (4).  Where one workgroup per CU
    // leaves at most 12 K tiles per split, the grid stays at one per CU
    // (at most one round, none of the CUs running two): M = 64, K = 8192,
    // N = 10240 (40 column groups) 28.4-29.9 us with 8 splits (320
    // workgroups), 29.6 with 11, 26.0 with 6; N = 8192 22.7 with 8 (one per
    // CU), 28.4 with 16.  32-row blocks take the same rule (M = 32, K =
    // 8192, N = 28672: 3 splits, 336 workgroups, 42.9 us; 4 splits 36.2).
    if (env_s == 0 && t.RB >= 2 && !(a.Kt >= 128 && S * wgs <= cus)) {
        const int one = static_cast<int>(std::min<int64_t>(std::max<int64_t>(1, cus / wgs), a.Kt / kSplitMinKt));
        if (ceil_div(a.Kt, std::max(one, 1)) <= 12) {
            S = std::max(one, 1);
        } else {
            const int two = static_cast<int>(std::min<int64_t>(2 * cus / wgs, a.Kt / 8));
            S = std::max(S, two);
        }
    }
    if (env_s >= 1) S = std::min(env_s, a.Kt);
    S = cap_split_rows(a, S, env_s);
    const int64_t per_split = static_cast<int64_t>(a.M) * a.N * 4;
    if (ws_cap >= 0) S = static_cast<int>(std::min<int64_t>(S, std::max<int64_t>(1, ws_cap / per_split)));
    // splits of equal length: no split ends up empty
    const int kps = ceil_div(a.Kt, std::max(S, 1));
    S = ceil_div(a.Kt, kps);
    if (S <= 1) return t;
    // 17..64 rows with K >= 16384: 64 x 128 (or 32 x 128) tiles with K in
    // two halves inside the workgroup, twice the workgroups of the 64 x 256
    // grid at the same split count (two workgroups per CU).  Measured with
    // the plan's split count, L = 1 against L = 2 (us): 64 rows, K = 28672,
    // N = 8192: 57.0-58.2 / 53.0-53.6; 48 rows 53.1-53.5 / 49.8-50.7; 32 rows
    // 41.2 / 38.5-39.4; 24 rows 38.8-40.7 / 34.4-37.0; 64 rows, K = 16384:
    // 36.3-37.8 / 33.9-35.4; K = 20480 42.8-43.1 / 40.7-42.9.  At K = 8192
    // L = 1 stays ahead (24.4 / 24.9), and halving the splits with L = 2
    // loses everywhere.
    if (env_l == 0 && t.RB >= 2 && a.Kt >= 128 && static_cast<int64_t>(S) * wgs <= cus) t.L = 2;
    t.split = true;
    t.S = S;
    t.kps = kps;
    t.ws_bytes = S * per_split;
    return t;
}

template <int L, int RB>
void launch_split_rb(const W4Args& a, unsigned splits, hipStream_t s) {
    constexpr int NK = (L == 2 || L == 4) ? 2 : (L == 3) ? 4 : 1;
    constexpr size_t lds = 2 * NK * 16 * RB * kW4TileK * 2;
    constexpr int threads = (L >= 3) ? 512 : 256;
    const dim3 grid(ceil_div(a.Nt, ((L == 1 || L == 4) ? 4 : 2) * MM_CT), ceil_div(a.M, 16 * RB), splits);
    if constexpr (L == 1 && RB == 4) {
        if (use_w32()) {
            if (a.gmul) w4_mma_kernel<4, true, false, false, 1, true, 4, false, false, true><<<grid, 256, kMma32Lds, s>>>(a);
            else w4_mma_kernel<4, false, false, false, 1, true, 4, false, false, true><<<grid, 256, kMma32Lds, s>>>(a);
            return;
        }
    }
    if (a.gmul) {
        if constexpr (lds > 64 * 1024) allow_cu_lds<&w4_mma_kernel<4, true, false, false, L, true, RB>>();
        w4_mma_kernel<4, true, false, false, L, true, RB><<<grid, threads, lds, s>>>(a);
    } else {
        if constexpr (lds > 64 * 1024) allow_cu_lds<&w4_mma_kernel<4, false, false, false, L, true, RB>>();
        w4_mma_kernel<4, false, false, false, L, true, RB><<<grid, threads, lds, s>>>(a);
    }
}

// the split launch's tile kernel (every layout with every row block in a
// tuning build, where LHQ_W4_THIN_L forces them; the plan's forms otherwise)
void launch_split_tiles(const W4Args& a, const TilePlan& t, hipStream_t s) {
#ifdef LHQ_TUNING_KNOBS
    if (t.L != 1) {
        auto by_rb = [&](auto lc) {
            constexpr int LL = decltype(lc)::value;
            if (t.RB == 1) launch_split_rb<LL, 1>(a, t.S, s);
            else if (t.RB == 2) launch_split_rb<LL, 2>(a, t.S, s);
            else launch_split_rb<LL, 4>(a, t.S, s);
        };
        if (t.L == 2) by_rb(std::integral_constant<int, 2>{});
        else if (t.L == 3) by_rb(std::integral_constant<int, 3>{});
        else by_rb(std::integral_constant<int, 4>{});
        return;
    }
#endif
    if (t.L == 3) launch_split_rb<3, 4>(a, t.S, s);
    else if (t.L == 2 && t.RB == 1) launch_split_rb<2, 1>(a, t.S, s);
    else if (t.L == 2 && t.RB == 2) launch_split_rb<2, 2>(a, t.S, s);
    else if (t.L == 2) launch_split_rb<2, 4>(a, t.S, s);
    else if (t.RB == 2) launch_split_rb<1, 2>(a, t.S, s);
    else launch_split_rb<1, 4>(a, t.S, s);
}

int launch_split(W4Args a, const TilePlan& t, void* ws, hipStream_t s, const char* who) {
    a.ws = static_cast<float*>(ws);
    a.kps = t.kps;
    launch_split_tiles(a, t, s);
    if (int st = check_launch(who)) return st;
    const int64_t mn = static_cast<int64_t>(a.M) * a.N;
    const bool vec = mn % 4 == 0 && (reinterpret_cast<uintptr_t>(a.C) & 7) == 0;
    const unsigned blocks = static_cast<unsigned>(ceil_div64(vec ? mn / 4 : mn, 256));
    if (vec) w4_splitk_reduce_kernel<true><<<blocks, 256, 0, s>>>(a.ws, static_cast<uint16_t*>(a.C), mn, t.S);
    else w4_splitk_reduce_kernel<false><<<blocks, 256, 0, s>>>(a.ws, static_cast<uint16_t*>(a.C), mn, t.S);
    return check_launch(who);
}

// ---------------------------------------------------------------------------
// The fp32 interface (gemm_quant.hpp:47-57) at thin grids: K split across
// workgroups over a caller workspace (lhq_gemm_w4a16_ws).  The tile kernel's
// fp32 form with 16-, 32- or 64-row blocks writes each split's fp32 partial
// sums to ws[s][M][N], and w4_splitk_reduce_f32_kernel adds them in split
// order and applies the reference's alpha / beta (deterministic).
// ---------------------------------------------------------------------------
template <int L, int RB>
void launch_split_f32_rb(const W4Args& a, unsigned splits, hipStream_t s) {
    constexpr int NW = L >= 3 ? 8 : 4, NK = L == 2 ? 2 : L == 3 ? 4 : 1, WN = L == 1 ? 4 : 2;
    constexpr size_t a_bytes = static_cast<size_t>(NK) * 16 * RB * kW4TileK * 4;
    constexpr int UPW = 4 * RB / (NW / NK), PS = UPW >= 4 ? 1 : 4 / UPW;
    constexpr size_t lds = 2 * a_bytes + static_cast<size_t>(NK) * RB * PS * 64 * 16;  // tiles, partial sums
    const dim3 grid(ceil_div(a.Nt, WN * MM_CT), ceil_div(a.M, 16 * RB), splits);
    if constexpr (L == 1 && RB == 4) {
        if (use_w32()) {
            if (a.gmul) {
                allow_cu_lds<&w4_mma_kernel<4, true, false, false, 1, true, 4, true, false, true>>();
                w4_mma_kernel<4, true, false, false, 1, true, 4, true, false, true><<<grid, 256, kMma32F32Lds, s>>>(a);
            } else {
                allow_cu_lds<&w4_mma_kernel<4, false, false, false, 1, true, 4, true, false, true>>();
                w4_mma_kernel<4, false, false, false, 1, true, 4, true, false, true><<<grid, 256, kMma32F32Lds, s>>>(a);
            }
            return;
        }
    }
    if (a.gmul) {
        allow_cu_lds<&w4_mma_kernel<4, true, false, false, L, true, RB, true>>();
        w4_mma_kernel<4, true, false, false, L, true, RB, true><<<grid, 64 * NW, lds, s>>>(a);
    } else {
        allow_cu_lds<&w4_mma_kernel<4, false, false, false, L, true, RB, true>>();
        w4_mma_kernel<4, false, false, false, L, true, RB, true><<<grid, 64 * NW, lds, s>>>(a);
    }
}

// ws_cap: the workspace bytes available (-1: as much as the plan wants).
// 16-, 32- or 64-row blocks (RB = 1, 2, 4) on 256-column workgroups (L = 1)
// (65..512 rows: 64-row blocks where the unsplit grid fills at most half
// the CUs, cap_split_rows; M = 128, K = N = 8192: 142 / 50.3 us, M = 256
// 146 / 85.3, M = 256, K = 28672 499 / 241)
// and S splits that bring the grid to about two workgroups per CU, each
// walking at least 4 K tiles.  Measured on MI355X (us, lhq_gemm_w4a16 /
// this split): M = 16, K = 8192, N = 28672 48.6 / 36.4; M = 16, K = 28672,
// N = 8192 88.7 / 40.8; M = 4, N = 28672 43.8 / 34.0; M = 32, N = 28672
// 70.7 / 55.3; M = 64, K = N = 8192 181 / 35.3; M = 48, K = N = 4096 91.5 /
// 22.8 (the unsplit 64-row tile leaves the chip nearly empty from 17 rows
// on); M = 8, K = 4096, N = 11008 17.4 / 14.8.  K halves or quarters
// inside the workgroup (L = 2, 3) with splits were within noise or slower
// (M = 16, K = N = 8192: 17.6-18.8 against 18.6).  It is not used at 2..16
// rows with K * N below 32 Mi, where the unsplit kernels win or tie (M = 2,
// K = N = 4096: 5.5 / 12.1; M = 8: 11.7 / 12.5; M = 16: 13.0 / 12.9).
TilePlan plan_thin_f32(const W4Args& a, int64_t ws_cap) {
    TilePlan t;
    // (read on every call in a tuning build, so one process can sweep them)
    const int env_on = tuning_knob("LHQ_W4_F32_SPLIT", -1);  // 0: never split, 1: split wherever allowed
    const int env_s = tuning_knob("LHQ_W4_F32_SPLIT_S", 0);  // force the split count
    const int env_l = tuning_knob("LHQ_W4_F32_SPLIT_L", 0);  // force the layout (1..3)
    if (env_on == 0 || a.M < 2 || a.M > tuning_knob("LHQ_W4_THIN_MMAX", kThinMaxRows)) return t;
    if (a.G < kW4TileK || a.K % kW4TileK != 0 || static_cast<int64_t>(a.M) * a.K >= (int64_t{1} << 31)) return t;
    if (env_on != 1 && a.M <= 16 && static_cast<int64_t>(a.K) * a.N < (int64_t{32} << 20)) return t;
    t.RB = a.M <= 16 ? 1 : a.M <= 32 ? 2 : 4;
    t.L = 1;
#ifdef LHQ_TUNING_KNOBS
    if (env_l >= 1 && env_l <= 3 && (t.RB < 4 || env_l == 1)) t.L = env_l;
#else
    (void)env_l;
#endif
    const int WN = t.L == 1 ? 4 : 2, per_cu = t.L >= 3 ? 1 : 2;
    const int64_t wgs = static_cast<int64_t>(ceil_div(a.Nt, WN * MM_CT)) * ceil_div(a.M, 16 * t.RB);
    const int cus = std::max(device_cus(), 1);
    // more than 64 rows: only where the unsplit grid leaves a CU without a
    // workgroup (M = 128, K = 8192, N = 28672, 224 workgroups: 154-162 us
    // unsplit, 139-140 with 2 splits; the bf16 form gains nothing there and
    // splits only grids of at most half the CUs)
    if (env_s == 0 && a.M > 64 && wgs > cus) return t;
    // about one round of the resident workgroups, at least 4 K tiles each
    int S = static_cast<int>(std::min<int64_t>(std::max<int64_t>(1, per_cu * cus / wgs), a.Kt / kSplitMinKt));
    if (env_s >= 1) S = std::min(env_s, a.Kt);
    S = cap_split_rows(a, S, env_s);
    const int64_t per_split = static_cast<int64_t>(a.M) * a.N * 4;
    if (ws_cap >= 0) S = static_cast<int>(std::min<int64_t>(S, std::max<int64_t>(1, ws_cap / per_split)));
    const int kps = ceil_div(a.Kt, std::max(S, 1));
    S = ceil_div(a.Kt, kps);
    if (S <= 1) return t;
    t.split = true;
    t.S = S;
    t.kps = kps;
    t.ws_bytes = S * per_split;
    return t;
}

int launch_split_f32(W4Args a, const TilePlan& t, void* ws, hipStream_t s, const char* who) {
    a.ws = static_cast<float*>(ws);
    a.kps = t.kps;
    const unsigned S = static_cast<unsigned>(t.S);
#ifdef LHQ_TUNING_KNOBS
    if (t.L == 3 && t.RB < 4) t.RB == 1 ? launch_split_f32_rb<3, 1>(a, S, s) : launch_split_f32_rb<3, 2>(a, S, s);
    else if (t.L == 2 && t.RB < 4) t.RB == 1 ? launch_split_f32_rb<2, 1>(a, S, s) : launch_split_f32_rb<2, 2>(a, S, s);
    else
#endif
    if (t.RB == 4) launch_split_f32_rb<1, 4>(a, S, s);
    else t.RB == 1 ? launch_split_f32_rb<1, 1>(a, S, s) : launch_split_f32_rb<1, 2>(a, S, s);
    if (int st = check_launch(who)) return st;
    const int64_t mn = static_cast<int64_t>(a.M) * a.N;
    const bool vec = mn % 4 == 0 && (reinterpret_cast<uintptr_t>(a.C) & 15) == 0;
    const unsigned blocks = static_cast<unsigned>(ceil_div64(vec ? mn / 4 : mn, 256));
    float* const C = static_cast<float*>(a.C);
    if (vec) w4_splitk_reduce_f32_kernel<true><<<blocks, 256, 0, s>>>(a.ws, C, mn, t.S, a.alpha, a.beta);
    else w4_splitk_reduce_f32_kernel<false><<<blocks, 256, 0, s>>>(a.ws, C, mn, t.S, a.alpha, a.beta);
    return check_launch(who);
}

// lhq_gemm_w4a16 with a workspace of ws_cap bytes at ws (0: none).
int gemm_w4a16_f32(const char* who, const float* A, const uint8_t* qweight, const float* scales, float* C, int M,
                   int N, int K, int G, float alpha, float beta, void* ws, int64_t ws_cap, void* stream) {
    if (int st = check_w4_shape(who, M, N, K, G)) return st;
    LHQ_REQUIRE(qweight && scales && C && (A || M == 0), "%s: null pointer", who);
    LHQ_REQUIRE(ws || ws_cap <= 0, "%s: null workspace with %lld bytes", who, static_cast<long long>(ws_cap));
    if (M == 0) return LHQ_OK;
    W4Args a = make_args(A, qweight, scales, nullptr, C, M, N, K, G, alpha, beta);
    if (ws_cap > 0) {
        const TilePlan t = plan_thin_f32(a, ws_cap);
        if (t.split) {
            LHQ_REQUIRE((reinterpret_cast<uintptr_t>(ws) & 15) == 0, "%s: workspace not 16-byte aligned", who);
            return launch_split_f32(a, t, ws, as_stream(stream), who);
        }
    }
    const int thin = f32_thin_layout(a, M);
    if (!thin && mma_applies(a, M, M)) return launch_mma_f32(a, as_stream(stream), who);
    if (thin == 2) return M <= 16 ? launch_mma_f32_rb<2, 1>(a, as_stream(stream), who)
                                  : launch_mma_f32_rb<2, 2>(a, as_stream(stream), who);
    if (thin == 3) return M <= 16 ? launch_mma_f32_rb<3, 1>(a, as_stream(stream), who)
                                  : launch_mma_f32_rb<3, 2>(a, as_stream(stream), who);
    if (thin == 1) return M <= 16 ? launch_mma_f32_rb<1, 1>(a, as_stream(stream), who)
                                  : launch_mma_f32_rb<1, 2>(a, as_stream(stream), who);
    return launch_w4<true, false, true>(a, 1, as_stream(stream));
}

// lhq_gemm_w4a16_bf16 with a workspace of ws_bytes at ws (ws_cap < 0: the
// plan may use as much as it wants, the caller has checked that it fits).
int gemm_w4a16_bf16_plan(const char* who, const uint16_t* A, const uint8_t* qweight, const uint16_t* scales,
                         const uint32_t* zeros, uint16_t* C, int M, int N, int K, int G, void* ws,
                         int64_t ws_cap, void* stream) {
    if (int st = check_w4_shape(who, M, N, K, G)) return st;
    LHQ_REQUIRE(qweight && scales && zeros && C && (A || M == 0), "%s: null pointer", who);
    LHQ_REQUIRE(ws || ws_cap <= 0, "%s: null workspace with %lld bytes", who, static_cast<long long>(ws_cap));
    if (M == 0) return LHQ_OK;
    W4Args a = make_args(A, qweight, scales, zeros, C, M, N, K, G, 1.0f, 0.0f);
    const TilePlan t = plan_thin(a, ws ? ws_cap : 0);
    if (t.split) {
        LHQ_REQUIRE((reinterpret_cast<uintptr_t>(ws) & 15) == 0, "%s: workspace not 16-byte aligned", who);
        return launch_split(a, t, ws, as_stream(stream), who);
    }
    if (mma_applies(a, M, M)) return launch_mma<false>(a, M, 0, 1, as_stream(stream), who);
    return launch_w4<false, true, false>(a, 1, as_stream(stream));
}

}  // namespace

// The no-allocation entry point's split-K scratch: one array per device, in
// the code object's zero-initialised device data (every GPU the library runs
// on holds it until the process ends).  Host code never uses the array's
// name as an address: it reaches each device's copy only through the
// pointer hipGetSymbolAddress returns with that device current.  The plan
// writes every partial sum it later reads, so nothing in it needs clearing
// between calls; calls that overlap on one GPU share it and race.
constexpr int64_t kNoAllocScratchBytes = int64_t{32} << 20;
static __device__ __align__(256) float scratch[kNoAllocScratchBytes / 4];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The current device's scratch address, looked up on the first call made on
// that device and kept.  hipGetSymbolAddress is no stream operation, so that
// first call may also be made under HIP graph capture (tested in a fresh
// process whose first call is captured).
int scratch_for_current_device(const char* who, void** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return set_error(LHQ_ERR_HIP, "%s: hipGetDevice: %s", who, hipGetErrorString(e));
    LHQ_SUPPORTED(dev >= 0 && dev < kMaxDevices, "%s: device %d beyond the %d this library tracks", who, dev,
                  kMaxDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return set_error(LHQ_ERR_HIP, "%s: scratch address on device %d: %s", who, dev, hipGetErrorString(e));
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return LHQ_OK;
}

}  // namespace
}  // namespace lhq

using namespace lhq;

extern "C" {

int lhq_gemm_w4a16(const float* A, const uint8_t* qweight, const float* scales, float* C, int M,
                   int N, int K, int G, float alpha, float beta, void* stream) {
    return gemm_w4a16_f32("gemm_w4a16", A, qweight, scales, C, M, N, K, G, alpha, beta, nullptr, 0, stream);
}

int64_t lhq_gemm_w4a16_workspace_bytes(int M, int N, int K, int G) {
    if (check_w4_shape("gemm_w4a16_workspace_bytes", M, N, K, G) || M == 0) return 0;
    const W4Args a = make_args(nullptr, nullptr, nullptr, nullptr, nullptr, M, N, K, G, 1.0f, 0.0f);
    return plan_thin_f32(a, -1).ws_bytes;
}

int lhq_gemm_w4a16_ws(const float* A, const uint8_t* qweight, const float* scales, float* C, int M, int N, int K,
                      int G, float alpha, float beta, void* workspace, int64_t workspace_bytes, void* stream) {
    LHQ_REQUIRE(workspace_bytes >= 0, "gemm_w4a16_ws: negative workspace_bytes");
    return gemm_w4a16_f32("gemm_w4a16_ws", A, qweight, scales, C, M, N, K, G, alpha, beta, workspace,
                          workspace ? workspace_bytes : 0, stream);
}

int lhq_gemm_w4a16_bf16(const uint16_t* A, const uint8_t* qweight, const uint16_t* scales,
                        const uint32_t* zeros, uint16_t* C, int M, int N, int K, int G,
                        void* stream) {
    if (int st = check_w4_shape("gemm_w4a16_bf16", M, N, K, G)) return st;
    LHQ_REQUIRE(qweight && scales && zeros && C && (A || M == 0), "gemm_w4a16_bf16: null pointer");
    if (M == 0) return LHQ_OK;
    W4Args a = make_args(A, qweight, scales, zeros, C, M, N, K, G, 1.0f, 0.0f);
    if (mma_applies(a, M, M)) return launch_mma<false>(a, M, 0, 1, as_stream(stream), "w4a16 prefill");
    return launch_w4<false, true, false>(a, 1, as_stream(stream));
}

int64_t lhq_gemm_w4a16_bf16_workspace_bytes(int M, int N, int K, int G) {
    if (check_w4_shape("gemm_w4a16_bf16_workspace_bytes", M, N, K, G) || M == 0) return 0;
    const W4Args a = make_args(nullptr, nullptr, nullptr, nullptr, nullptr, M, N, K, G, 1.0f, 0.0f);
    return plan_thin(a, -1).ws_bytes;
}

int lhq_gemm_w4a16_bf16_ws(const uint16_t* A, const uint8_t* qweight, const uint16_t* scales,
                           const uint32_t* zeros, uint16_t* C, int M, int N, int K, int G, void* workspace,
                           int64_t workspace_bytes, void* stream) {
    LHQ_REQUIRE(workspace_bytes >= 0, "gemm_w4a16_bf16_ws: negative workspace_bytes");
    return gemm_w4a16_bf16_plan("gemm_w4a16_bf16_ws", A, qweight, scales, zeros, C, M, N, K, G, workspace,
                                workspace ? workspace_bytes : 0, stream);
}

int lhq_gemm_w4a16_bf16_noalloc(const uint16_t* A, const uint8_t* qweight, const uint16_t* scales,
                                const uint32_t* zeros, uint16_t* C, int M, int N, int K, int G, void* stream) {
    const char* who = "gemm_w4a16_bf16_noalloc";
    if (int st = check_w4_shape(who, M, N, K, G)) return st;
    // the workspace entry point's plan with a workspace of min(need, the
    // scratch): a shape whose plan asks for more runs fewer splits, as
    // lhq_gemm_w4a16_bf16_ws does with a 32 MiB workspace
    const int64_t need = lhq_gemm_w4a16_bf16_workspace_bytes(M, N, K, G);
    const int64_t cap = need < kNoAllocScratchBytes ? need : kNoAllocScratchBytes;
    void* ws = nullptr;
    if (cap > 0)
        if (int st = scratch_for_current_device(who, &ws)) return st;
    return gemm_w4a16_bf16_plan(who, A, qweight, scales, zeros, C, M, N, K, G, ws, cap, stream);
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
    if (mma_applies(a, M, M)) return launch_mma<false>(a, M, 0, batch, as_stream(stream), "w4a16 prefill batched");
    return launch_w4<false, true, false>(a, batch, as_stream(stream));
}

int lhq_gemm_w4a16_bf16_grouped(const uint16_t* A, const int32_t* offsets, const uint8_t* const* qweights,
                                const uint16_t* const* scales, const uint32_t* const* zeros, uint16_t* C,
                                int num_groups, int row_capacity, int N, int K, int G, void* stream) {
    return grouped_w4<false>("gemm_w4a16_bf16_grouped", A, offsets, qweights, scales, zeros, C, num_groups,
                             row_capacity, N, K, G, nullptr, 0, stream);
}

int lhq_gemm_w4a16_bf16_grouped_swiglu(const uint16_t* A, const int32_t* offsets, const uint8_t* const* qweights,
                                       const uint16_t* const* scales, const uint32_t* const* zeros, uint16_t* act,
                                       int num_groups, int row_capacity, int I, int K, int G, void* stream) {
    return grouped_w4<true>("gemm_w4a16_bf16_grouped_swiglu", A, offsets, qweights, scales, zeros, act,
                            num_groups, row_capacity, I, K, G, nullptr, 0, stream);
}

int64_t lhq_gemm_w4a16_bf16_grouped_workspace_bytes(int num_groups, int row_capacity, int N, int K, int G) {
    if (check_w4_shape("gemm_w4a16_bf16_grouped_workspace_bytes", row_capacity, N, K, G) || num_groups <= 0 ||
        row_capacity == 0)
        return 0;
    const W4Args a = grouped_args<false>(nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, num_groups,
                                         row_capacity, N, K, G);
    return grouped_uses_tiles(a) ? std::max<int64_t>(1, grouped_pk_slots(a)) * kPkSlotBytes : 0;
}

int64_t lhq_gemm_w4a16_bf16_grouped_swiglu_workspace_bytes(int num_groups, int row_capacity, int I, int K, int G) {
    if (check_w4_shape("gemm_w4a16_bf16_grouped_swiglu_workspace_bytes", row_capacity, I, K, G) ||
        num_groups <= 0 || row_capacity == 0)
        return 0;
    const W4Args a = grouped_args<true>(nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, num_groups,
                                        row_capacity, I, K, G);
    return grouped_uses_tiles(a) ? std::max<int64_t>(1, grouped_pk_slots(a)) * kPkSlotBytes : 0;
}

int lhq_gemm_w4a16_bf16_grouped_ws(const uint16_t* A, const int32_t* offsets, const uint8_t* const* qweights,
                                   const uint16_t* const* scales, const uint32_t* const* zeros, uint16_t* C,
                                   int num_groups, int row_capacity, int N, int K, int G, void* workspace,
                                   int64_t workspace_bytes, void* stream) {
    return grouped_w4<false>("gemm_w4a16_bf16_grouped_ws", A, offsets, qweights, scales, zeros, C, num_groups,
                             row_capacity, N, K, G, workspace, workspace ? workspace_bytes : 0, stream);
}

int lhq_gemm_w4a16_bf16_grouped_swiglu_ws(const uint16_t* A, const int32_t* offsets,
                                          const uint8_t* const* qweights, const uint16_t* const* scales,
                                          const uint32_t* const* zeros, uint16_t* act, int num_groups,
                                          int row_capacity, int I, int K, int G, void* workspace,
                                          int64_t workspace_bytes, void* stream) {
    return grouped_w4<true>("gemm_w4a16_bf16_grouped_swiglu_ws", A, offsets, qweights, scales, zeros, act,
                            num_groups, row_capacity, I, K, G, workspace, workspace ? workspace_bytes : 0, stream);
}

}  // extern "C"
