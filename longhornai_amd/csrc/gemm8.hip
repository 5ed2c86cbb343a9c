// gemm8.hip -- 8-bit-operand GEMMs for gfx950: W8A8 int8 (int32 accumulate)
// and FP8 E4M3 (fp32 accumulate), LDS-staged MFMA tiles.
//
// Reference: gemm_w8a8 (gemm_quant.cpp:29-49) runs an int32 dot product per
// output with B strided by N, then C += ((alpha*a_s)*b_s)*float(acc);
// gemm_fp8_e4m3 (gemm_quant.cpp:87-104) accumulates decoded e4m3 products in
// fp32 and adds ((alpha*sA)*sB)*acc.
//
// Here a 256-thread workgroup owns a 256x256 output tile; the four waves
// (2x2) each own 128x128 of it: 8x8 blocks of 16x16 int8 MFMA accumulators
// in the W8A8 kernel (dma_tile_m16), 4x4 blocks of 32x32 in the FP8 and
// register-staged kernels (and the 32x32x32 int8 tile dma_tile, kept for
// comparison in tuning builds).  A (row
// major [M,K]) and the prepacked k-contiguous B^T ([Np,Kp], lhq_b8_prepack)
// are staged through double-buffered LDS tiles of 256 x 128 bytes with a
// 16-byte row pad (conflict-free 128-bit LDS reads).  Integer accumulation is
// exact, so the int32 result equals the reference's bit for bit at any tiling;
// the fp32 epilogue repeats the reference's multiply order with no fused
// multiply-add, so the fp32 output is bit-exact too.  Workgroups are mapped
// XCD-aware: consecutive tiles of one group of tile rows land on one XCD so
// its L2 sees the A rows and B columns they share.  Where the tiles fill at
// most half the CUs, every workgroup takes a 256x128 half tile instead; up to
// 32 rows gemm8_mid_kernel runs 16x16 MFMA blocks straight from global
// memory with K split across its waves (the M = 1 GEMV of config 1 and
// batched decode).
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
    int c_vec;  // C is 16-byte aligned (vector stores allowed where rows are)
    float alpha, beta;
};

// Tile order: workgroup b runs on XCD (b % 8); give each XCD a contiguous
// range of tile ids, and walk tile ids in groups of `group_m` tile rows
// (column-major inside a group) so concurrently running tiles share A rows
// and B columns.
__device__ __forceinline__ void tile_of_id(int id, const Gemm8Args& p, int& tm, int& tn) {
    const int gm = p.group_m;
    const int per_group = gm * p.tiles_n;
    const int group = id / per_group;
    const int first = group * gm;
    const int rows = min(p.tiles_m - first, gm);
    const int in = id - group * per_group;
    tm = first + in % rows;
    tn = in / rows;
}
__device__ __forceinline__ void tile_of(int b, const Gemm8Args& p, int& tm, int& tn) {
    // XCD x receives blocks x, x+8, ...: q + (x < r) of them; hand it the
    // contiguous id range starting at x*q + min(x, r) (a bijection).
    const int total = p.tiles_m * p.tiles_n;
    const int q = total / 8, r = total % 8;
    const int xcd = b % 8, slot = b / 8;
    tile_of_id(xcd * q + min(xcd, r) + slot, p, tm, tn);
}

// Epilogue shared by the 8-bit kernels: scale, apply beta and store the
// 256x256 tile.  Element 4q+r of block (i, j) in lane l is C[row][col] with
// row = m0 + 128*wm + 32*i + (l & 31) and
// col = n0 + 128*wn + 32*j + 4*(l >> 5) + 8*q + r: four adjacent columns
// per (i, j, q), stored as one vector.  INTERIOR: the whole tile is in range
// and rows are 16-byte aligned (N % 4 == 0), so nothing is tested per
// element; edge tiles test rows and columns.  Offsets are 32-bit from the
// tile's first element (the launcher bounds 256*N).  LS: the int8 scales
// of this tile are staged in LDS at ls (ls[r] = A_s[m0 + r],
// ls[256 + c] = B_s[n0 + c], clamped to the last row / column).
template <int OP, int EPI, bool INTERIOR, bool LS, typename Acc>
__device__ __forceinline__ void gemm8_store(const Gemm8Args& p, const Acc (&acc)[4][4], int m0, int n0, int wm,
                                            int wn, int lane, const float* ls) {
    const int lr = lane & 31, lh = lane >> 5;
    const bool vec_ok = INTERIOR || (p.c_vec && (p.N & 3) == 0);
    float row_scale[4];     // int8: alpha * A_s[row] (gemm_quant.cpp:44-45)
    float combined = 0.0f;  // fp8: (alpha * sA) * sB (gemm_quant.cpp:98)
    if constexpr (EPI != EPI_I32) {
        if constexpr (OP == OP_I8) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int rt = wm * 128 + i * 32 + lr;
                const int row = m0 + rt;
                row_scale[i] = p.alpha * (LS ? ls[rt] : p.As[INTERIOR ? row : min(row, p.M - 1)]);
            }
        } else {
            combined = p.alpha * p.As[0];
            combined = combined * p.Bs[0];
        }
    }
    const size_t tile_off = static_cast<size_t>(m0) * p.N + n0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int cb = wn * 128 + j * 32 + 4 * lh;  // column within the tile
        float bs[4][4];
        if constexpr (OP == OP_I8 && EPI != EPI_I32) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                if constexpr (LS) {
                    // cb + 8q is a multiple of 4: one 16-byte LDS read
                    const f32x4_t v = *reinterpret_cast<const f32x4_t*>(ls + BM + cb + 8 * q);
#pragma unroll
                    for (int r = 0; r < 4; ++r) bs[q][r] = v[r];
                } else {
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int col = n0 + cb + 8 * q + r;
                        bs[q][r] = p.Bs[INTERIOR ? col : min(col, p.N - 1)];
                    }
                }
            }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int rt = wm * 128 + i * 32 + lr;  // row within the tile
            if (!INTERIOR && m0 + rt >= p.M) continue;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int ct = cb + 8 * q;
                const int col = n0 + ct;
                if (!INTERIOR && col >= p.N) continue;
                const uint32_t o = static_cast<uint32_t>(rt) * static_cast<uint32_t>(p.N) + static_cast<uint32_t>(ct);
                const bool full = INTERIOR || (vec_ok && col + 3 < p.N);
                if constexpr (EPI == EPI_I32) {
                    const i32x4_t v = {acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
                    int32_t* Cp = static_cast<int32_t*>(p.C) + tile_off + o;
                    if (full) {
                        *reinterpret_cast<i32x4_t*>(Cp) = v;
                    } else {
#pragma unroll
                        for (int r = 0; r < 4; ++r)
                            if (col + r < p.N) Cp[r] = v[r];
                    }
                } else {
                    float f[4];
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        if constexpr (OP == OP_I8) {
                            f[r] = row_scale[i] * bs[q][r];  // left to right, as the reference
                            f[r] = f[r] * static_cast<float>(acc[i][j][4 * q + r]);
                        } else {
                            f[r] = combined * acc[i][j][4 * q + r];
                        }
                    }
                    if constexpr (EPI == EPI_F32) {
                        // apply_beta (gemm_quant.cpp:12-21), then C += rescaled
                        float* Cp = static_cast<float*>(p.C) + tile_off + o;
                        if (full) {
                            f32x4_t c = {0.f, 0.f, 0.f, 0.f};
                            if (p.beta != 0.0f) c = *reinterpret_cast<const f32x4_t*>(Cp);
#pragma unroll
                            for (int r = 0; r < 4; ++r) {
                                const float base = (p.beta == 0.0f) ? 0.0f : (p.beta == 1.0f) ? c[r] : c[r] * p.beta;
                                c[r] = base + f[r];
                            }
                            *reinterpret_cast<f32x4_t*>(Cp) = c;
                        } else {
#pragma unroll
                            for (int r = 0; r < 4; ++r) {
                                if (col + r >= p.N) continue;
                                const float base = (p.beta == 0.0f) ? 0.0f : (p.beta == 1.0f) ? Cp[r] : Cp[r] * p.beta;
                                Cp[r] = base + f[r];
                            }
                        }
                    } else {
                        // bf16 output of C = 0 + rescaled (beta = 0)
                        uint16_t* Cp = static_cast<uint16_t*>(p.C) + tile_off + o;
                        const uint32_t lo = pack_bf16x2(0.0f + f[0], 0.0f + f[1]);
                        const uint32_t hi = pack_bf16x2(0.0f + f[2], 0.0f + f[3]);
                        if (full) {
                            *reinterpret_cast<u32x2_t*>(Cp) = u32x2_t{lo, hi};
                        } else {
                            const uint16_t h[4] = {static_cast<uint16_t>(lo), static_cast<uint16_t>(lo >> 16),
                                                   static_cast<uint16_t>(hi), static_cast<uint16_t>(hi >> 16)};
#pragma unroll
                            for (int r = 0; r < 4; ++r)
                                if (col + r < p.N) Cp[r] = h[r];
                        }
                    }
                }
            }
        }
    }
}

// Interior-tile epilogue of the int8 DMA kernel, through LDS.  Per 32-row
// block i of the wave's 128x128 quadrant:
//   1. the raw int32 accumulators go to the wave's LDS area, row-major
//      (straight from the accumulator registers, no VALU work);
//   2. the wave reads them back along rows, CPL consecutive columns per lane
//      (8 for bf16 output, 4 otherwise), scales them and stores 16 bytes per
//      lane: bf16 4 rows x 256 B, fp32 / int32 2 rows x 512 B per store.
// In that layout a lane owns the same columns for every row, so it keeps
// just CPL column scales in registers and reads one (broadcast) row scale
// per row.  Scaling is the reference's ((alpha*A_s[r]) * B_s[c]) * acc
// (gemm_quant.cpp:44-46); with beta = 0 the "0 + x" of apply_beta is folded
// into the last multiply as fma(s, acc, +0), which is exact: for a nonzero
// product no rounding to zero can occur (|acc| >= 1 and a nonzero fp32 s is
// >= 2^-149), and an exactly zero product gives +0 either way (-0 + +0 =
// +0).  area: this wave's 32 rows of 128 int32 plus a 4-word pad per row
// (row starts 4 banks apart).  ls: the tile's scales in LDS (A_s, then B_s;
// clamped to the last row / column).  EDGE: the tile crosses M or N (or
// rows are not 16-byte aligned); rows and columns are tested and partial
// column groups stored element by element.
// JB: 32-column accumulator blocks per wave (4: a 128x128 quadrant of a
// 256x256 tile; 2: a 128x64 quadrant of a 256x128 half tile).
constexpr int STAGED_PITCH = 4 * (128 + 4);

// FP8: fp32 accumulators (staged as their bit patterns) and the per-tensor
// scales of gemm_fp8_e4m3 (gemm_quant.cpp:95-101: combined = (alpha * sA) * sB,
// C = beta-applied C + combined * acc; with beta = 0, 0 + x is kept as an
// add: an fp32 accumulator can be small enough for the product to underflow,
// where fma(s, acc, +0) could return -0).
// AI = 8: acc holds 8 x 2JB blocks of 16x16 (the 16x16x64 tile): block
// (i, j) in lane l is row 16i + (l & 15), columns 16j + 4(l >> 4) ..+3 of
// the quadrant, one 16-byte row piece per block.
template <int EPI, bool EDGE, int JB = 4, bool FP8 = false, typename Acc = i32x16_t, int AI = 4, int AJ = 4>
__device__ __forceinline__ void gemm8_store_staged(const Gemm8Args& p, const Acc (&acc)[AI][AJ], int m0, int n0,
                                                   int wm, int wn, int lane, const float* ls, uint8_t* area) {
    constexpr int WQ = 32 * JB;                   // quadrant width
    constexpr int CPL = EPI == EPI_BF16 ? 8 : 4;  // columns per lane (16 output bytes)
    constexpr int LPR = WQ / CPL;                 // lanes per row
    constexpr int RPP = 64 / LPR;                 // rows per pass
    const int lr = lane & 31, lh = lane >> 5;
    const int rsub = lane / LPR, cl = lane % LPR;
    float bsc[CPL];  // B_s of the lane's columns
    if constexpr (FP8) {
#pragma unroll
        for (int c = 0; c < CPL; ++c) bsc[c] = p.Bs[0];
    } else if constexpr (EPI != EPI_I32) {
#pragma unroll
        for (int c = 0; c < CPL; c += 4) {
            const f32x4_t v = *reinterpret_cast<const f32x4_t*>(ls + BM + wn * WQ + cl * CPL + c);
#pragma unroll
            for (int r = 0; r < 4; ++r) bsc[c + r] = v[r];
        }
    }
    // an accumulator as fp32: int8 converts the int32, FP8 reinterprets bits
    auto accf = [](int32_t v) { return FP8 ? __int_as_float(v) : static_cast<float>(v); };
    // this wave's quadrant of C, 32-bit element offsets from its first element
    const size_t quad_off = static_cast<size_t>(m0 + wm * 128) * p.N + n0 + wn * WQ;
    const bool beta0 = p.beta == 0.0f;
    const int cols_left = p.N - (n0 + wn * WQ + cl * CPL);  // in-range columns from the lane's first
    const bool vec_ok = !EDGE || (p.c_vec && cols_left >= CPL && p.N % CPL == 0);
    // 1. raw accumulators of block i, row lr, columns 32j + 4lh + 8q ..+3
    auto stage_block = [&](int i) {
        if constexpr (AI == 8) {
            // rows 32i .. 32i+31 are 16x16 block rows 2i and 2i + 1
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int j = 0; j < 2 * JB; ++j)
                    *reinterpret_cast<i32x4_t*>(area + (16 * h + (lane & 15)) * STAGED_PITCH +
                                                (16 * j + 4 * (lane >> 4)) * 4) =
                        __builtin_bit_cast(i32x4_t, acc[2 * i + h][j]);
        } else {
#pragma unroll
            for (int j = 0; j < JB; ++j)
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    *reinterpret_cast<i32x4_t*>(area + lr * STAGED_PITCH + (j * 32 + 4 * lh + 8 * q) * 4) =
                        __builtin_bit_cast(i32x4_t,
                                           decltype(acc[i][j].xyzw){acc[i][j][4 * q], acc[i][j][4 * q + 1],
                                                                    acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]});
        }
    };
    auto wave_sync = [&]() {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };
    stage_block(0);
    wave_sync();  // the wave reads back what its other lanes wrote
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        // 2. along rows: every LDS read of the block first (data and row
        // scales, 64 + 8..16 registers), then the passes that scale and store
        constexpr int PASSES = 32 / RPP;
        int32_t ab[PASSES][CPL];
        float rsb[PASSES];
#pragma unroll
        for (int t = 0; t < PASSES; ++t) {
            const int R = t * RPP + rsub;
            const uint8_t* src = area + R * STAGED_PITCH + cl * CPL * 4;
#pragma unroll
            for (int c = 0; c < CPL; c += 4) {
                const i32x4_t v = *reinterpret_cast<const i32x4_t*>(src + c * 4);
#pragma unroll
                for (int r = 0; r < 4; ++r) ab[t][c + r] = v[r];
            }
            if constexpr (FP8) rsb[t] = p.As[0];
            else if constexpr (EPI != EPI_I32) rsb[t] = ls[wm * 128 + i * 32 + R];
        }
        // block i + 1 goes to LDS while block i is scaled and stored: a
        // wave's LDS operations execute in order, so these writes land after
        // the reads above
        __builtin_amdgcn_sched_barrier(0);
        if (i + 1 < 4) stage_block(i + 1);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int t = 0; t < PASSES; ++t) {
            const int R = t * RPP + rsub;                  // row within the block
            const int rq = i * 32 + R;                     // row within the quadrant
            if (EDGE && (m0 + wm * 128 + rq >= p.M || cols_left <= 0)) continue;
            const int32_t (&a)[CPL] = ab[t];
            const uint32_t o = static_cast<uint32_t>(rq) * static_cast<uint32_t>(p.N) + static_cast<uint32_t>(cl * CPL);
            if constexpr (EPI == EPI_I32) {
                int32_t* Cp = static_cast<int32_t*>(p.C) + quad_off + o;
                if (vec_ok) {
                    *reinterpret_cast<i32x4_t*>(Cp) = i32x4_t{a[0], a[1], a[2], a[3]};
                } else {
#pragma unroll
                    for (int c = 0; c < 4; ++c)
                        if (c < cols_left) Cp[c] = a[c];
                }
            } else {
                const float rs = p.alpha * rsb[t];  // gemm_quant.cpp:44-45
                float f[CPL];
                if constexpr (EPI == EPI_BF16) {
                    // C = 0 + rescaled, rounded to bf16
#pragma unroll
                    for (int c = 0; c < CPL; ++c) f[c] = __builtin_fmaf(rs * bsc[c], accf(a[c]), 0.0f);
                    const u32x4_t v = {pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3]), pack_bf16x2(f[4], f[5]),
                                       pack_bf16x2(f[6], f[7])};
                    uint16_t* Cp = static_cast<uint16_t*>(p.C) + quad_off + o;
                    if (vec_ok) {
                        *reinterpret_cast<u32x4_t*>(Cp) = v;
                    } else {
#pragma unroll
                        for (int c = 0; c < CPL; ++c)
                            if (c < cols_left) Cp[c] = static_cast<uint16_t>(v[c >> 1] >> (16 * (c & 1)));
                    }
                } else {
                    float* Cp = static_cast<float*>(p.C) + quad_off + o;
                    f32x4_t c4 = {0.f, 0.f, 0.f, 0.f};
                    if (!vec_ok) {
                        // partial group: element by element, same operations
#pragma unroll
                        for (int c = 0; c < 4; ++c) {
                            if (c >= cols_left) continue;
                            float x;
                            if (beta0 && !FP8) {
                                x = __builtin_fmaf(rs * bsc[c], accf(a[c]), 0.0f);
                            } else if (beta0) {
                                f[c] = rs * bsc[c];
                                f[c] = f[c] * accf(a[c]);
                                x = 0.0f + f[c];
                            } else {
                                f[c] = rs * bsc[c];
                                f[c] = f[c] * accf(a[c]);
                                const float base = (p.beta == 1.0f) ? Cp[c] : Cp[c] * p.beta;
                                x = base + f[c];
                            }
                            Cp[c] = x;
                        }
                        continue;
                    }
                    if (beta0 && !FP8) {
#pragma unroll
                        for (int c = 0; c < 4; ++c) c4[c] = __builtin_fmaf(rs * bsc[c], accf(a[c]), 0.0f);
                    } else if (beta0) {
#pragma unroll
                        for (int c = 0; c < 4; ++c) {
                            f[c] = rs * bsc[c];
                            f[c] = f[c] * accf(a[c]);
                            c4[c] = 0.0f + f[c];
                        }
                    } else {
                        // apply_beta (gemm_quant.cpp:12-21), then C += rescaled
                        c4 = *reinterpret_cast<const f32x4_t*>(Cp);
#pragma unroll
                        for (int c = 0; c < 4; ++c) {
                            f[c] = rs * bsc[c];
                            f[c] = f[c] * accf(a[c]);
                            const float base = (p.beta == 1.0f) ? c4[c] : c4[c] * p.beta;
                            c4[c] = base + f[c];
                        }
                    }
                    *reinterpret_cast<f32x4_t*>(Cp) = c4;
                }
            }
        }
        wave_sync();  // block i + 1 is in LDS for every lane
    }
}

template <int OP, int EPI, bool LS = false, typename Acc>
__device__ __forceinline__ void gemm8_epilogue(const Gemm8Args& p, const Acc (&acc)[4][4], int m0, int n0, int wm,
                                               int wn, int lane, const float* ls = nullptr) {
    if (m0 + BM <= p.M && n0 + BN <= p.N && (p.N & 3) == 0 && p.c_vec)
        gemm8_store<OP, EPI, true, LS>(p, acc, m0, n0, wm, wn, lane, ls);
    else
        gemm8_store<OP, EPI, false, LS>(p, acc, m0, n0, wm, wn, lane, ls);
}

template <int OP, int EPI>
__global__ __launch_bounds__(NTHREADS) void gemm8_kernel(Gemm8Args p) {
    __shared__ __attribute__((aligned(16))) uint8_t lds[2][2][TILE_BYTES];

    int tm, tn;
    tile_of(blockIdx.x, p, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;

    // Global -> register staging.  Every load is unconditional: rows past M
    // read row M-1 and k past K reads the row's last 16 bytes; both are
    // replaced by zero codes before they reach LDS (a zero code times the
    // zero-padded B contributes nothing, and for e4m3 a stray NaN code
    // could not hide behind a zero weight).  Loads issued on only some
    // control paths would make every later wait in the loop a full drain.
    struct Stage {
        u32x4_t a[CHUNKS], b[CHUNKS];
        uint32_t a_ok;  // bit i: chunk i of A is in range
    };
    const int r_base = tid >> 3, kc = (tid & 7) * 16;
    // Byte offsets fit in 32 bits (the launcher checks M*K and Np*Kp); the
    // row parts are loop-invariant, only k advances.
    uint32_t a_row[CHUNKS], b_row[CHUNKS];
#pragma unroll
    for (int i = 0; i < CHUNKS; ++i) {
        const int r = r_base + (NTHREADS / 8) * i;
        a_row[i] = static_cast<uint32_t>(min(m0 + r, p.M - 1)) * static_cast<uint32_t>(p.K);
        b_row[i] = static_cast<uint32_t>(n0 + r) * static_cast<uint32_t>(p.Kp);
    }
    const uint32_t m_rows_ok = static_cast<uint32_t>(max(0, min(p.M - m0, BM)));  // rows of this tile in range
    auto load_stage = [&](Stage& st, int kt) {
        const int gk = kt * BK + kc;
        const uint32_t ka = static_cast<uint32_t>(min(gk, p.K - 16));
        st.a_ok = 0;
#pragma unroll
        for (int i = 0; i < CHUNKS; ++i) {
            const uint32_t r = static_cast<uint32_t>(r_base + (NTHREADS / 8) * i);
            st.a_ok |= static_cast<uint32_t>(r < m_rows_ok && gk < p.K) << i;
            st.a[i] = *reinterpret_cast<const u32x4_t*>(p.A + (a_row[i] + ka));
            st.b[i] = *reinterpret_cast<const u32x4_t*>(p.Bt + (b_row[i] + static_cast<uint32_t>(gk)));
        }
    };
    auto store_stage = [&](const Stage& st, int buf) {
        const u32x4_t zero = {0, 0, 0, 0};
#pragma unroll
        for (int i = 0; i < CHUNKS; ++i) {
            const int r = r_base + (NTHREADS / 8) * i;
            *reinterpret_cast<u32x4_t*>(&lds[buf][0][r * LROW + kc]) = ((st.a_ok >> i) & 1u) ? st.a[i] : zero;
            *reinterpret_cast<u32x4_t*>(&lds[buf][1][r * LROW + kc]) = st.b[i];
        }
    };

    using Acc = typename std::conditional<OP == OP_I8, i32x16_t, f32x16_t>::type;
    Acc acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = Acc{};

    const int a_off = (wm * 128 + (lane & 31)) * LROW + 16 * (lane >> 5);
    const int b_off = (wn * 128 + (lane & 31)) * LROW + 16 * (lane >> 5);

    // One 128-deep k tile from LDS buffer `buf`: four 32-deep k steps, the
    // operand fragments of step kk+1 read while the 16 MFMAs of step kk run.
    auto compute = [&](int buf) {
        const uint8_t* la = &lds[buf][0][a_off];
        const uint8_t* lb = &lds[buf][1][b_off];
        u32x4_t fa[2][4], fb[2][4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            fa[0][i] = *reinterpret_cast<const u32x4_t*>(la + i * 32 * LROW);
            fb[0][i] = *reinterpret_cast<const u32x4_t*>(lb + i * 32 * LROW);
        }
#pragma unroll
        for (int kk = 0; kk < BK / 32; ++kk) {
            const int cur = kk & 1;
            if (kk + 1 < BK / 32) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    fa[cur ^ 1][i] = *reinterpret_cast<const u32x4_t*>(la + i * 32 * LROW + (kk + 1) * 32);
                    fb[cur ^ 1][i] = *reinterpret_cast<const u32x4_t*>(lb + i * 32 * LROW + (kk + 1) * 32);
                }
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    // B^T fragment as the MFMA's row operand, A as its
                    // column operand: the accumulator is the tile transposed,
                    // so each lane ends up with four adjacent C columns
                    if constexpr (OP == OP_I8) {
                        acc[i][j] = mfma_i8_32x32x32(fb[cur][j], fa[cur][i], acc[i][j]);
                    } else {
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_fp8_fp8(
                            __builtin_bit_cast(long, u32x2_t{fb[cur][j][0], fb[cur][j][1]}),
                            __builtin_bit_cast(long, u32x2_t{fa[cur][i][0], fa[cur][i][1]}), acc[i][j], 0, 0, 0);
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_fp8_fp8(
                            __builtin_bit_cast(long, u32x2_t{fb[cur][j][2], fb[cur][j][3]}),
                            __builtin_bit_cast(long, u32x2_t{fa[cur][i][2], fa[cur][i][3]}), acc[i][j], 0, 0, 0);
                    }
                }
        }
    };

    // One k tile in flight in registers while the previous one is consumed
    // from LDS (a second register stage would not fit beside the 256
    // accumulator registers).
    const int nk = p.Kp / BK;
    Stage st;
    load_stage(st, 0);
    store_stage(st, 0);
    __syncthreads();
    for (int kt = 0; kt + 1 < nk; ++kt) {
        const int buf = kt & 1;
        load_stage(st, kt + 1);
        compute(buf);
        store_stage(st, buf ^ 1);
        __syncthreads();
    }
    compute((nk - 1) & 1);

    gemm8_epilogue<OP, EPI>(p, acc, m0, n0, wm, wn, lane);
}

// ---------------------------------------------------------------------------
// int8 kernel with an LDS-DMA pipeline (W8A8; the default int8 path).
//
// Same 256x256 tile, waves and MFMA as gemm8_kernel, but operands move
// global -> LDS with global_load_lds_dwordx4 (no register staging) through
// DS_STAGES buffers of 64-byte k steps held in dynamic LDS (32 KiB each).
// A stage's buffer is refilled, DS_STAGES stages ahead, as soon as every
// wave has read its fragments into registers, so DS_STAGES - 1 stages are
// in flight while one is multiplied.  The per-stage rendezvous is an
// explicit `s_waitcnt vmcnt` on this wave's older DMAs plus `s_barrier` (the
// fence of __syncthreads would drain every DMA in flight).  Fragments of the
// next 32-deep k step are read from LDS while the MFMAs of the current one
// run.  Stages past the last k tile still issue their DMA, re-reading the
// last tile into a buffer nothing reads again, so every wave always has the
// same number of DMAs outstanding and the wait counts are constants.  The
// tile's 256 row and 256 column scales are DMA'd into LDS ahead of the first
// stage, so the epilogue reads them without a global round trip.
//
// LDS layout per buffer and operand: 256 rows x 64 bytes, 16-byte chunk c of
// row r stored in slot c ^ ((r >> 2) & 3); the 32 rows one MFMA operand
// read touches then cover every bank once per phase of the 128-bit read.
// gfx950 serves a 64-lane ds_read_b128 in four phases of 16 lanes: lane
// bit 5 and the parity of lane bits 2..4 pick the phase (lane quads
// {0,3,5,6}, {1,2,4,7} and the same + 8), over 64 banks of 4 bytes; a
// phase is conflict-free when its 16 lanes cover 16 distinct 16-byte bank
// groups.  (Measured with reads of known addresses: a pair of lanes on
// one bank group costs a cycle exactly when both are in the same phase.)
// Rows past M read row M-1 and k past K reads the row's last 16 bytes: int8
// codes times the zero-padded B contribute nothing, and those rows are
// never stored.
// ---------------------------------------------------------------------------
constexpr int DS_BK = 64;                     // k bytes per stage
constexpr int DS_STAGES = 4;                  // LDS buffers (default)
constexpr int DS_OP_BYTES = BM * DS_BK;       // one operand of one stage (16 KiB)
constexpr int DS_SCALE_BYTES = (BM + BN) * 4;                 // int8 scales of one tile

#define LHQ_LDS_AS __attribute__((address_space(3)))

// One output tile of BM rows x 64*JB columns (JB = 4: the full 256x256
// tile; JB = 2: a 256x128 half tile) starting at (m0, n0), with the LDS of
// the calling workgroup.  acc is the caller's (one set of accumulator
// registers for both tile widths; a half tile uses blocks j < 2).  Returns
// with every LDS access of the tile complete in this wave (the caller
// separates tiles with a barrier).
template <int EPI, int STAGES, int JB>
__device__ __forceinline__ void dma_tile(const Gemm8Args& p, uint8_t* ds_lds, int m0, int n0,
                                         i32x16_t (&acc)[4][4]) {
    constexpr int DPS = 4 + JB;  // DMAs per wave per stage: 4 of A, JB of B
    constexpr int NT = 4 * JB;   // MFMAs per 32-deep k step
    static_assert(STAGES >= 3 && DPS * (STAGES - 2) <= 63, "vmcnt range");
    static_assert(STAGES * 2 * DS_OP_BYTES + DS_SCALE_BYTES <= 160 * 1024, "LDS");
    static_assert(4 * 32 * STAGED_PITCH <= STAGES * 2 * DS_OP_BYTES, "epilogue staging fits the stages");
    auto stage_buf = [&](int u) { return ds_lds + u * 2 * DS_OP_BYTES; };
    float* const lds_scales = reinterpret_cast<float*>(ds_lds + STAGES * 2 * DS_OP_BYTES);

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;

    // DMA: wave w moves A chunks c = (4w + i)*64 + lane (i < 4) and B chunks
    // c = (JB*w + i)*64 + lane (i < JB): row r = c >> 2, LDS slot c & 3,
    // global chunk (c & 3) ^ ((r >> 2) & 3).
    uint32_t a_row[4], b_src[JB];
    int kca[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int c = (4 * wave + i) * 64 + lane;
        const int r = c >> 2;
        kca[i] = ((c & 3) ^ ((r >> 2) & 3)) * 16;
        a_row[i] = static_cast<uint32_t>(min(m0 + r, p.M - 1)) * static_cast<uint32_t>(p.K);
    }
#pragma unroll
    for (int i = 0; i < JB; ++i) {
        const int c = (JB * wave + i) * 64 + lane;
        const int r = c >> 2;
        b_src[i] = static_cast<uint32_t>(n0 + r) * static_cast<uint32_t>(p.Kp) +
                   static_cast<uint32_t>(((c & 3) ^ ((r >> 2) & 3)) * 16);
    }
    const int nk = p.Kp / DS_BK;
    // DMA d (0..DPS-1) of stage s into buf: A and B chunk sets alternate
    // while both last (d < 2*JB), then the remaining A sets
    auto dma = [&](uint8_t* buf, int s, int d) {
        const int k0 = min(s, nk - 1) * DS_BK;
        const bool is_b = d < 2 * JB && (d & 1);
        const int i = d < 2 * JB ? d >> 1 : d - JB;
        if (!is_b) {
            // k past K: the row's last in-range 16 bytes (their product with
            // the zero-padded B is zero)
            const uint32_t ka = static_cast<uint32_t>(min(k0 + kca[i], p.K - 16));
            __builtin_amdgcn_global_load_lds(p.A + (a_row[i] + ka), (LHQ_LDS_AS void*)(buf + (4 * wave + i) * 1024),
                                             16, 0, 0);
        } else {
            __builtin_amdgcn_global_load_lds(p.Bt + (b_src[i] + static_cast<uint32_t>(k0)),
                                             (LHQ_LDS_AS void*)(buf + DS_OP_BYTES + (JB * wave + i) * 1024), 16, 0, 0);
        }
    };
    auto issue = [&](uint8_t* buf, int s) {
#pragma unroll
        for (int d = 0; d < DPS; ++d) dma(buf, s, d);
    };

#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < JB; ++j) acc[i][j] = i32x16_t{};

    // operand fragments: row (lane & 31) of each 32-row block, k chunk
    // 2*kk + (lane >> 5), swizzled by the row's (r >> 2) & 3
    const int swz = ((lane & 31) >> 2) & 3;
    const int a_base = (wm * 128 + (lane & 31)) * DS_BK;
    const int b_base = DS_OP_BYTES + (wn * 32 * JB + (lane & 31)) * DS_BK;
    using Frag = u32x4_t[4 + JB];  // [0..3]: A blocks i, [4..]: B blocks j
    // fragment x (A block x for x < 4, B block x - 4 otherwise) of k step kk
    auto read = [&](const uint8_t* buf, int kk, Frag& f, int x) {
        const int off = (((2 * kk + (lane >> 5)) ^ swz) * 16);
        const int base = x < 4 ? a_base + x * 32 * DS_BK : b_base + (x - 4) * 32 * DS_BK;
        f[x] = *reinterpret_cast<const u32x4_t*>(buf + base + off);
    };
    // MFMA t (0..NT-1) of one k step: block (t / JB, t % JB)
    auto mfma = [&](const Frag& f, int t) {
        const int i = t / JB, j = t % JB;
        acc[i][j] = mfma_i8_32x32x32(f[4 + j], f[i], acc[i][j]);
    };
    // Rendezvous: this wave's DMA for the next stage has landed (the
    // STAGES - 2 younger stages may still be in flight), its own LDS reads
    // are done, and every wave got this far, so all reads of the current
    // stage's buffer are complete and the buffer can take the DMA STAGES
    // stages ahead.
    auto rendezvous = [&]() {
        asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(DPS * (STAGES - 2)) : "memory");
    };

    // One stage: fragments of its first k step are in f0 on entry.  The
    // MFMAs are issued with LDS reads and DMAs between them, so the matrix
    // pipe always has work queued while those issue:
    //   first k step:  MFMA t, then read fragment t of the second k step
    //                  (t < 4 + JB);
    //   rendezvous;
    //   second k step: MFMA t, then the next of these 2*(4 + JB) operations:
    //                  the next stage's first-k-step fragment reads, then
    //                  this stage's DMAs (one per MFMA for the full tile).
    // Each k step starts with an MFMA on fragments read long before, so the
    // compiler's wait for them (which drains every LDS read in flight) comes
    // before the next reads are issued.  sched_barrier pins the order.
    constexpr int NOPS = 2 * DPS;
    Frag f0, f1;
    auto step = [&](uint8_t* cur, const uint8_t* next, int s) {
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            mfma(f0, t);
            if (t < 4 + JB) read(cur, 1, f1, t);
            __builtin_amdgcn_sched_barrier(0);
        }
        rendezvous();
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            mfma(f1, t);
#pragma unroll
            for (int o = t * NOPS / NT; o < (t + 1) * NOPS / NT; ++o) {
                if (o < 4 + JB)
                    read(next, 0, f0, o);
                else
                    dma(cur, s + STAGES, o - (4 + JB));
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    // The tile's scales go to LDS first (wave w: rows / columns 64w..64w+63,
    // clamped); the wait for stage 0 below also covers them.
    if constexpr (EPI != EPI_I32) {
        const int r = min(m0 + 64 * wave + lane, p.M - 1), c = min(n0 + 64 * wave + lane, p.N - 1);
        __builtin_amdgcn_global_load_lds(p.As + r, (LHQ_LDS_AS void*)(lds_scales + 64 * wave), 4, 0, 0);
        __builtin_amdgcn_global_load_lds(p.Bs + c, (LHQ_LDS_AS void*)(lds_scales + BM + 64 * wave), 4, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < STAGES; ++u) issue(stage_buf(u), u);
    // stage 0 landed everywhere
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(DPS * (STAGES - 1)) : "memory");
#pragma unroll
    for (int x = 0; x < 4 + JB; ++x) read(stage_buf(0), 0, f0, x);
    for (int s = 0; s < nk; s += STAGES) {
#pragma unroll
        for (int u = 0; u < STAGES; ++u)
            if (u == 0 || s + u < nk) step(stage_buf(u), stage_buf((u + 1) % STAGES), s + u);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    // every wave's DMAs have landed and every wave is done with the stage
    // buffers: the epilogue may reuse them
    __syncthreads();
    uint8_t* const area = ds_lds + wave * 32 * STAGED_PITCH;
    if (m0 + BM <= p.M && n0 + 64 * JB <= p.N && p.N % 8 == 0 && p.c_vec)
        gemm8_store_staged<EPI, false, JB>(p, acc, m0, n0, wm, wn, lane, lds_scales, area);
    else
        gemm8_store_staged<EPI, true, JB>(p, acc, m0, n0, wm, wn, lane, lds_scales, area);
}

// The same tile on v_mfma_i32_16x16x64_i8.  Each wave's 128 x 64*JB
// quadrant is 8 x 2JB blocks of 16x16 (4 accumulator registers each, the
// same 256 in all); a 64-byte k stage is ONE MFMA per block.  DMA pipeline
// and LDS layout are dma_tile's, with chunk c of row r in slot
// c ^ ((r >> 2) & 2).  Fragment of 16-row block x: row (lane & 15), global
// k chunk (lane >> 4), i.e. LDS slot (lane >> 4) ^ ((row >> 2) & 2).  Lane
// l of quad q = l >> 2 reads bank group 4(l & 3) + slot with slot
// (q >> 2) ^ (q & 2): the four quads of every read phase take four distinct
// slots, so the read is conflict-free.  dma_tile's swizzle c ^ ((r >> 2) & 3) gives this
// read a two-way conflict in every phase (quads 0 and 5 on one slot, 3
// and 6 on another): 8 LDS cycles per read instead of 4.  B is the MFMA's first operand, so lane l of block
// (i, j) holds C row 16i + (l & 15), columns 16j + 4(l >> 4) ..+3.
// Stage s (its fragments fa / fb in registers on entry):
//   rendezvous: stage s+1 landed (this wave's DMAs; s+2, s+3 may still be
//     in flight), this wave's reads of stage s's buffer done, every wave
//     here (the buffer is free for stage s + STAGES);
//   block rows 0..3, all columns, one MFMA per block; after row i the
//     next stage's A fragment of row i (read in place);
//   block rows 4..7 column by column; after column j the next stage's B
//     fragment of column j, after the last column the A fragments of rows
//     4..7;
//   the DMAs of stage s + STAGES spread over the whole stage, one every
//     8*NB / DPS MFMAs.  Issued back to back after the stage's first eight
//     MFMAs they measured slower (M=4096: 212.5 against 206.7 us, zero
//     operands 177 against 166 us; M=2048: 114 against 108.7 us): a wave
//     issues in order, so a memory instruction that cannot issue holds
//     back the MFMAs behind it.
// Register-only, on random int8 operands, this instruction in turn over
// the accumulators sustains ~12% more than the 32x32x32 form (a higher
// clock under the power limit).
template <int EPI, int JB>
__device__ __forceinline__ void dma_tile_m16(const Gemm8Args& p, uint8_t* ds_lds, int m0, int n0,
                                             i32x4_t (&acc)[8][8]) {
    constexpr int STAGES = 4;
    constexpr int DPS = 4 + JB;  // DMAs per wave per stage: 4 of A, JB of B
    constexpr int NB = 2 * JB;   // 16-column blocks per wave
    static_assert(DPS * (STAGES - 2) <= 63, "vmcnt range");
    static_assert(STAGES * 2 * DS_OP_BYTES + DS_SCALE_BYTES <= 160 * 1024, "LDS");
    static_assert(4 * 32 * STAGED_PITCH <= STAGES * 2 * DS_OP_BYTES, "epilogue staging fits the stages");
    auto stage_buf = [&](int u) { return ds_lds + u * 2 * DS_OP_BYTES; };
    float* const lds_scales = reinterpret_cast<float*>(ds_lds + STAGES * 2 * DS_OP_BYTES);

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;

    uint32_t a_row[4], b_src[JB];
    int kca[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int c = (4 * wave + i) * 64 + lane;
        const int r = c >> 2;
        kca[i] = ((c & 3) ^ ((r >> 2) & 2)) * 16;
        a_row[i] = static_cast<uint32_t>(min(m0 + r, p.M - 1)) * static_cast<uint32_t>(p.K);
    }
#pragma unroll
    for (int i = 0; i < JB; ++i) {
        const int c = (JB * wave + i) * 64 + lane;
        const int r = c >> 2;
        b_src[i] = static_cast<uint32_t>(n0 + r) * static_cast<uint32_t>(p.Kp) +
                   static_cast<uint32_t>(((c & 3) ^ ((r >> 2) & 2)) * 16);
    }
    const int nk = p.Kp / DS_BK;
    // stages past the last reload the last one (no branch in the MFMA
    // stream); they land in buffers no later stage reads
    auto dma = [&](uint8_t* buf, int s, int d) {
        const int k0 = min(s, nk - 1) * DS_BK;
        const bool is_b = d < 2 * JB && (d & 1);
        const int i = d < 2 * JB ? d >> 1 : d - JB;
        if (!is_b) {
            const uint32_t ka = static_cast<uint32_t>(min(k0 + kca[i], p.K - 16));
            __builtin_amdgcn_global_load_lds(p.A + (a_row[i] + ka), (LHQ_LDS_AS void*)(buf + (4 * wave + i) * 1024),
                                             16, 0, 0);
        } else {
            __builtin_amdgcn_global_load_lds(p.Bt + (b_src[i] + static_cast<uint32_t>(k0)),
                                             (LHQ_LDS_AS void*)(buf + DS_OP_BYTES + (JB * wave + i) * 1024), 16, 0, 0);
        }
    };

#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j) acc[i][j] = i32x4_t{};

    const int r16 = lane & 15;
    const int off = ((lane >> 4) ^ ((r16 >> 2) & 2)) * 16;
    const int a_base = (wm * 128 + r16) * DS_BK + off;
    const int b_base = DS_OP_BYTES + (wn * 32 * JB + r16) * DS_BK + off;
    auto rd_a = [&](const uint8_t* buf, int x) {
        return *reinterpret_cast<const u32x4_t*>(buf + a_base + x * 16 * DS_BK);
    };
    auto rd_b = [&](const uint8_t* buf, int x) {
        return *reinterpret_cast<const u32x4_t*>(buf + b_base + x * 16 * DS_BK);
    };
    u32x4_t fa[8], fb[NB];
    auto mma = [&](int i, int j) { acc[i][j] = mfma_i8_16x16x64(fb[j], fa[i], acc[i][j]); };

    if constexpr (EPI != EPI_I32) {
        const int r = min(m0 + 64 * wave + lane, p.M - 1), c = min(n0 + 64 * wave + lane, p.N - 1);
        __builtin_amdgcn_global_load_lds(p.As + r, (LHQ_LDS_AS void*)(lds_scales + 64 * wave), 4, 0, 0);
        __builtin_amdgcn_global_load_lds(p.Bs + c, (LHQ_LDS_AS void*)(lds_scales + BM + 64 * wave), 4, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < STAGES; ++u)
#pragma unroll
        for (int d = 0; d < DPS; ++d) dma(stage_buf(u), u, d);
    // stage 0 (and the scales) landed everywhere
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(DPS * (STAGES - 1)) : "memory");
#pragma unroll
    for (int x = 0; x < 8; ++x) fa[x] = rd_a(stage_buf(0), x);
#pragma unroll
    for (int x = 0; x < NB; ++x) fb[x] = rd_b(stage_buf(0), x);
    auto step = [&](uint8_t* cur, const uint8_t* nxt, int s) {
        asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(DPS * (STAGES - 2)) : "memory");
        // MFMA t of the stage (issue order) is followed by DMA t / SP when
        // t % SP == SP / 2: one DMA every SP MFMAs over the whole stage
        constexpr int SP = 8 * NB / DPS;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < NB; ++j) {
                mma(i, j);
                const int t = i * NB + j;
                if (t % SP == SP / 2 && t / SP < DPS) dma(cur, s + STAGES, t / SP);
                if (j == NB - 1) fa[i] = rd_a(nxt, i);
                __builtin_amdgcn_sched_barrier(0);
            }
#pragma unroll
        for (int j = 0; j < NB; ++j)
#pragma unroll
            for (int i = 4; i < 8; ++i) {
                mma(i, j);
                const int t = 4 * NB + 4 * j + (i - 4);
                if (t % SP == SP / 2 && t / SP < DPS) dma(cur, s + STAGES, t / SP);
                if (i == 7) fb[j] = rd_b(nxt, j);
                if (j == NB - 1) fa[i] = rd_a(nxt, i);
                __builtin_amdgcn_sched_barrier(0);
            }
    };
    for (int s = 0; s < nk; s += STAGES) {
#pragma unroll
        for (int u = 0; u < STAGES; ++u)
            if (u == 0 || s + u < nk) step(stage_buf(u), stage_buf((u + 1) % STAGES), s + u);
    }
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
    // every wave's DMAs have landed and every wave is done with the stage
    // buffers: the epilogue may reuse them
    __syncthreads();
    uint8_t* const area = ds_lds + wave * 32 * STAGED_PITCH;
    if (m0 + BM <= p.M && n0 + 64 * JB <= p.N && p.N % 8 == 0 && p.c_vec)
        gemm8_store_staged<EPI, false, JB, false, i32x4_t, 8, 8>(p, acc, m0, n0, wm, wn, lane, lds_scales, area);
    else
        gemm8_store_staged<EPI, true, JB, false, i32x4_t, 8, 8>(p, acc, m0, n0, wm, wn, lane, lds_scales, area);
}

// The kernel.  A plain launch has one workgroup per tile (gridDim.x ==
// tiles), in tile_of's order.  A persistent launch has G = gridDim.x < tiles
// workgroups, one per CU: R = tiles / G rounds of full tiles, then the
// rem = tiles - R*G tiles left split into 256x128 halves, one per workgroup
// (the launcher requires 2*rem <= G and G % 8 == 0).  At M=4096, N=14336
// that is 896 tiles = 3 rounds + 128 tiles: 3.5 tiles of work per CU instead
// of 4 rounds with the last one half empty.  Persistent full tiles keep
// tile_of's locality: XCD x (workgroups x, x+8, ...) walks the contiguous id
// range x*R*G/8 .. (x+1)*R*G/8, G/8 tiles per round.
template <int EPI, int STAGES, bool M16>
__global__ __launch_bounds__(NTHREADS) void gemm8_dma_kernel(Gemm8Args p) {
    // Dynamic LDS: the compiler does not see the DMA as a store into it, so
    // it may neither assume its contents nor insert its own waits for it;
    // the rendezvous inside the tile orders every access.
    extern __shared__ __attribute__((aligned(1024))) uint8_t ds_lds[];
    const int G = gridDim.x, b = blockIdx.x;
    const int total = p.tiles_m * p.tiles_n;
    const int R = total / G, rem = total - R * G;
    const int per_xcd = G / 8, xcd = b % 8, slot = b / 8;
    // (each call site names its tile width: a shared helper taking the width
    // at run time is not inlined, and the accumulators then live in scratch)
    typename std::conditional<M16, i32x4_t[8][8], i32x16_t[4][4]>::type acc;
    if constexpr (EPI != EPI_BF16) {
        // fp32 / int32 outputs keep one tile per workgroup: their epilogues
        // need more registers than a persistent loop leaves without spills.
        // A launch of twice the tiles: every workgroup one 256 x 128 half
        // tile
        int tm, tn;
        if (G == 2 * total) {
            tile_of_id(b >> 1, p, tm, tn);
            if constexpr (M16) dma_tile_m16<EPI, 2>(p, ds_lds, tm * BM, tn * BN + (b & 1) * (BN / 2), acc);
            else dma_tile<EPI, STAGES, 2>(p, ds_lds, tm * BM, tn * BN + (b & 1) * (BN / 2), acc);
            return;
        }
        tile_of(b, p, tm, tn);
        if constexpr (M16) dma_tile_m16<EPI, 4>(p, ds_lds, tm * BM, tn * BN, acc);
        else dma_tile<EPI, STAGES, 4>(p, ds_lds, tm * BM, tn * BN, acc);
        return;
    }
    for (int r = 0; r < R; ++r) {
        int tm, tn;
        if (G == total)
            tile_of(b, p, tm, tn);
        else
            tile_of_id(xcd * R * per_xcd + r * per_xcd + slot, p, tm, tn);
        if (r > 0) __syncthreads();  // the previous epilogue's LDS reads are done
        if constexpr (M16) dma_tile_m16<EPI, 4>(p, ds_lds, tm * BM, tn * BN, acc);
        else dma_tile<EPI, STAGES, 4>(p, ds_lds, tm * BM, tn * BN, acc);
    }
    if (b < 2 * rem) {
        int tm, tn;
        tile_of_id(R * G + (b >> 1), p, tm, tn);
        __syncthreads();
        if constexpr (M16) dma_tile_m16<EPI, 2>(p, ds_lds, tm * BM, tn * BN + (b & 1) * (BN / 2), acc);
        else dma_tile<EPI, STAGES, 2>(p, ds_lds, tm * BM, tn * BN + (b & 1) * (BN / 2), acc);
    }
}

// ---------------------------------------------------------------------------
// FP8 (e4m3) kernel on the LDS-DMA pipeline: gemm_fp8_e4m3
// (gemm_quant.cpp:87-104) with fp32 accumulation on gfx950's
// v_mfma_scale_f32_32x32x64_f8f6f4.  Same tile, waves, buffers, swizzle and
// DMA schedule as the int8 tile above; a stage's 64 k bytes are ONE MFMA per
// 32x32 block instead of two: a lane's two 16-byte fragments of the stage
// (k chunks (lane >> 5) and 2 + (lane >> 5)) form its 32-byte operand.  The
// instruction assigns k to lanes differently, but A and B are read with the
// same lane -> k mapping, so the 64 products of a block are the same ones.
// The whole next stage is read into the fragment registers in place, each
// fragment as soon as the current stage's last MFMA on it has issued (A
// block i after block row i, B block j in the last row), so one register set
// serves; the rendezvous opens each stage (the next stage has landed, every
// wave has read the current buffer, which then takes its DMA STAGES stages
// ahead).  Requires K % 128 == 0: no padded k reaches the MFMA (a padded A
// byte could be the NaN code, and NaN times the zero padding of B is NaN).
// Rows past M read row M-1; those rows are never stored.
// ---------------------------------------------------------------------------
// JB: 32-column blocks per wave (4: a 256x256 tile; 2: a 256x128 half tile,
// with JB B DMAs per wave and stage instead of 4).
template <int STAGES, int JB = 4>
__device__ __forceinline__ void dma_tile_fp8(const Gemm8Args& p, uint8_t* ds_lds, int m0, int n0,
                                             f32x16_t (&acc)[4][4]) {
    constexpr int DPS = 4 + JB;  // DMAs per wave per stage: 4 of A, JB of B
    static_assert(JB == 4 || JB == 2, "whole or half tiles");
    static_assert(STAGES >= 3 && DPS * (STAGES - 2) <= 63, "vmcnt range");
    auto stage_buf = [&](int u) { return ds_lds + u * 2 * DS_OP_BYTES; };
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    uint32_t a_row[4], b_src[JB];
    int kca[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int c = (4 * wave + i) * 64 + lane;
        const int r = c >> 2;
        kca[i] = ((c & 3) ^ ((r >> 2) & 3)) * 16;
        a_row[i] = static_cast<uint32_t>(min(m0 + r, p.M - 1)) * static_cast<uint32_t>(p.K);
    }
    // B rows n0 .. n0 + 64 JB - 1 (< Np: a half tile is the first or second
    // half of a whole one)
#pragma unroll
    for (int i = 0; i < JB; ++i) {
        const int c = (JB * wave + i) * 64 + lane;
        const int r = c >> 2;
        b_src[i] = static_cast<uint32_t>(n0 + r) * static_cast<uint32_t>(p.Kp) +
                   static_cast<uint32_t>(((c & 3) ^ ((r >> 2) & 3)) * 16);
    }
    const int nk = p.Kp / DS_BK;
    // DMA d of stage s (clamped to the last stage) into buf: A and B
    // alternate while both last, then the rest of A
    auto dma = [&](uint8_t* buf, int s, int d) {
        const uint32_t k0 = static_cast<uint32_t>(min(s, nk - 1) * DS_BK);
        const bool is_b = d < 2 * JB && (d & 1);
        const int i = d < 2 * JB ? d >> 1 : d - JB;
        if (!is_b)
            __builtin_amdgcn_global_load_lds(p.A + (a_row[i] + k0 + static_cast<uint32_t>(kca[i])),
                                             (LHQ_LDS_AS void*)(buf + (4 * wave + i) * 1024), 16, 0, 0);
        else
            __builtin_amdgcn_global_load_lds(p.Bt + (b_src[i] + k0),
                                             (LHQ_LDS_AS void*)(buf + DS_OP_BYTES + (JB * wave + i) * 1024), 16, 0,
                                             0);
    };
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x16_t{};

    const int swz = ((lane & 31) >> 2) & 3;
    const int a_base = (wm * 128 + (lane & 31)) * DS_BK;
    const int b_base = DS_OP_BYTES + (wn * 32 * JB + (lane & 31)) * DS_BK;
    u32x4_t f[4 + JB][2];  // [A blocks 0..3, B blocks 0..JB-1][k half]
    auto read = [&](const uint8_t* buf, int x) {
        const int base = x < 4 ? a_base + x * 32 * DS_BK : b_base + (x - 4) * 32 * DS_BK;
#pragma unroll
        for (int kk = 0; kk < 2; ++kk)
            f[x][kk] = *reinterpret_cast<const u32x4_t*>(buf + base + (((2 * kk + (lane >> 5)) ^ swz) * 16));
    };
    auto rendezvous = [&]() {
        asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(DPS * (STAGES - 2)) : "memory");
    };
    // stage s from buffer cur; fragments already in f; next: the buffer of s + 1
    auto step = [&](uint8_t* cur, const uint8_t* next, int s) {
        rendezvous();
#pragma unroll
        for (int t = 0; t < 4 * JB; ++t) {
            const int i = t / JB, j = t % JB;
            acc[i][j] = mfma_fp8_32x32x64(f[4 + j][0], f[4 + j][1], f[i][0], f[i][1], acc[i][j]);
            if (t < DPS) dma(cur, s + STAGES, t);
            if (j == JB - 1 && i < 3) read(next, i);  // A block i is done
            if (i == 3) {
                read(next, 4 + j);                    // B block j is done
                if (j == JB - 1) read(next, 3);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };
#pragma unroll
    for (int u = 0; u < STAGES; ++u)
#pragma unroll
        for (int d = 0; d < DPS; ++d) dma(stage_buf(u), u, d);
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(DPS * (STAGES - 1)) : "memory");
#pragma unroll
    for (int x = 0; x < 4 + JB; ++x) read(stage_buf(0), x);
    for (int s = 0; s < nk; s += STAGES) {
#pragma unroll
        for (int u = 0; u < STAGES; ++u)
            if (u == 0 || s + u < nk) step(stage_buf(u), stage_buf((u + 1) % STAGES), s + u);
    }
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
    // every wave's DMAs have landed and no wave reads the stage buffers again:
    // the epilogue stages its accumulators there
    __syncthreads();
    uint8_t* const area = ds_lds + wave * 32 * STAGED_PITCH;
    static_assert(4 * 32 * STAGED_PITCH <= STAGES * 2 * DS_OP_BYTES, "epilogue staging fits the stages");
    if (m0 + BM <= p.M && n0 + 64 * JB <= p.N && p.N % 8 == 0 && p.c_vec)
        gemm8_store_staged<EPI_F32, false, JB, true>(p, acc, m0, n0, wm, wn, lane, nullptr, area);
    else
        gemm8_store_staged<EPI_F32, true, JB, true>(p, acc, m0, n0, wm, wn, lane, nullptr, area);
}

// One tile per workgroup; a launch of twice the tiles: every workgroup one
// 256 x 128 half tile.
template <int STAGES>
__global__ __launch_bounds__(NTHREADS) void gemm8_fp8_dma_kernel(Gemm8Args p) {
    extern __shared__ __attribute__((aligned(1024))) uint8_t ds_lds[];
    const int total = p.tiles_m * p.tiles_n;
    f32x16_t acc[4][4];
    int tm, tn;
    if (static_cast<int>(gridDim.x) == 2 * total) {
        tile_of_id(blockIdx.x >> 1, p, tm, tn);
        dma_tile_fp8<STAGES, 2>(p, ds_lds, tm * BM, tn * BN + (blockIdx.x & 1) * (BN / 2), acc);
        return;
    }
    tile_of(blockIdx.x, p, tm, tn);
    dma_tile_fp8<STAGES>(p, ds_lds, tm * BM, tn * BN, acc);
}

// ---------------------------------------------------------------------------
// Small- and mid-size int8 kernel (W8A8 with M <= kMidMaxM: the M = 1 GEMV
// of config 1 and batched decode).  There the 256x256 tile kernel runs
// ceil(N/256) workgroups -- 56 at N = 14336, under a quarter of the CUs --
// each walking all of K, and the rows past M are MFMA work for nothing.  Here a 64 W-thread workgroup owns an
// output block of RB 16-row blocks by T 16-column tiles and its W waves
// split K; per 64-deep k step a lane loads 16 contiguous k bytes of each of
// its T B^T columns and RB A rows (1 KiB loads per wave), and RB * T
// v_mfma_i32_16x16x64_i8 accumulate the blocks (rows past M read row M-1,
// their outputs are not stored; k past K reads the row's last 16 bytes, B^T
// is zero there).  BATCH k steps are loaded before they are consumed.
// Waves 1.. hand their int32 blocks to wave 0 through LDS, which adds them
// (integer addition: the reference's accumulator exactly) and writes the
// reference's epilogue (C += ((alpha * a_s) * b_s) * acc, no fused
// multiply-add).
// ---------------------------------------------------------------------------
constexpr int kMidMaxM = 32;
constexpr int kMidMaxFp8M = 32;

// RB 16-row blocks by T 16-column tiles per workgroup, W waves splitting K,
// BATCH k steps loaded before they are consumed, MINW workgroups per CU in
// the register budget
// OP_FP8 (gemm_fp8_e4m3, K % 128 == 0): fp32 accumulators, each 16-byte
// operand feeding two v_mfma_f32_16x16x32_fp8_fp8 (its low and high 8
// bytes), the waves' partial blocks added in wave order, and the tile
// kernel's fp8 epilogue.
template <int EPI, int RB = 4, int T = 4, int W = 4, int BATCH = 4, int MINW = 2, int OP = OP_I8>
__global__ __launch_bounds__(64 * W, MINW) void gemm8_mid_kernel(Gemm8Args p) {
    static_assert((W - 1) * RB * T * 64 * 16 <= 60 * 1024, "reduction area");
    static_assert(OP == OP_I8 || EPI == EPI_F32, "fp8: fp32 output");
    using Acc = typename std::conditional<OP == OP_I8, i32x4_t, f32x4_t>::type;
    __shared__ Acc red[W - 1][RB * T][64];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n0 = blockIdx.x * 16 * T, m0 = blockIdx.y * 16 * RB;
    const int kl = 16 * (lane >> 4);  // this lane's 16 k within a 64-deep step
    const int steps = p.Kp / 64;
    const int per = (steps + W - 1) / W;
    const int s0 = min(wave * per, steps), s1 = min(s0 + per, steps);
    const uint8_t* a_row[RB];
    const uint8_t* b_col[T];
    // rows past M read row M-1; columns n0 + 16 t + (lane & 15) < Np (B^T
    // rows are zero-padded to a multiple of 256 >= ceil(N / (16 T)) * 16 T)
#pragma unroll
    for (int i = 0; i < RB; ++i)
        a_row[i] = p.A + static_cast<size_t>(min(m0 + 16 * i + (lane & 15), p.M - 1)) * p.K;
#pragma unroll
    for (int t = 0; t < T; ++t) b_col[t] = p.Bt + static_cast<size_t>(n0 + 16 * t + (lane & 15)) * p.Kp;

    Acc acc[RB][T];
#pragma unroll
    for (int i = 0; i < RB; ++i)
#pragma unroll
        for (int t = 0; t < T; ++t) acc[i][t] = Acc{};
    for (int sb = s0; sb < s1; sb += BATCH) {
        u32x4_t a[BATCH][RB], b[BATCH][T];
#pragma unroll
        for (int u = 0; u < BATCH; ++u) {
            // steps past this wave's range re-read its last one (discarded)
            const int k = min(sb + u, s1 - 1) * 64 + kl;
#pragma unroll
            for (int i = 0; i < RB; ++i) a[u][i] = *reinterpret_cast<const u32x4_t*>(a_row[i] + min(k, p.K - 16));
#pragma unroll
            for (int t = 0; t < T; ++t) b[u][t] = *reinterpret_cast<const u32x4_t*>(b_col[t] + k);
        }
#pragma unroll
        for (int u = 0; u < BATCH; ++u)
            if (sb + u < s1)
#pragma unroll
                for (int i = 0; i < RB; ++i)
#pragma unroll
                    for (int t = 0; t < T; ++t) {
                        if constexpr (OP == OP_I8) {
                            acc[i][t] = mfma_i8_16x16x64(a[u][i], b[u][t], acc[i][t]);
                        } else {
                            // k 16 g .. + 7 of the step, then + 8 .. + 15, in
                            // every lane group g (A and B alike)
                            acc[i][t] = mfma_fp8_16x16x32(u32x2_t{a[u][i][0], a[u][i][1]},
                                                          u32x2_t{b[u][t][0], b[u][t][1]}, acc[i][t]);
                            acc[i][t] = mfma_fp8_16x16x32(u32x2_t{a[u][i][2], a[u][i][3]},
                                                          u32x2_t{b[u][t][2], b[u][t][3]}, acc[i][t]);
                        }
                    }
    }
    if (wave > 0) {
#pragma unroll
        for (int i = 0; i < RB; ++i)
#pragma unroll
            for (int t = 0; t < T; ++t) red[wave - 1][i * T + t][lane] = acc[i][t];
    }
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int w = 0; w < W - 1; ++w)
#pragma unroll
        for (int i = 0; i < RB; ++i)
#pragma unroll
            for (int t = 0; t < T; ++t) acc[i][t] += red[w][i * T + t][lane];

    // D element j of block (i, t) in lane l: row m0 + 16 i + 4 (l >> 4) + j,
    // column n0 + 16 t + (l & 15)
    if constexpr (OP == OP_FP8) {
        float combined = p.alpha * p.As[0];  // gemm_quant.cpp:98
        combined = combined * p.Bs[0];
        float* Cp = static_cast<float*>(p.C);
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const int c = n0 + 16 * t + (lane & 15);
            if (c >= p.N) continue;
#pragma unroll
            for (int i = 0; i < RB; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int r = m0 + 16 * i + 4 * (lane >> 4) + j;
                    if (r >= p.M) continue;
                    const size_t o = static_cast<size_t>(r) * p.N + c;
                    // apply_beta (gemm_quant.cpp:12-21), then C += rescaled
                    const float base = (p.beta == 0.0f) ? 0.0f : (p.beta == 1.0f) ? Cp[o] : Cp[o] * p.beta;
                    Cp[o] = base + combined * acc[i][t][j];
                }
        }
        return;
    }
#pragma unroll
    for (int t = 0; t < T; ++t) {
        const int c = n0 + 16 * t + (lane & 15);
        if (c >= p.N) continue;
        float bs = 0.0f;
        if constexpr (EPI != EPI_I32) bs = p.Bs[c];
#pragma unroll
        for (int i = 0; i < RB; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int r = m0 + 16 * i + 4 * (lane >> 4) + j;
                if (r >= p.M) continue;
                const size_t o = static_cast<size_t>(r) * p.N + c;
                if constexpr (EPI == EPI_I32) {
                    static_cast<int32_t*>(p.C)[o] = acc[i][t][j];
                } else {
                    float f = p.alpha * p.As[r];  // gemm_quant.cpp:44-46, left to right
                    f = f * bs;
                    f = f * static_cast<float>(acc[i][t][j]);
                    if constexpr (EPI == EPI_F32) {
                        // apply_beta (gemm_quant.cpp:12-21), then C += rescaled
                        float* Cp = static_cast<float*>(p.C);
                        const float base = (p.beta == 0.0f) ? 0.0f : (p.beta == 1.0f) ? Cp[o] : Cp[o] * p.beta;
                        Cp[o] = base + f;
                    } else {
                        static_cast<uint16_t*>(p.C)[o] = f32_to_bf16(0.0f + f);
                    }
                }
            }
    }
}

template <int EPI, int RB, int T, int W, int BATCH, int MINW, int OP = OP_I8>
void launch_mid(const Gemm8Args& p, void* stream) {
    const dim3 grid(ceil_div(p.N, 16 * T), ceil_div(p.M, 16 * RB));
    gemm8_mid_kernel<EPI, RB, T, W, BATCH, MINW, OP><<<grid, 64 * W, 0, as_stream(stream)>>>(p);
}

int env_int(const char* name, int dflt) { return tuning_knob(name, dflt); }

// Compute units of the current device (one persistent workgroup each).
int device_cus() {
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        return 0;
    return cus;
}

template <int EPI, int STAGES, bool M16>
int launch_dma(const Gemm8Args& p, int tiles, void* stream, const char* who) {
    static_assert(!M16 || STAGES == 4, "the 16x16x64 tile runs four stages");
    constexpr size_t lds = static_cast<size_t>(STAGES) * 2 * DS_OP_BYTES + DS_SCALE_BYTES;
    static const hipError_t attr =
        hipFuncSetAttribute(reinterpret_cast<const void*>(&gemm8_dma_kernel<EPI, STAGES, M16>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
    if (attr != hipSuccess)
        return set_error(LHQ_ERR_HIP, "%s: dynamic LDS attribute: %s", who, hipGetErrorString(attr));
    // Persistent launch (one workgroup per CU) when the tiles leave a
    // partial last round that splits into at most one half tile per
    // workgroup (LHQ_GEMM8_PERSIST=0 disables).  A tile takes a whole CU
    // (256 accumulator registers per wave, ~130 KiB of LDS).
    static const int persist = env_int("LHQ_GEMM8_PERSIST", 1);
    static const int cus = device_cus();
    // tiles filling at most half the CUs: every workgroup a 256 x 128 half
    // tile, twice the workgroups
    static const int halves = env_int("LHQ_GEMM8_HALVES", 1);
    if (halves && cus > 0 && 2 * tiles <= cus) {
        gemm8_dma_kernel<EPI, STAGES, M16><<<2 * tiles, NTHREADS, lds, as_stream(stream)>>>(p);
        return check_launch(who);
    }
    const int G = cus;
    const int rem = G > 0 ? tiles % G : 0;
    if (EPI == EPI_BF16 && persist && G > 0 && G % 8 == 0 && tiles > G && rem != 0 && 2 * rem <= G) {
        gemm8_dma_kernel<EPI, STAGES, M16><<<G, NTHREADS, lds, as_stream(stream)>>>(p);
        return check_launch(who);
    }
    gemm8_dma_kernel<EPI, STAGES, M16><<<tiles, NTHREADS, lds, as_stream(stream)>>>(p);
    return check_launch(who);
}

template <int STAGES>
int launch_fp8_dma(const Gemm8Args& p, int tiles, void* stream, const char* who) {
    constexpr size_t lds = static_cast<size_t>(STAGES) * 2 * DS_OP_BYTES;
    static const hipError_t attr =
        hipFuncSetAttribute(reinterpret_cast<const void*>(&gemm8_fp8_dma_kernel<STAGES>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
    if (attr != hipSuccess)
        return set_error(LHQ_ERR_HIP, "%s: dynamic LDS attribute: %s", who, hipGetErrorString(attr));
    // tiles filling at most half the CUs: every workgroup a half tile
    static const int halves = env_int("LHQ_GEMM8_HALVES", 1);
    static const int cus = device_cus();
    const int wgs = (halves && cus > 0 && 2 * tiles <= cus) ? 2 * tiles : tiles;
    gemm8_fp8_dma_kernel<STAGES><<<wgs, NTHREADS, lds, as_stream(stream)>>>(p);
    return check_launch(who);
}

template <int OP, int EPI>
int launch_gemm8(const uint8_t* A, const uint8_t* Bt, const float* As, const float* Bs, void* C, int M,
                 int N, int K, float alpha, float beta, void* stream, const char* who) {
    LHQ_REQUIRE(M >= 0 && N > 0 && K > 0, "%s: bad dims M=%d N=%d K=%d", who, M, N, K);
    LHQ_SUPPORTED(K % 16 == 0, "%s: K=%d must be a multiple of 16 (pad A and B with zeros)", who, K);
    LHQ_REQUIRE(Bt && C && (A || M == 0), "%s: null pointer", who);
    if (EPI != EPI_I32) LHQ_REQUIRE(As && Bs, "%s: null scale pointer", who);
    if (M == 0) return LHQ_OK;
    LHQ_SUPPORTED(N < (1 << 23), "%s: N=%d above 2^23 is not supported", who, N);
    LHQ_SUPPORTED(static_cast<int64_t>(M) * K < (int64_t{1} << 32) &&
                      static_cast<int64_t>(ceil_div(N, BN)) * BN * (ceil_div(K, BK) * BK) < (int64_t{1} << 32),
                  "%s: operands above 4 GiB are not supported (M=%d N=%d K=%d)", who, M, N, K);
    static const int group_m = env_int("LHQ_GEMM8_GROUP_M", 4);
    Gemm8Args p{};
    p.A = A; p.Bt = Bt; p.As = As; p.Bs = Bs; p.C = C;
    p.M = M; p.N = N; p.K = K; p.Kp = ceil_div(K, BK) * BK;
    p.tiles_m = ceil_div(M, BM);
    p.tiles_n = ceil_div(N, BN);
    p.group_m = group_m > 0 ? group_m : 4;
    p.alpha = alpha; p.beta = beta;
    p.c_vec = (reinterpret_cast<uintptr_t>(C) % 16) == 0;
    const int tiles = p.tiles_m * p.tiles_n;
    // int8: the LDS-DMA pipeline (LHQ_GEMM8_DMA=0 selects the register-
    // staged kernel); fp8: the LDS-DMA pipeline when K % 128 == 0 (no K
    // padding), else the register-staged kernel, which zeroes the K padding
    // of A before it reaches the MFMA
    static const int use_dma = env_int("LHQ_GEMM8_DMA", 1);
    static const int use_small = env_int("LHQ_GEMM8_SKINNY", 1);
    if constexpr (OP == OP_FP8) {
        // up to 32 rows (K % 128 == 0): the mid-size kernel's 32 x 32 blocks.
        // K = 4096, N = 14336 (us, whole tiles / here): M = 1 40.9 / 15.9,
        // M = 17 42.1 / 19.2, M = 32 44.2 / 22.9; a 16 x 16 block on 8 waves
        // at M <= 16 measured 15.0 / 18.1 / 21.0 at M = 1 / 8 / 16 against
        // 15.9 / 17.6 / 18.9.  Above, the tile kernel (half tiles where the
        // tiles fill at most half the CUs); 64 x 64 blocks here took 34.7 /
        // 46.4 us at M = 64 / 128
        static const int fp8_mid_max = env_int("LHQ_GEMM8_FP8_MID", kMidMaxFp8M);
        // up to 16 rows the int8 form below: 16-row blocks of one 16-column
        // tile, four waves each loading its whole K range at once (us, K =
        // 4096, N = 14336, 32 x 32 blocks -> this: M = 1 15.9 -> 13.2-13.7,
        // M = 4 16.8 -> 14.7-15.0, M = 8 17.4 -> 15.9, M = 16 18.8 -> 18.9)
        if (M <= 16 && M <= fp8_mid_max && K % BK == 0) {
            launch_mid<EPI_F32, 1, 1, 4, 16, 2, OP_FP8>(p, stream);
            return check_launch(who);
        }
        if (M <= fp8_mid_max && K % BK == 0) {
            launch_mid<EPI_F32, 2, 2, 4, 8, 2, OP_FP8>(p, stream);
            return check_launch(who);
        }
        if (use_dma && K % BK == 0) return launch_fp8_dma<DS_STAGES>(p, tiles, stream, who);
    }
    if constexpr (OP == OP_I8) {
        // up to 16 rows: 16-row blocks of one 16-column tile, four waves
        // each loading its whole K range (16 steps at K = 4096) at once.
        // Measured against eight waves of eight steps (us, K = 4096): M = 1,
        // N = 4096 (config 1) 6.45 -> 6.05; N = 14336: M = 1 14.8 -> 13.7,
        // M = 8 17.8 -> 15.7, M = 16 20.5 -> 18.3 (16 waves of four steps
        // 6.25 at config 1; two tiles on eight waves 7.74)
        if (use_small && M <= 16) {
            launch_mid<EPI, 1, 1, 4, 16, 2>(p, stream);
            return check_launch(who);
        }
        static const int mid_max = env_int("LHQ_GEMM8_MID", kMidMaxM);  // largest M for the mid-size kernel
        if (use_small && M <= mid_max) {
#ifdef LHQ_TUNING_KNOBS
            static const int mid_form = env_int("LHQ_GEMM8_MID_FORM", 0);
            switch (mid_form) {
                case 1: launch_mid<EPI, 4, 2, 4, 4, 2>(p, stream); return check_launch(who);
                case 2: launch_mid<EPI, 2, 4, 4, 4, 2>(p, stream); return check_launch(who);
                case 3: launch_mid<EPI, 2, 2, 8, 4, 2>(p, stream); return check_launch(who);
                case 4: launch_mid<EPI, 2, 4, 8, 2, 1>(p, stream); return check_launch(who);
                case 5: launch_mid<EPI, 4, 1, 4, 8, 2>(p, stream); return check_launch(who);
                case 6: launch_mid<EPI, 2, 2, 4, 8, 2>(p, stream); return check_launch(who);
                default: break;
            }
#endif
            // 32 x 32 blocks, eight k steps per batch: M = 17 19.5-19.7 us,
            // M = 32 23.2 (K = 4096, N = 14336), against 24.5 / 26.3 for 64 x
            // 64 blocks and 42.6 / 43.4 on whole tiles.  From 33 rows the tile
            // kernel's half tiles match or beat 64 x 64 blocks (M = 48: 29.4
            // here; M = 65 on half tiles 29.9, M = 64 here 32.4)
            launch_mid<EPI, 2, 2, 4, 8, 2>(p, stream);
            return check_launch(who);
        }
#ifdef LHQ_TUNING_KNOBS
        // sweep build only: the 32x32x32 tile (LHQ_GEMM8_M16=0, 3 or 4
        // stages) and the register-staged kernel (LHQ_GEMM8_DMA=0); the
        // product library compiles only the 16x16x64 tile for int8
        if (use_dma) {
            static const int m16 = env_int("LHQ_GEMM8_M16", 1);
            static const int stages = env_int("LHQ_GEMM8_STAGES", DS_STAGES);
            if (m16) return launch_dma<EPI, 4, true>(p, tiles, stream, who);
            switch (stages) {
                case 3: return launch_dma<EPI, 3, false>(p, tiles, stream, who);
                default: return launch_dma<EPI, 4, false>(p, tiles, stream, who);
            }
        }
#else
        (void)use_dma;
        return launch_dma<EPI, 4, true>(p, tiles, stream, who);
#endif
    }
#ifndef LHQ_TUNING_KNOBS
    if constexpr (OP == OP_FP8) {
#endif
        gemm8_kernel<OP, EPI><<<tiles, NTHREADS, 0, as_stream(stream)>>>(p);
        return check_launch(who);
#ifndef LHQ_TUNING_KNOBS
    }
#endif
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
