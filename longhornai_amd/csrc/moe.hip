// moe.hip -- the MoE routing around the grouped W4A16 GEMM, on gfx950:
// dispatch (a stable counting sort of the (token, slot) pairs by expert, then
// the row gather), the gate-weighted combine, and the quantized expert MLP
// (gate and up projections in one grouped launch with a SwiGLU epilogue,
// then the down projection).
//
// Reference: moe.hpp:63-102, moe.cpp:102-221 -- CPU loops over host arrays.
// Here the group table `offsets` is produced on the device and consumed by
// the grouped GEMM on the device: nothing goes back to the host between
// routing and combine.  All work is integer bookkeeping and byte moves except
// the combine's fp32 sums, which keep the reference's order and rounding.
#include "common.hpp"

namespace lhq {
namespace {

constexpr int kRankThreads = 1024;               // one workgroup ranks every slot
constexpr int kRankWaves = kRankThreads / 64;
constexpr int kMaxExperts = 512;                 // LDS: kRankWaves x kMaxExperts counters (32 KiB)
constexpr int kMaxTopK = 64;                     // the combine's per-token slot list

// Dispatch, step 1 (one workgroup of 16 waves).  Wave w owns the contiguous
// slot range [w*per, (w+1)*per) of the S = T*topk pairs, slot s = t*topk + k.
//   a) per-wave counts per expert (LDS atomics: a count does not depend on
//      order) -- moe.cpp:111-118;
//   b) offsets = exclusive scan of the per-expert totals (moe.cpp:119-123);
//      wave w's first position inside expert e = offsets[e] + the counts of
//      waves 0..w-1 for e;
//   c) each wave walks its range in order, 64 slots at a time; the lanes that
//      name one expert take consecutive positions in lane order (ballot +
//      prefix popcount), so positions follow slot order inside each expert:
//      the reference's stable placement (moe.cpp:124-139).
// Writes token_idx, slot_idx, slot_pos; an id outside [0, E) is dropped
// (slot_pos -1), and positions past offsets[E] get token_idx = slot_idx = -1.
__global__ __launch_bounds__(kRankThreads) void moe_rank_kernel(const int32_t* __restrict__ ids, int S, int topk,
                                                                int E, int32_t* __restrict__ offsets,
                                                                int32_t* __restrict__ token_idx,
                                                                int32_t* __restrict__ slot_idx,
                                                                int32_t* __restrict__ slot_pos) {
    __shared__ int32_t cnt[kRankWaves][kMaxExperts];
    __shared__ int32_t scan[kMaxExperts];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    for (int i = threadIdx.x; i < kRankWaves * kMaxExperts; i += kRankThreads) (&cnt[0][0])[i] = 0;
    __syncthreads();

    const int per = (S + kRankWaves - 1) / kRankWaves;
    const int s0 = min(S, wave * per), s1 = min(S, s0 + per);
    for (int s = s0 + lane; s < s1; s += 64) {
        const int e = ids[s];
        if (e >= 0 && e < E) atomicAdd(&cnt[wave][e], 1);
    }
    __syncthreads();

    // b) inclusive scan of the totals (Hillis-Steele; every thread runs the
    //    same number of rounds, so the barriers are uniform)
    const int e = threadIdx.x;
    int total = 0;
    if (e < E)
        for (int w = 0; w < kRankWaves; ++w) total += cnt[w][e];
    if (e < E) scan[e] = total;
    __syncthreads();
    for (int d = 1; d < E; d <<= 1) {
        const int v = (e < E && e >= d) ? scan[e - d] : 0;
        __syncthreads();
        if (e < E) scan[e] += v;
        __syncthreads();
    }
    if (e < E) {
        int run = scan[e] - total;  // exclusive
        offsets[e] = run;
        if (e == E - 1) offsets[E] = scan[e];
        for (int w = 0; w < kRankWaves; ++w) {
            const int c = cnt[w][e];
            cnt[w][e] = run;
            run += c;
        }
    }
    __syncthreads();

    // c) positions in slot order
    for (int base = s0; base < s1; base += 64) {
        const int s = base + lane;
        const bool in = s < s1;
        const int ex = in ? ids[s] : -1;
        const bool valid = in && ex >= 0 && ex < E;
        int pos = -1;
        uint64_t rem = __ballot(valid);
        while (rem) {
            const int leader = __builtin_ctzll(rem);
            const int el = __shfl(ex, leader);
            const uint64_t m = __ballot(valid && ex == el);
            const int b = cnt[wave][el];
            if (valid && ex == el) pos = b + __popcll(m & ((uint64_t{1} << lane) - 1));
            if (lane == leader) cnt[wave][el] = b + __popcll(m);
            rem &= ~m;
        }
        if (in) {
            slot_pos[s] = pos;
            if (valid) {
                token_idx[pos] = s / topk;
                slot_idx[pos] = s % topk;
            }
        }
    }
    const int placed = E > 0 ? scan[E - 1] : 0;
    for (int s = placed + static_cast<int>(threadIdx.x); s < S; s += kRankThreads) {
        token_idx[s] = -1;
        slot_idx[s] = -1;
    }
}

// Dispatch, step 2: the row copy (moe.cpp:136-137).  Workgroup (t, y) reads
// VB-byte units y*256 .. y*256+255 of token t's row once and writes them to
// each of the token's dispatched positions.
template <int VB>
struct VecOf;
template <>
struct VecOf<16> { using T = u32x4_t; };
template <>
struct VecOf<4> { using T = uint32_t; };
template <>
struct VecOf<2> { using T = uint16_t; };

template <int VB>
__global__ __launch_bounds__(256) void moe_gather_kernel(const uint8_t* __restrict__ hidden,
                                                         const int32_t* __restrict__ slot_pos,
                                                         uint8_t* __restrict__ out, int64_t row_bytes, int topk) {
    using V = typename VecOf<VB>::T;
    const int64_t t = blockIdx.x;
    const int64_t off = (static_cast<int64_t>(blockIdx.y) * 256 + threadIdx.x) * VB;
    if (off >= row_bytes) return;
    const V v = *reinterpret_cast<const V*>(hidden + t * row_bytes + off);
    for (int k = 0; k < topk; ++k) {
        const int pos = slot_pos[t * topk + k];
        if (pos >= 0) *reinterpret_cast<V*>(out + static_cast<int64_t>(pos) * row_bytes + off) = v;
    }
}

// Dispatch in one launch for at most kSmallSlots slots (decode-sized
// batches), where the two launches above cost more than their work.  Grid
// (T, row chunks) as the gather.  Every workgroup holds all S ids in LDS and
// finds the positions of its token's slots itself: slot s of expert e goes to
// position #{valid s' : (e', s') < (e, s)} in (expert, slot) order, which is
// offsets[e] + the earlier slots of e -- the placement of the two-launch path
// (moe.cpp:111-139).  Then it copies its chunk of the token's row to each of
// those positions.  Chunk 0 of each token writes its slot_pos / token_idx /
// slot_idx entries; workgroup (0, 0) writes offsets[0..E] (histogram, then a
// block scan) and the unplaced tail of token_idx / slot_idx.
constexpr int kSmallSlots = 256;

template <int VB>
__global__ __launch_bounds__(kSmallSlots) void moe_dispatch_small_kernel(
    const int32_t* __restrict__ ids, int S, int topk, int E, int32_t* __restrict__ offsets,
    int32_t* __restrict__ token_idx, int32_t* __restrict__ slot_idx, int32_t* __restrict__ slot_pos,
    const uint8_t* __restrict__ hidden, uint8_t* __restrict__ out, int64_t row_bytes) {
    using V = typename VecOf<VB>::T;
    __shared__ int32_t sid[kSmallSlots];    // expert of each slot, -1 where dropped
    __shared__ int32_t spos[kMaxTopK];      // positions of this token's slots
    __shared__ int32_t cnt[kMaxExperts];    // workgroup (0, 0): slots per expert
    __shared__ int32_t wsum[kSmallSlots / 64];
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int t = blockIdx.x;
    const int my = tid < S ? ids[tid] : -1;
    const bool valid = tid < S && my >= 0 && my < E;
    sid[tid] = valid ? my : -1;
    if (tid < topk) spos[tid] = 0;
    __syncthreads();

    for (int k = 0; k < topk; ++k) {
        const int s = t * topk + k;
        const int e = sid[s];  // the same in every lane
        if (e < 0) continue;
        const uint64_t b = __ballot(valid && (my < e || (my == e && tid < s)));
        if (lane == 0 && b) atomicAdd(&spos[k], __popcll(b));
    }
    __syncthreads();

    const int64_t off = (static_cast<int64_t>(blockIdx.y) * kSmallSlots + tid) * VB;
    if (off < row_bytes) {
        const V v = *reinterpret_cast<const V*>(hidden + static_cast<int64_t>(t) * row_bytes + off);
        for (int k = 0; k < topk; ++k)
            if (sid[t * topk + k] >= 0) *reinterpret_cast<V*>(out + static_cast<int64_t>(spos[k]) * row_bytes + off) = v;
    }
    if (blockIdx.y == 0 && tid < topk) {
        const int s = t * topk + tid;
        const bool ok = sid[s] >= 0;
        slot_pos[s] = ok ? spos[tid] : -1;
        if (ok) {
            token_idx[spos[tid]] = t;
            slot_idx[spos[tid]] = tid;
        }
    }
    if (blockIdx.x != 0 || blockIdx.y != 0) return;  // (uniform over the workgroup)

    for (int e = tid; e < kMaxExperts; e += kSmallSlots) cnt[e] = 0;
    __syncthreads();
    if (valid) atomicAdd(&cnt[my], 1);
    __syncthreads();
    // exclusive scan of cnt[0..E): thread i owns experts 2i and 2i+1
    const int a = 2 * tid < E ? cnt[2 * tid] : 0;
    const int b = 2 * tid + 1 < E ? cnt[2 * tid + 1] : 0;
    int x = a + b;
    for (int d = 1; d < 64; d <<= 1) {
        const int y = __shfl_up(x, d);
        if (lane >= d) x += y;
    }
    if (lane == 63) wsum[wave] = x;
    __syncthreads();
    for (int w = 0; w < wave; ++w) x += wsum[w];
    const int excl = x - a - b;
    if (2 * tid < E) offsets[2 * tid] = excl;
    if (2 * tid + 1 < E) offsets[2 * tid + 1] = excl + a;
    const int placed = wsum[0] + wsum[1] + wsum[2] + wsum[3];
    if (tid == 0) offsets[E] = placed;
    for (int s = placed + tid; s < S; s += kSmallSlots) {
        token_idx[s] = -1;
        slot_idx[s] = -1;
    }
}

// slot_pos from token_idx / slot_idx (the inverse of the dispatch layout):
// fill with -1, then one store per dispatched slot.
__global__ void moe_fill_kernel(int32_t* p, int64_t n, int32_t v) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}
__global__ void moe_invert_kernel(const int32_t* __restrict__ token_idx, const int32_t* __restrict__ slot_idx,
                                  int32_t* __restrict__ slot_pos, int T, int topk) {
    const int64_t s = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (s >= static_cast<int64_t>(T) * topk) return;
    const int t = token_idx[s], k = slot_idx[s];
    if (t >= 0 && t < T && k >= 0 && k < topk) slot_pos[static_cast<int64_t>(t) * topk + k] = static_cast<int32_t>(s);
}

// Combine (moe.cpp:198-221): output[t] = the sum, over t's dispatched slots
// in position order, of gate[t, k] * y[pos] -- the reference zeroes the
// output and adds one product per slot in slot order (expert-major), so a
// token's terms arrive in ascending position.  fp32, product and sum each
// rounded (contraction off), starting from +0.  Workgroup (t, y): thread 0
// sorts the token's positions into LDS, then each thread sums four
// consecutive elements per 1024-element chunk.  BF16: y bf16 (widened
// exactly); the output is bf16 (the sum rounded once) or, without Q8, the
// type of y.
// Q8 (one workgroup per token, grid.y = 1): the output row is quantized to
// int8 per token in the epilogue -- q8_quantize_per_row (quant.cpp:52-63)
// applied to the fp32 sums, which stay in LDS: max-abs (a NaN never wins,
// quant.cpp:21-28), scale = m / 127 (1 when m == 0), inv = 1 / scale,
// q = saturate-then-round-to-nearest-even(x * inv).
template <bool BF16, bool Q8>
__global__ __launch_bounds__(256) void moe_combine_kernel(const void* __restrict__ y,
                                                          const int32_t* __restrict__ slot_pos,
                                                          const float* __restrict__ gates, void* __restrict__ out,
                                                          float* __restrict__ scales, int H, int topk) {
    // hipcc contracts a * b + c into one fused multiply-add by default; the
    // reference rounds the product and the sum separately
#pragma clang fp contract(off)
    __shared__ int32_t sp[kMaxTopK];
    __shared__ float sg[kMaxTopK];
    __shared__ int ns;
    __shared__ float wmax[4];
    extern __shared__ float qrow[];  // Q8: the token's fp32 row
    const int64_t t = blockIdx.x;
    if (threadIdx.x == 0) {
        int n = 0;
        for (int k = 0; k < topk; ++k) {
            const int p = slot_pos[t * topk + k];
            if (p < 0 || p >= static_cast<int64_t>(gridDim.x) * topk) continue;  // y has T*topk rows
            const float g = gates[t * topk + k];
            int j = n++;
            while (j > 0 && sp[j - 1] > p) {
                sp[j] = sp[j - 1];
                sg[j] = sg[j - 1];
                --j;
            }
            sp[j] = p;
            sg[j] = g;
        }
        ns = n;
    }
    __syncthreads();
    const int n = ns;
    const bool vec = (H % 4 == 0);  // then every chunk holds 4 elements
    const int step = static_cast<int>(gridDim.y) * 1024;
    float m = 0.0f;
    for (int i0 = (static_cast<int>(blockIdx.y) * 256 + static_cast<int>(threadIdx.x)) * 4; i0 < H; i0 += step) {
        const int cnt = min(4, H - i0);
        float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int j = 0; j < n; ++j) {
            const int64_t base = static_cast<int64_t>(sp[j]) * H + i0;
            float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            if constexpr (BF16) {
                const uint16_t* yp = static_cast<const uint16_t*>(y) + base;
                if (vec) {
                    const u32x2_t w = *reinterpret_cast<const u32x2_t*>(yp);
                    v[0] = __uint_as_float(w[0] << 16);
                    v[1] = __uint_as_float(w[0] & 0xffff0000u);
                    v[2] = __uint_as_float(w[1] << 16);
                    v[3] = __uint_as_float(w[1] & 0xffff0000u);
                } else {
                    for (int q = 0; q < cnt; ++q) v[q] = bf16_to_f32(yp[q]);
                }
            } else {
                const float* yp = static_cast<const float*>(y) + base;
                if (vec) {
                    const f32x4_t w = *reinterpret_cast<const f32x4_t*>(yp);
                    v[0] = w[0];
                    v[1] = w[1];
                    v[2] = w[2];
                    v[3] = w[3];
                } else {
                    for (int q = 0; q < cnt; ++q) v[q] = yp[q];
                }
            }
            const float g = sg[j];
#pragma unroll
            for (int q = 0; q < 4; ++q) acc[q] = acc[q] + g * v[q];
        }
        const int64_t ob = t * H + i0;
        if constexpr (Q8) {
            for (int q = 0; q < cnt; ++q) {
                qrow[i0 + q] = acc[q];
                const float a = fabsf(acc[q]);
                m = (a > m) ? a : m;
            }
        } else if constexpr (BF16) {
            uint16_t* op = static_cast<uint16_t*>(out) + ob;
            if (vec) {
                *reinterpret_cast<u32x2_t*>(op) = u32x2_t{pack_bf16x2(acc[0], acc[1]), pack_bf16x2(acc[2], acc[3])};
            } else {
                for (int q = 0; q < cnt; ++q) op[q] = f32_to_bf16(acc[q]);
            }
        } else {
            float* op = static_cast<float*>(out) + ob;
            if (vec) {
                *reinterpret_cast<f32x4_t*>(op) = f32x4_t{acc[0], acc[1], acc[2], acc[3]};
            } else {
                for (int q = 0; q < cnt; ++q) op[q] = acc[q];
            }
        }
    }
    if constexpr (Q8) {
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) {
            const float o = __shfl_xor(m, off, 64);
            m = (o > m) ? o : m;
        }
        if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = m;
        __syncthreads();
        m = wmax[0];
#pragma unroll
        for (int w = 1; w < 4; ++w) m = (wmax[w] > m) ? wmax[w] : m;
        const float scale = (m > 0.0f) ? m / 127.0f : 1.0f;
        const float inv = 1.0f / scale;
        int8_t* op = static_cast<int8_t*>(out) + t * H;
        // each thread quantizes the elements it summed (its own LDS entries)
        for (int i0 = static_cast<int>(threadIdx.x) * 4; i0 < H; i0 += 1024) {
            if (vec) {
                uint32_t w = 0;
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    w |= static_cast<uint32_t>(static_cast<uint8_t>(sat_rint(qrow[i0 + q] * inv, 127))) << (8 * q);
                *reinterpret_cast<uint32_t*>(op + i0) = w;
            } else {
                for (int q = 0; q < min(4, H - i0); ++q) op[i0 + q] = static_cast<int8_t>(sat_rint(qrow[i0 + q] * inv, 127));
            }
        }
        if (threadIdx.x == 0) scales[t] = scale;
    }
}

bool aligned(const void* p, unsigned a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

int check_routing(const char* who, int T, int H, int E, int topk) {
    LHQ_REQUIRE(T >= 0 && H > 0 && E > 0 && topk > 0, "%s: bad dims T=%d H=%d E=%d top_k=%d", who, T, H, E, topk);
    LHQ_REQUIRE(static_cast<int64_t>(T) * topk < (int64_t{1} << 31), "%s: T*top_k=%lld exceeds int32", who,
                static_cast<long long>(T) * topk);
    LHQ_SUPPORTED(E <= kMaxExperts, "%s: n_experts=%d exceeds %d", who, E, kMaxExperts);
    return LHQ_OK;
}

int dispatch(const char* who, const void* hidden, int elem, const int32_t* ids, int32_t* offsets,
             int32_t* token_idx, int32_t* slot_idx, int32_t* slot_pos, void* out, int T, int H, int E, int topk,
             void* stream) {
    if (int st = check_routing(who, T, H, E, topk)) return st;
    LHQ_REQUIRE(offsets && (T == 0 || (hidden && ids && token_idx && slot_idx && slot_pos && out)),
                "%s: null pointer", who);
    hipStream_t s = as_stream(stream);
    const int S = T * topk;
    const int64_t row_bytes = static_cast<int64_t>(H) * elem;
    const int vb = (row_bytes % 16 == 0 && aligned(hidden, 16) && aligned(out, 16)) ? 16
                   : (row_bytes % 4 == 0 && aligned(hidden, 4) && aligned(out, 4)) ? 4
                                                                                   : 2;
    const int64_t chunks = ceil_div64(row_bytes / vb, 256);
    LHQ_SUPPORTED(T == 0 || chunks <= 65535, "%s: hidden_dim=%d too large", who, H);
    const dim3 grid(static_cast<unsigned>(T), static_cast<unsigned>(chunks));
    const uint8_t* h = static_cast<const uint8_t*>(hidden);
    uint8_t* o = static_cast<uint8_t*>(out);
    // one launch for decode-sized batches (T = 1, top-2 of 8, H = 4096 bf16:
    // 4.5 us for the two launches)
    if (S >= 1 && S <= kSmallSlots && topk <= kMaxTopK) {
        if (vb == 16)
            moe_dispatch_small_kernel<16><<<grid, kSmallSlots, 0, s>>>(ids, S, topk, E, offsets, token_idx, slot_idx,
                                                                     slot_pos, h, o, row_bytes);
        else if (vb == 4)
            moe_dispatch_small_kernel<4><<<grid, kSmallSlots, 0, s>>>(ids, S, topk, E, offsets, token_idx, slot_idx,
                                                                    slot_pos, h, o, row_bytes);
        else
            moe_dispatch_small_kernel<2><<<grid, kSmallSlots, 0, s>>>(ids, S, topk, E, offsets, token_idx, slot_idx,
                                                                    slot_pos, h, o, row_bytes);
        return check_launch(who);
    }
    moe_rank_kernel<<<1, kRankThreads, 0, s>>>(ids, S, topk, E, offsets, token_idx, slot_idx, slot_pos);
    if (int st = check_launch(who)) return st;
    if (T == 0) return LHQ_OK;
    if (vb == 16) moe_gather_kernel<16><<<grid, 256, 0, s>>>(h, slot_pos, o, row_bytes, topk);
    else if (vb == 4) moe_gather_kernel<4><<<grid, 256, 0, s>>>(h, slot_pos, o, row_bytes, topk);
    else moe_gather_kernel<2><<<grid, 256, 0, s>>>(h, slot_pos, o, row_bytes, topk);
    return check_launch(who);
}

constexpr int kQ8MaxH = 16384;  // Q8 keeps the row in LDS (64 KiB)

template <bool BF16, bool Q8>
int combine(const char* who, const void* y, const int32_t* slot_pos, const float* gates, void* out, float* scales,
            int T, int H, int topk, void* stream) {
    LHQ_REQUIRE(T >= 0 && H > 0 && topk > 0, "%s: bad dims T=%d H=%d top_k=%d", who, T, H, topk);
    LHQ_SUPPORTED(topk <= kMaxTopK, "%s: top_k=%d exceeds %d", who, topk, kMaxTopK);
    LHQ_SUPPORTED(!Q8 || H <= kQ8MaxH, "%s: hidden_dim=%d exceeds %d", who, H, kQ8MaxH);
    if (T == 0) return LHQ_OK;
    LHQ_REQUIRE(y && slot_pos && gates && out && (scales || !Q8), "%s: null pointer", who);
    // vector loads of y (8 bytes bf16, 16 bytes fp32) and stores of the output
    const unsigned ya = BF16 ? 8 : 16, oa = Q8 ? 4 : ya;
    LHQ_REQUIRE(H % 4 != 0 || (aligned(y, ya) && aligned(out, oa)),
                "%s: y and output must be aligned to their 4-element vectors", who);
    const dim3 grid(static_cast<unsigned>(T), Q8 ? 1u : static_cast<unsigned>(ceil_div(H, 1024)));
    const size_t lds = Q8 ? static_cast<size_t>(H) * sizeof(float) : 0;
    moe_combine_kernel<BF16, Q8><<<grid, 256, lds, as_stream(stream)>>>(y, slot_pos, gates, out, scales, H, topk);
    return check_launch(who);
}

}  // namespace
}  // namespace lhq

using namespace lhq;

extern "C" {

int lhq_moe_dispatch_f32(const float* hidden, const int32_t* expert_ids, int32_t* expert_offsets, int32_t* token_idx,
                         int32_t* slot_idx, int32_t* slot_pos, float* expert_inputs, int n_tokens, int hidden_dim,
                         int n_experts, int top_k, void* stream) {
    return dispatch("moe_dispatch_f32", hidden, 4, expert_ids, expert_offsets, token_idx, slot_idx, slot_pos,
                    expert_inputs, n_tokens, hidden_dim, n_experts, top_k, stream);
}

int lhq_moe_dispatch_bf16(const uint16_t* hidden, const int32_t* expert_ids, int32_t* expert_offsets,
                          int32_t* token_idx, int32_t* slot_idx, int32_t* slot_pos, uint16_t* expert_inputs,
                          int n_tokens, int hidden_dim, int n_experts, int top_k, void* stream) {
    return dispatch("moe_dispatch_bf16", hidden, 2, expert_ids, expert_offsets, token_idx, slot_idx, slot_pos,
                    expert_inputs, n_tokens, hidden_dim, n_experts, top_k, stream);
}

int lhq_moe_slot_positions(const int32_t* token_idx, const int32_t* slot_idx, int32_t* slot_pos, int n_tokens,
                           int top_k, void* stream) {
    LHQ_REQUIRE(n_tokens >= 0 && top_k > 0, "moe_slot_positions: bad dims T=%d top_k=%d", n_tokens, top_k);
    const int64_t S = static_cast<int64_t>(n_tokens) * top_k;
    LHQ_REQUIRE(S < (int64_t{1} << 31), "moe_slot_positions: T*top_k exceeds int32");
    if (S == 0) return LHQ_OK;
    LHQ_REQUIRE(token_idx && slot_idx && slot_pos, "moe_slot_positions: null pointer");
    hipStream_t s = as_stream(stream);
    const unsigned blocks = static_cast<unsigned>(ceil_div64(S, 256));
    moe_fill_kernel<<<blocks, 256, 0, s>>>(slot_pos, S, -1);
    moe_invert_kernel<<<blocks, 256, 0, s>>>(token_idx, slot_idx, slot_pos, n_tokens, top_k);
    return check_launch("moe_slot_positions");
}

int lhq_moe_combine_f32(const float* expert_outputs, const int32_t* slot_pos, const float* gate_weights,
                        float* output, int n_tokens, int hidden_dim, int top_k, void* stream) {
    return combine<false, false>("moe_combine_f32", expert_outputs, slot_pos, gate_weights, output, nullptr,
                                 n_tokens, hidden_dim, top_k, stream);
}

int lhq_moe_combine_bf16(const uint16_t* expert_outputs, const int32_t* slot_pos, const float* gate_weights,
                         uint16_t* output, int n_tokens, int hidden_dim, int top_k, void* stream) {
    return combine<true, false>("moe_combine_bf16", expert_outputs, slot_pos, gate_weights, output, nullptr,
                                n_tokens, hidden_dim, top_k, stream);
}

int lhq_moe_combine_q8_f32(const float* expert_outputs, const int32_t* slot_pos, const float* gate_weights,
                           int8_t* q_out, float* scales_out, int n_tokens, int hidden_dim, int top_k, void* stream) {
    return combine<false, true>("moe_combine_q8_f32", expert_outputs, slot_pos, gate_weights, q_out, scales_out,
                                n_tokens, hidden_dim, top_k, stream);
}

int lhq_moe_combine_q8_bf16(const uint16_t* expert_outputs, const int32_t* slot_pos, const float* gate_weights,
                            int8_t* q_out, float* scales_out, int n_tokens, int hidden_dim, int top_k, void* stream) {
    return combine<true, true>("moe_combine_q8_bf16", expert_outputs, slot_pos, gate_weights, q_out, scales_out,
                               n_tokens, hidden_dim, top_k, stream);
}

int lhq_moe_expert_mlp_w4a16_bf16(const uint16_t* expert_inputs, const int32_t* expert_offsets,
                                  const uint8_t* const* gate_up_qweights, const uint16_t* const* gate_up_scales,
                                  const uint32_t* const* gate_up_zeros, const uint8_t* const* down_qweights,
                                  const uint16_t* const* down_scales, const uint32_t* const* down_zeros,
                                  uint16_t* act, uint16_t* expert_outputs, int n_experts, int row_capacity,
                                  int hidden_dim, int intermediate_dim, int group_size, void* stream) {
    if (int st = lhq_gemm_w4a16_bf16_grouped_swiglu(expert_inputs, expert_offsets, gate_up_qweights, gate_up_scales,
                                                    gate_up_zeros, act, n_experts, row_capacity, intermediate_dim,
                                                    hidden_dim, group_size, stream))
        return st;
    return lhq_gemm_w4a16_bf16_grouped(act, expert_offsets, down_qweights, down_scales, down_zeros, expert_outputs,
                                       n_experts, row_capacity, hidden_dim, intermediate_dim, group_size, stream);
}

int lhq_moe_expert_mlp_w4a16_bf16_ws(const uint16_t* expert_inputs, const int32_t* expert_offsets,
                                     const uint8_t* const* gate_up_qweights, const uint16_t* const* gate_up_scales,
                                     const uint32_t* const* gate_up_zeros, const uint8_t* const* down_qweights,
                                     const uint16_t* const* down_scales, const uint32_t* const* down_zeros,
                                     uint16_t* act, uint16_t* expert_outputs, int n_experts, int row_capacity,
                                     int hidden_dim, int intermediate_dim, int group_size, void* workspace,
                                     int64_t workspace_bytes, void* stream) {
    if (int st = lhq_gemm_w4a16_bf16_grouped_swiglu_ws(expert_inputs, expert_offsets, gate_up_qweights,
                                                       gate_up_scales, gate_up_zeros, act, n_experts, row_capacity,
                                                       intermediate_dim, hidden_dim, group_size, workspace,
                                                       workspace_bytes, stream))
        return st;
    return lhq_gemm_w4a16_bf16_grouped_ws(act, expert_offsets, down_qweights, down_scales, down_zeros,
                                          expert_outputs, n_experts, row_capacity, hidden_dim, intermediate_dim,
                                          group_size, workspace, workspace_bytes, stream);
}

}  // extern "C"
