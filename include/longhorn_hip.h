/*
 * longhorn_hip.h -- C ABI of liblonghorn_hip.so, the MI355X (gfx950) backend
 * of LonghornAI's quantized-GEMM path.
 *
 * Conventions for every entry point:
 *   - All array arguments are DEVICE pointers (hipMalloc'd or equivalent),
 *     row-major, tightly packed, unless stated otherwise.
 *   - `stream` is a hipStream_t passed as void* (NULL = the null stream).
 *     Work is enqueued on it; nothing synchronises.  No entry point
 *     allocates device memory.
 *   - Return value: LHQ_OK (0) or an LHQ_ERR_* code; lhq_last_error()
 *     returns a per-thread message for the last failure.  Nothing throws,
 *     nothing aborts, and nothing falls back to the CPU.
 *   - dims are int (int64_t for flat element counts), as in the reference.
 *
 * Each entry point names the reference function it replaces (file:line in
 * the LonghornAI tree).  The reference functions take host pointers and run
 * on the CPU; the lh:: drop-in library (the kernels/ headers) keeps those
 * signatures and forwards here.
 */
#ifndef LONGHORN_HIP_H
#define LONGHORN_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status ------------------------------------------------------------ */
#define LHQ_OK 0
#define LHQ_ERR_INVALID 1     /* null pointer, negative or inconsistent dims */
#define LHQ_ERR_UNSUPPORTED 2 /* valid for the reference, not for this kernel */
#define LHQ_ERR_HIP 3         /* the HIP runtime reported an error */

const char* lhq_status_string(int status);
const char* lhq_last_error(void);
int lhq_version(void); /* major*10000 + minor*100 + patch */

/* ---- int8 symmetric quantizers: quant.hpp:28-48 / quant.cpp:34-105 ------ */
/* Per-tensor (quant.hpp:31-34).  The scale lives in device memory. */
int lhq_q8_quantize_per_tensor(const float* src, int8_t* dst, float* scale_out,
                               int64_t n, void* stream);
int lhq_q8_dequantize_per_tensor(const int8_t* src, const float* scale, float* dst,
                                 int64_t n, void* stream);
/* Per-row / per-token (quant.hpp:38-41). */
int lhq_q8_quantize_per_row(const float* src, int8_t* dst, float* scales_out,
                            int rows, int dim, void* stream);
int lhq_q8_dequantize_per_row(const int8_t* src, const float* scales, float* dst,
                              int rows, int dim, void* stream);
/* Per-token quantization of bfloat16 activations: quant.cpp:52-63 applied to
 * the exact fp32 widening of each bf16 value (benchmark config 3). */
int lhq_q8_quantize_per_row_bf16(const uint16_t* src, int8_t* dst, float* scales_out,
                                 int rows, int dim, void* stream);
/* Per-column / per-output-channel (quant.hpp:45-48). */
int lhq_q8_quantize_per_col(const float* src, int8_t* dst, float* scales_out,
                            int rows, int cols, void* stream);
int lhq_q8_dequantize_per_col(const int8_t* src, const float* scales, float* dst,
                              int rows, int cols, void* stream);

/* ---- int4 group quantizers: quant.hpp:50-75 / quant.cpp:111-172 --------- */
/* Reference layout: packed u8 [K/2, N] (row 2i low nibble, 2i+1 high,
 * two's-complement int4 in [-7,7]); scales fp32 [K/G, N]. */
int lhq_q4_quantize_groupwise(const float* src, uint8_t* packed, float* scales_out,
                              int K, int N, int group_size, void* stream);
int lhq_q4_dequantize_groupwise(const uint8_t* packed, const float* scales, float* dst,
                                int K, int N, int group_size, void* stream);
/* Asymmetric int4 (no reference counterpart; benchmark configs 2, 4, 5):
 * unsigned codes u in [0,15] packed like the reference, fp16 scale and one
 * zero-point byte per (group, column); w = (u - z) * s. */
int lhq_q4a_quantize_groupwise(const float* src, uint8_t* packed, uint16_t* scales_f16,
                               uint8_t* zeros, int K, int N, int group_size, void* stream);
int lhq_q4a_dequantize_groupwise(const uint8_t* packed, const uint16_t* scales_f16,
                                 const uint8_t* zeros, float* dst, int K, int N,
                                 int group_size, void* stream);

/* ---- FP8 E4M3 quantizers: quant.hpp:77-94 / quant.cpp:176-249 ----------- */
int lhq_fp8_quantize_per_tensor(const float* src, uint8_t* dst, float* scale_out,
                                int64_t n, void* stream);
int lhq_fp8_dequantize_per_tensor(const uint8_t* src, const float* scale, float* dst,
                                  int64_t n, void* stream);
int lhq_fp8_quantize_per_row(const float* src, uint8_t* dst, float* scales_out,
                             int rows, int dim, void* stream);
int lhq_fp8_dequantize_per_row(const uint8_t* src, const float* scales, float* dst,
                               int rows, int dim, void* stream);
int lhq_fp8_quantize_per_col(const float* src, uint8_t* dst, float* scales_out,
                             int rows, int cols, void* stream);
int lhq_fp8_dequantize_per_col(const uint8_t* src, const float* scales, float* dst,
                               int rows, int cols, void* stream);

/* ---- prepacked weight layouts (no reference counterpart: the reference
 * reads [K/2,N] / [K,N] row-major directly, gemm_quant.cpp:42,66) --------- */
/* W4 prepacked layout (Nt = ceil(N/16), Kt = ceil(K/128), NG = K/G):
 *   qweight [Nt][Kt][64][16 B]: a 1 KiB tile holds 16 columns x 128 k; the
 *     16 bytes of lane l are the B operands of four 16x16x32 MFMAs for column
 *     16*nt + (l & 15): dword j covers k = 128*kt + 32*j + 8*(l >> 4) + e,
 *     e = 0..7, element e in nibble e < 4 ? 2e : 2(e-4)+1; codes are
 *     unsigned (symmetric q is stored as q + 8).
 *   scales  [Nt][NG][16] fp32 (symmetric) or fp16 (asymmetric).
 *   zeros   [Nt][ceil(NG/8)][16] u32, group g in nibble g % 8.
 * Sizes in bytes: */
int64_t lhq_w4_qweight_bytes(int K, int N);
int64_t lhq_w4_scales_bytes(int K, int N, int group_size, int fp16_scales);
int64_t lhq_w4_zeros_bytes(int K, int N, int group_size);
/* From the reference layout (quant.hpp:52-59; q4_get quant.hpp:68-75):
 * fp32 scales kept as fp32, implied zero point 8. */
int lhq_w4_prepack_sym(const uint8_t* packed, const float* scales, int K, int N,
                       int group_size, uint8_t* qweight, float* scales_out, void* stream);
/* From the asymmetric layout written by lhq_q4a_quantize_groupwise. */
int lhq_w4_prepack_asym(const uint8_t* packed, const uint16_t* scales_f16,
                        const uint8_t* zeros, int K, int N, int group_size,
                        uint8_t* qweight, uint16_t* scales_out, uint32_t* zeros_out,
                        void* stream);
/* Gate and up projections of a SwiGLU MLP in one W4 tensor (no reference
 * counterpart; feeds lhq_gemm_w4a16_bf16_grouped_swiglu): both prepacked by
 * lhq_w4_prepack_asym for [K, I]; column tile 2j of the output is gate tile
 * j, tile 2j+1 is up tile j.  Each output array is twice the size given by
 * lhq_w4_*_bytes(K, I, ...).  All pointers 16-byte aligned. */
int lhq_w4_interleave_gate_up(const uint8_t* gate_qweight, const uint16_t* gate_scales,
                              const uint32_t* gate_zeros, const uint8_t* up_qweight,
                              const uint16_t* up_scales, const uint32_t* up_zeros, int K, int I,
                              int group_size, uint8_t* qweight, uint16_t* scales_out,
                              uint32_t* zeros_out, void* stream);
/* Prepacked W4 weights on disk (no reference counterpart: the reference keeps
 * weights in caller memory and plans safetensors loaders, PLAN.md:326-333).
 * The file is safetensors: tensors "qweight" U8, "scales" F16 (asymmetric,
 * fp16_scales = 1, with "zeros" U32) or F32 (symmetric), in the layout above;
 * metadata format = "lhq-w4-prepacked", version = "1", layout =
 * "w4-tile16x128-v1", K, N, group_size and fnv1a64 (16 hex digits over the
 * data section).  Loading checks every field, size and the checksum before
 * any copy; save and load are synchronous on `stream` and use host memory
 * only.  lhq_w4_file_info reads and checks a file without touching a GPU. */
int lhq_w4_save(const char* path, const uint8_t* qweight, const void* scales,
                const uint32_t* zeros, int K, int N, int group_size, int fp16_scales,
                void* stream);
int lhq_w4_file_info(const char* path, int* K, int* N, int* group_size, int* fp16_scales);
int lhq_w4_load(const char* path, uint8_t* qweight, void* scales, uint32_t* zeros, int K, int N,
                int group_size, int fp16_scales, void* stream);
/* 8-bit B operand (int8 or fp8 e4m3) [K, N] -> k-contiguous Bt [Np][Kp]
 * with Np = N rounded up to 256 and Kp = K rounded up to 128, zero padded. */
int64_t lhq_b8_prepacked_bytes(int K, int N);
int lhq_b8_prepack(const uint8_t* B, int K, int N, uint8_t* Bt, void* stream);

/* ---- W4A16 GEMM: gemm_quant.hpp:47-57 / gemm_quant.cpp:54-82 ----------- */
/* Reference semantics: fp32 A [M,K]; symmetric W4 prepacked by
 * lhq_w4_prepack_sym; C fp32 [M,N] = beta*C + alpha*A@W (beta == 0 never
 * reads C).  group_size must be a multiple of 32 that divides K.
 * Non-finite activations (this and every W4A16 entry point below): the
 * kernels sum x*(q - z) through exact group sums that subtract an
 * activation sum, so a row of A holding +-Inf or NaN gives NaN in every
 * output of that row; other rows are unaffected.  The reference's
 * term-by-term sum (gemm_quant.cpp:78) gives +-Inf there (NaN only where a
 * weight is zero or infinities of both signs meet).  Callers who need that
 * propagation use lhq_q4_dequantize_groupwise + lhq_gemm_f32, as the lh::
 * drop-in does when its host activations hold a non-finite value. */
int lhq_gemm_w4a16(const float* A, const uint8_t* qweight, const float* scales,
                   float* C, int M, int N, int K, int group_size, float alpha, float beta,
                   void* stream);
/* lhq_gemm_w4a16 with a caller workspace (no reference counterpart: the
 * reference's CPU loop needs no partial sums; the lh:: drop-in of
 * gemm_w4a16_groupwise passes one).  At 2..64 rows, and at 65..512 rows
 * where the unsplit grid leaves a CU idle (group_size a multiple
 * of 128, K % 128 == 0), K is split across workgroups: each split writes fp32
 * partial sums to `workspace`, and a second kernel adds them in split order
 * and applies alpha / beta as lhq_gemm_w4a16 does (deterministic).  The
 * split count is the most the workspace allows, up to
 * lhq_gemm_w4a16_workspace_bytes for the shape (0: no split); with a NULL or
 * smaller workspace the call runs with fewer splits or as lhq_gemm_w4a16.
 * workspace: device memory, 16-byte aligned, any contents, not shared with a
 * call running concurrently.  Results match lhq_gemm_w4a16 within fp32
 * reassociation. */
int64_t lhq_gemm_w4a16_workspace_bytes(int M, int N, int K, int group_size);
int lhq_gemm_w4a16_ws(const float* A, const uint8_t* qweight, const float* scales, float* C,
                      int M, int N, int K, int group_size, float alpha, float beta,
                      void* workspace, int64_t workspace_bytes, void* stream);
/* Benchmark configs 2/5: bf16 A [M,K]; asymmetric W4 (fp16 scales, u4
 * zeros) prepacked by lhq_w4_prepack_asym; bf16 C [M,N] = A@W, fp32 accumulate. */
int lhq_gemm_w4a16_bf16(const uint16_t* A, const uint8_t* qweight, const uint16_t* scales,
                        const uint32_t* zeros, uint16_t* C, int M, int N, int K,
                        int group_size, void* stream);
/* lhq_gemm_w4a16_bf16 with a caller workspace (no reference counterpart:
 * the reference's CPU loop needs no partial sums).  Where the output grid
 * cannot fill the GPU (2 <= M <= 64 rows, or up to 512 rows where the
 * unsplit grid fills at most half the GPU; group_size a multiple of 128,
 * and weights large enough for the tile kernel), K is split across
 * workgroups: each split writes fp32 partial sums to `workspace` and they
 * are added in split order into C (deterministic).  The split count is
 * the most the workspace allows, up to what
 * lhq_gemm_w4a16_bf16_workspace_bytes reports for the shape (0: no split);
 * with a NULL or smaller workspace the call runs with fewer splits or none,
 * same results to the bf16 bar.  workspace: device memory, 16-byte aligned, not
 * shared with a call running concurrently.  Results match
 * lhq_gemm_w4a16_bf16 within fp32 reassociation. */
int64_t lhq_gemm_w4a16_bf16_workspace_bytes(int M, int N, int K, int group_size);
int lhq_gemm_w4a16_bf16_ws(const uint16_t* A, const uint8_t* qweight, const uint16_t* scales,
                           const uint32_t* zeros, uint16_t* C, int M, int N, int K, int group_size,
                           void* workspace, int64_t workspace_bytes, void* stream);
/* lhq_gemm_w4a16_bf16_ws for callers that cannot allocate (code under HIP
 * graph capture, serving loops, harnesses that forbid hipMalloc); no
 * counterpart in the reference.  It allocates nothing: the split-K partial
 * sums go to a static 32 MiB device array of the library, one per GPU, held
 * until the process ends, whose address is looked up on the first call on
 * each device (that call may be under graph capture).  The split plan is
 * lhq_gemm_w4a16_bf16_ws's with a workspace of
 * min(lhq_gemm_w4a16_bf16_workspace_bytes, 32 MiB) bytes, and the results
 * are bit-identical to that call's: a shape whose plan asks for more than
 * 32 MiB (2..16 rows at very long K, e.g. M=16, K=131072, N=16384) runs
 * fewer splits.  Calls that overlap on one GPU share the array and race:
 * serialize them (one stream, or events). */
int lhq_gemm_w4a16_bf16_noalloc(const uint16_t* A, const uint8_t* qweight, const uint16_t* scales,
                                const uint32_t* zeros, uint16_t* C, int M, int N, int K,
                                int group_size, void* stream);
/* Uniform batch of independent W4A16 GEMMs (the gemm_batched contract,
 * gemm.cpp:59-67): A [batch,M,K], weights stacked with the per-matrix
 * strides lhq_w4_*_bytes, C [batch,M,N]. */
int lhq_gemm_w4a16_bf16_batched(const uint16_t* A, const uint8_t* qweight,
                                const uint16_t* scales, const uint32_t* zeros, uint16_t* C,
                                int batch, int M, int N, int K, int group_size, void* stream);
/* Ragged grouped W4A16 for MoE experts in ONE launch (benchmark config 4).
 * Group e owns rows [offsets[e], offsets[e+1]) of A [rows, K] and C [rows, N]
 * (the expert_offsets table of moe.cpp:111-123, device-resident); its
 * weights are at qweights[e], scales[e], zeros[e] (device arrays of device
 * pointers).  row_capacity bounds offsets[E] (the rows A and C hold). */
int lhq_gemm_w4a16_bf16_grouped(const uint16_t* A, const int32_t* offsets,
                                const uint8_t* const* qweights,
                                const uint16_t* const* scales,
                                const uint32_t* const* zeros, uint16_t* C,
                                int num_groups, int row_capacity, int N, int K,
                                int group_size, void* stream);

/* The gate / up half of moe_expert_mlp (moe.cpp:185-192) on W4A16 experts,
 * the hook of moe.hpp:26-28: per group, act = bf16(silu(A@Wg) * (A@Wu)),
 * silu(v) = v / (1 + exp(-v)), from fp32 accumulators, in one launch.  The
 * weights of group e are lhq_w4_interleave_gate_up output; act [rows, I]. */
int lhq_gemm_w4a16_bf16_grouped_swiglu(const uint16_t* A, const int32_t* offsets,
                                       const uint8_t* const* qweights,
                                       const uint16_t* const* scales,
                                       const uint32_t* const* zeros, uint16_t* act,
                                       int num_groups, int row_capacity, int I, int K,
                                       int group_size, void* stream);

/* The two grouped launches above with a caller workspace (no reference
 * counterpart: the reference's per-expert CPU loops need no partial sums).
 * Where the tile kernel runs (enough rows per group), one persistent launch
 * of two workgroups per CU walks the (group, 64-row tile, 256-column group)
 * tiles counted from the device-side offsets table, one tile at a time per
 * workgroup; where the tiles fill less than three quarters of one round,
 * they are split along K evenly over all workgroups (stream-K), each K
 * segment's fp32 partial sums going to `workspace`, and a second kernel on
 * the stream adds each split tile's segments in K order (deterministic) and
 * writes it.  Results match the calls without a workspace within fp32
 * reassociation (bit for bit where nothing is split).
 * lhq_gemm_w4a16_bf16_grouped[_swiglu]_workspace_bytes gives the bytes the
 * call can use for a table of num_groups groups over row_capacity rows: 0
 * where the shape runs no tile kernel, 64 KiB where the tile count's bound
 * from row_capacity rules the split out, up to ~56 MiB on MI355X otherwise.
 * A smaller workspace (at least 64 KiB) still takes the persistent launch
 * and splits only when the segments fit; NULL or less runs the launch
 * without one.
 * workspace: device memory, 16-byte aligned, any contents, not shared with
 * a call running concurrently (calls in order on one stream may share it). */
int64_t lhq_gemm_w4a16_bf16_grouped_workspace_bytes(int num_groups, int row_capacity, int N, int K,
                                                    int group_size);
int64_t lhq_gemm_w4a16_bf16_grouped_swiglu_workspace_bytes(int num_groups, int row_capacity, int I,
                                                           int K, int group_size);
int lhq_gemm_w4a16_bf16_grouped_ws(const uint16_t* A, const int32_t* offsets,
                                   const uint8_t* const* qweights, const uint16_t* const* scales,
                                   const uint32_t* const* zeros, uint16_t* C, int num_groups,
                                   int row_capacity, int N, int K, int group_size, void* workspace,
                                   int64_t workspace_bytes, void* stream);
int lhq_gemm_w4a16_bf16_grouped_swiglu_ws(const uint16_t* A, const int32_t* offsets,
                                          const uint8_t* const* qweights,
                                          const uint16_t* const* scales,
                                          const uint32_t* const* zeros, uint16_t* act,
                                          int num_groups, int row_capacity, int I, int K,
                                          int group_size, void* workspace, int64_t workspace_bytes,
                                          void* stream);

/* ---- MoE routing: moe.hpp:63-102 / moe.cpp:102-221 ---------------------- */
/* moe_dispatch (moe.hpp:75-78, moe.cpp:102-140): expert_ids [T, top_k] ->
 * expert_offsets [E+1], token_idx / slot_idx [T*top_k] (stable: slot order
 * within each expert), the rows of hidden [T, H] copied to
 * expert_inputs [T*top_k, H], and slot_pos [T*top_k], the position
 * (t, k) went to (no reference counterpart: the inverse map combine uses).
 * An id outside [0, E) is dropped (slot_pos -1; positions past
 * expert_offsets[E] hold token_idx = slot_idx = -1).  E <= 512. */
int lhq_moe_dispatch_f32(const float* hidden, const int32_t* expert_ids,
                         int32_t* expert_offsets, int32_t* token_idx, int32_t* slot_idx,
                         int32_t* slot_pos, float* expert_inputs, int n_tokens, int hidden_dim,
                         int n_experts, int top_k, void* stream);
int lhq_moe_dispatch_bf16(const uint16_t* hidden, const int32_t* expert_ids,
                          int32_t* expert_offsets, int32_t* token_idx, int32_t* slot_idx,
                          int32_t* slot_pos, uint16_t* expert_inputs, int n_tokens,
                          int hidden_dim, int n_experts, int top_k, void* stream);
/* slot_pos from the reference's dispatch outputs (token_idx, slot_idx must
 * be the layout moe_dispatch writes: each (t, k) at most once). */
int lhq_moe_slot_positions(const int32_t* token_idx, const int32_t* slot_idx, int32_t* slot_pos,
                           int n_tokens, int top_k, void* stream);
/* moe_combine (moe.hpp:96-102, moe.cpp:198-221): output[t] = sum over t's
 * slots in position order of gate_weights[t, k] * expert_outputs[pos],
 * fp32 with the reference's rounding (bit-exact); top_k <= 64.  The bf16
 * form widens expert_outputs exactly and rounds the sum once. */
int lhq_moe_combine_f32(const float* expert_outputs, const int32_t* slot_pos,
                        const float* gate_weights, float* output, int n_tokens, int hidden_dim,
                        int top_k, void* stream);
int lhq_moe_combine_bf16(const uint16_t* expert_outputs, const int32_t* slot_pos,
                         const float* gate_weights, uint16_t* output, int n_tokens,
                         int hidden_dim, int top_k, void* stream);
/* moe_combine followed by q8_quantize_per_row (quant.cpp:52-63) on its fp32
 * sums, fused: the combine's epilogue quantizes each token's row to int8
 * with one fp32 scale per token -- the per-token activations a W8A8 layer
 * reads next (no reference counterpart as one call; bit-exact with the two
 * reference functions composed).  hidden_dim <= 16384. */
int lhq_moe_combine_q8_f32(const float* expert_outputs, const int32_t* slot_pos,
                           const float* gate_weights, int8_t* q_out, float* scales_out,
                           int n_tokens, int hidden_dim, int top_k, void* stream);
int lhq_moe_combine_q8_bf16(const uint16_t* expert_outputs, const int32_t* slot_pos,
                            const float* gate_weights, int8_t* q_out, float* scales_out,
                            int n_tokens, int hidden_dim, int top_k, void* stream);
/* moe_expert_mlp (moe.hpp:80-94, moe.cpp:150-196) with W4A16 experts:
 * lhq_gemm_w4a16_bf16_grouped_swiglu into act [row_capacity, I] (caller's
 * buffer), then lhq_gemm_w4a16_bf16_grouped with the down weights into
 * expert_outputs [row_capacity, H], bf16. */
int lhq_moe_expert_mlp_w4a16_bf16(const uint16_t* expert_inputs, const int32_t* expert_offsets,
                                  const uint8_t* const* gate_up_qweights,
                                  const uint16_t* const* gate_up_scales,
                                  const uint32_t* const* gate_up_zeros,
                                  const uint8_t* const* down_qweights,
                                  const uint16_t* const* down_scales,
                                  const uint32_t* const* down_zeros, uint16_t* act,
                                  uint16_t* expert_outputs, int n_experts, int row_capacity,
                                  int hidden_dim, int intermediate_dim, int group_size,
                                  void* stream);
/* The same with the grouped launches' workspace (lhq_gemm_w4a16_bf16_grouped_ws;
 * the two launches run in order on `stream` and share it): the larger of
 * lhq_gemm_w4a16_bf16_grouped_swiglu_workspace_bytes(n_experts, row_capacity,
 * intermediate_dim, hidden_dim, group_size) and
 * lhq_gemm_w4a16_bf16_grouped_workspace_bytes(n_experts, row_capacity,
 * hidden_dim, intermediate_dim, group_size) lets both split fully. */
int lhq_moe_expert_mlp_w4a16_bf16_ws(const uint16_t* expert_inputs, const int32_t* expert_offsets,
                                     const uint8_t* const* gate_up_qweights,
                                     const uint16_t* const* gate_up_scales,
                                     const uint32_t* const* gate_up_zeros,
                                     const uint8_t* const* down_qweights,
                                     const uint16_t* const* down_scales,
                                     const uint32_t* const* down_zeros, uint16_t* act,
                                     uint16_t* expert_outputs, int n_experts, int row_capacity,
                                     int hidden_dim, int intermediate_dim, int group_size,
                                     void* workspace, int64_t workspace_bytes, void* stream);

/* ---- W8A8 GEMM: gemm_quant.hpp:34-45 / gemm_quant.cpp:29-49 ------------ */
/* Reference semantics, bit-exact: Aq int8 [M,K]; Bt = lhq_b8_prepack(Bq);
 * C[m,n] = beta-applied C + ((alpha*A_s[m])*B_s[n])*float(acc). */
int lhq_gemm_w8a8(const int8_t* Aq, const int8_t* Bt, const float* A_scales,
                  const float* B_scales, float* C, int M, int N, int K, float alpha,
                  float beta, void* stream);
/* Benchmark config 3: same, alpha = 1, beta = 0, output rounded to bf16. */
int lhq_gemm_w8a8_bf16(const int8_t* Aq, const int8_t* Bt, const float* A_scales,
                       const float* B_scales, uint16_t* C, int M, int N, int K,
                       void* stream);
/* Debug: the raw int32 accumulator of gemm_quant.cpp:38-43, [M,N]. */
int lhq_gemm_w8a8_i32(const int8_t* Aq, const int8_t* Bt, int32_t* acc, int M, int N,
                      int K, void* stream);

/* ---- FP8 E4M3 GEMM: gemm_quant.hpp:59-70 / gemm_quant.cpp:87-104 ------- */
/* A e4m3 [M,K]; Bt = lhq_b8_prepack(B e4m3 [K,N]); per-tensor scales in
 * device memory; C = beta-applied C + ((alpha*sA)*sB)*acc, fp32 acc. */
int lhq_gemm_fp8_e4m3(const uint8_t* A, const uint8_t* Bt, const float* A_scale,
                      const float* B_scale, float* C, int M, int N, int K, float alpha,
                      float beta, void* stream);

/* ---- fp32 GEMM: gemm.hpp:13-29 / gemm.cpp:5-75 -------------------------- */
/* lh::gemm semantics (beta first; beta == 0 never reads C). */
int lhq_gemm_f32(const float* A, const float* B, float* C, int M, int N, int K,
                 float alpha, float beta, void* stream);
/* lh::gemm_ref semantics: C = alpha*acc + beta*C, C always read. */
int lhq_gemm_f32_ref(const float* A, const float* B, float* C, int M, int N, int K,
                     float alpha, float beta, void* stream);
int lhq_gemm_f32_batched(const float* A, const float* B, float* C, int batch, int M,
                         int N, int K, float alpha, float beta, void* stream);

/* ---- diagnostics (no counterpart in the reference) ----------------------- */
/* Converts all 2^32 fp32 bit patterns to bf16 with the instruction the
 * kernels use (v_cvt_pk_bf16_f32) and counts results that differ from the
 * reference's rule (dtypes.hpp:87-98).  counts: 2 device uint64, set to
 * {non-NaN mismatches, NaN mismatches}; both are 0 on a conforming device. */
int lhq_selftest_bf16(unsigned long long* counts, void* stream);
/* The matrix-core rate probes bench.py uses are in the separate diagnostics
 * library (include/longhorn_diag.h, liblonghorn_diag.so). */

#ifdef __cplusplus
}
#endif

#endif /* LONGHORN_HIP_H */
