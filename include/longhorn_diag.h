/* longhorn_diag.h -- matrix-core rate probes (liblonghorn_diag.so).
 *
 * A diagnostics library beside the product library (longhorn_hip.h): it
 * measures the hardware for the benchmark's roofline figures and has no
 * counterpart in the reference.  Nothing on the quantized-GEMM path calls
 * it.  Entry points validate their arguments before any launch and return
 * LHD_OK or an error status, with a per-thread message from
 * lhd_last_error(). */
#ifndef LONGHORN_DIAG_H
#define LONGHORN_DIAG_H

#ifdef __cplusplus
extern "C" {
#endif

#define LHD_OK 0
#define LHD_ERR_INVALID 1
#define LHD_ERR_HIP 3

const char* lhd_last_error(void);
/* Matrix-core rate probe: `blocks` workgroups of 4 waves, each wave running
 * `iters` rounds of 4 MFMAs on register operands (no memory traffic), so the
 * launch time gives the sustained MFMA rate with the GPU loaded.  Kinds 0..5
 * rotate over 4 independent accumulators: 0: v_mfma_i32_32x32x32_i8 (65,536
 * ops each), 1: v_mfma_f32_16x16x32_bf16 (16,384 flops), 2:
 * v_mfma_f32_32x32x16_bf16 (32,768 flops), 3: v_mfma_i32_16x16x64_i8
 * (32,768 ops); 4, 5: kind 1 with 2 or 4 independent integer VALU operations
 * per MFMA (whether VALU work overlaps the matrix core's).  Kinds 6, 7: one
 * dependent chain (each MFMA accumulates onto the previous result) of kind 1's
 * and kind 3's instruction.  One launch performs blocks * 4 * iters * 4
 * MFMAs.  sink: `blocks` device ints (written). */
int lhd_probe_mfma_rate(int kind, int blocks, int iters, int* sink, void* stream);
/* Matrix-core rate on the caller's operand values: `blocks` workgroups of 4
 * waves; each wave loads two sets of 8 fragments (4 A blocks, 4 B blocks)
 * from `operands` once, then runs `iters` rounds of 32 MFMAs: two k steps,
 * each one MFMA on each of 16 accumulators in turn (the W8A8 / FP8 tiles'
 * order).  The rate depends on the values through the power limit.  Kinds:
 * 0: v_mfma_i32_32x32x32_i8 (65,536 ops each), 1:
 * v_mfma_scale_f32_32x32x64_f8f6f4, e4m3 with unit scales (131,072 flops),
 * 2: v_mfma_f32_16x16x32_bf16 (16,384 flops), 3 and 4: kind 0 issued as
 * k chains of 2 and 4 MFMAs on one accumulator (each round 32 and 64 MFMAs),
 * 5 and 6: v_mfma_i32_16x16x64_i8 (32,768 ops) on the same fragments, as k
 * chains of 4 (64 per round) and one per accumulator in turn (32 per round),
 * 7: that instruction as k chains of 2 (32 per round).
 * operands: 32 KiB of device
 * memory; fragment x (0..7) of set s (0..1) for lane l is the 16 bytes at
 * ((8s + x) * 64 + l) * 16 (kind 1: the fragment's low half there, its high
 * half 16 KiB further).  sink: `blocks` device ints (written).  clocks: null,
 * or 2 * `blocks` device uint64 set to {shader-clock ticks, 100 MHz ticks}
 * over wave 0's loop in each workgroup. */
int lhd_probe_mfma_operands(int kind, const void* operands, int blocks, int iters, int* sink,
                            unsigned long long* clocks, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LONGHORN_DIAG_H */
