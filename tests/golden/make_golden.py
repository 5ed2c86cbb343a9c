"""Write tests/golden/ref_vectors.npz from the reference's own code.

The reference ships no golden vectors, so these are produced by running the
reference's quant / gemm_quant / gemm sources, compiled where they lie into
oracle/_ref/libref.so (oracle/Makefile), on small seeded inputs.  Only the
resulting data (inputs and outputs) is committed; the test
tests/test_oracle_pins.py checks the C restatement against it on machines
where the reference tree is absent.

Run:  make -C oracle && python tests/golden/make_golden.py
"""
from __future__ import annotations

import hashlib
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle import Ref  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "ref_vectors.npz")


def special_floats() -> np.ndarray:
    """fp32 values around every rounding / range boundary of the 16- and
    8-bit formats, plus random bit patterns."""
    vals = [0.0, -0.0, np.inf, -np.inf, np.nan, 1.0, -1.0, 448.0, 464.0, 480.0, 65504.0, 65520.0, 70000.0,
            57344.0, 61440.0, 2.0 ** -9, 2.0 ** -10, 1.5 * 2.0 ** -10, 2.0 ** -14, 2.0 ** -24, 2.0 ** -25,
            1.5 * 2.0 ** -25, 2.0 ** -16, 2.0 ** -17, 3.0 * 2.0 ** -18, 1e-30, 3.4e38]
    out = []
    for v in vals:
        f = np.float32(v)
        b = f.view(np.uint32)
        for d in (-2, -1, 0, 1, 2):
            out.append(np.uint32((int(b) + d) % 2 ** 32 if np.isfinite(f) else b).view(np.float32))
    # every power of two in range and the midpoints between format neighbours
    for e in range(-30, 20):
        for m in range(0, 16):
            x = np.float32((1.0 + m / 16.0) * 2.0 ** e)
            for mid in (x, np.float32(x * (1 + 1 / 32)), np.float32(x * (1 + 1 / 256)),
                        np.float32(x * (1 + 1 / 2048)), np.float32(x * (1 + 1 / 512))):
                out += [mid, -mid]
    g = np.random.default_rng(2024)
    out += list(g.integers(0, 2 ** 32, 4000, dtype=np.uint64).astype(np.uint32).view(np.float32))
    out += list((g.standard_normal(2000) * 10).astype(np.float32))
    return np.array(out, np.float32)


def main() -> None:
    r = Ref()
    g = np.random.default_rng(7)
    d = {}

    # -- conversions (dtypes.hpp) -------------------------------------------
    d["e4m3_decode"] = r.e4m3_to_f32_n(np.arange(256, dtype=np.uint8)).view(np.uint32)
    d["e5m2_decode"] = r.e5m2_to_f32_n(np.arange(256, dtype=np.uint8)).view(np.uint32)
    f16_all = r.f16_to_f32_n(np.arange(65536, dtype=np.uint16)).view(np.uint32)
    d["f16_decode_sha256"] = np.frombuffer(hashlib.sha256(f16_all.tobytes()).digest(), np.uint8)
    xs = special_floats()
    d["conv_x"] = xs.view(np.uint32)
    d["conv_f16"] = r.f32_to_f16_n(xs)
    d["conv_bf16"] = r.f32_to_bf16_n(xs)
    d["conv_e4m3"] = r.f32_to_e4m3_n(xs)
    d["conv_e5m2"] = r.f32_to_e5m2_n(xs)

    # -- quantizers (quant.cpp) ----------------------------------------------
    x = g.uniform(-3, 3, (12, 96)).astype(np.float32)
    x[0] = 0.0
    x[1, :6] = [0.5, 1.5, 2.5, -0.5, 3.0, -3.0]
    x[2, 3] = np.nan
    d["q_x"] = x
    d["q8_row_q"], d["q8_row_s"] = r.q8_quantize_per_row(x)
    d["q8_col_q"], d["q8_col_s"] = r.q8_quantize_per_col(x)
    q, s = r.q8_quantize_per_tensor(x)
    d["q8_tensor_q"], d["q8_tensor_s"] = q, np.float32(s)
    d["fp8_row_q"], d["fp8_row_s"] = r.fp8_quantize_per_row(x)
    d["fp8_col_q"], d["fp8_col_s"] = r.fp8_quantize_per_col(x)
    q, s = r.fp8_quantize_per_tensor(x)
    d["fp8_tensor_q"], d["fp8_tensor_s"] = q, np.float32(s)
    w = g.uniform(-1, 1, (64, 24)).astype(np.float32)
    w[:32, 0] = 0.0
    d["q4_w"] = w
    for G in (32, 8, 64):
        d[f"q4_G{G}_p"], d[f"q4_G{G}_s"] = r.q4_quantize_groupwise(w, G)
        d[f"q4_G{G}_deq"] = r.q4_dequantize_groupwise(d[f"q4_G{G}_p"], d[f"q4_G{G}_s"], 64, 24, G)
    w3 = g.uniform(-1, 1, (30, 5)).astype(np.float32)   # odd group: pairs straddle groups
    d["q4_G3_w"] = w3
    d["q4_G3_p"], d["q4_G3_s"] = r.q4_quantize_groupwise(w3, 3)

    # -- GEMMs (gemm_quant.cpp, gemm.cpp) --------------------------------------
    A = g.uniform(-1, 1, (32, 64)).astype(np.float32)
    B = g.uniform(-1, 1, (64, 48)).astype(np.float32)
    C0 = g.uniform(-1, 1, (32, 48)).astype(np.float32)
    d["g_A"], d["g_B"], d["g_C0"] = A, B, C0
    Aq, As = r.q8_quantize_per_row(A)
    Bq, Bs = r.q8_quantize_per_col(B)
    d["w8_Aq"], d["w8_As"], d["w8_Bq"], d["w8_Bs"] = Aq, As, Bq, Bs
    ab = [(1.0, 0.0), (0.5, 2.0), (1.0, 1.0), (-0.3, -0.7)]
    d["alpha_beta"] = np.array(ab, np.float32)
    for i, (al, be) in enumerate(ab):
        d[f"w8a8_{i}"] = r.gemm_w8a8(Aq, Bq, As, Bs, C0, al, be)
        d[f"gemm_{i}"] = r.gemm(A, B, C0, al, be)
        d[f"gemm_ref_{i}"] = r.gemm_ref(A, B, C0, al, be)
    # int32 accumulator through unit scales: |acc| < 2^24 so float(acc) is exact
    d["w8a8_acc"] = r.gemm_w8a8(Aq, Bq, np.ones(32, np.float32), np.ones(48, np.float32)).astype(np.int32)
    Bp, Bsc = r.q4_quantize_groupwise(B, 32)
    d["w4_Bp"], d["w4_Bs"] = Bp, Bsc
    for i, (al, be) in enumerate(ab):
        d[f"w4a16_{i}"] = r.gemm_w4a16_groupwise(A, Bp, Bsc, 48, 32, C0, al, be)
    A2 = g.uniform(-1, 1, (4, 256)).astype(np.float32)
    B2 = (g.standard_normal((256, 64)) * 0.02).astype(np.float32)
    Bp2, Bs2 = r.q4_quantize_groupwise(B2, 128)
    d["w4g128_A"], d["w4g128_Bp"], d["w4g128_Bs"] = A2, Bp2, Bs2
    d["w4g128_C"] = r.gemm_w4a16_groupwise(A2, Bp2, Bs2, 64, 128)
    a8, sa = r.fp8_quantize_per_tensor(A)
    b8, sb = r.fp8_quantize_per_tensor(B)
    d["fp8_A"], d["fp8_B"], d["fp8_sa"], d["fp8_sb"] = a8, b8, np.float32(sa), np.float32(sb)
    for i, (al, be) in enumerate(ab):
        d[f"fp8gemm_{i}"] = r.gemm_fp8_e4m3(a8, b8, sa, sb, C0, al, be)
    Ab = g.uniform(-1, 1, (3, 5, 7)).astype(np.float32)
    Bb = g.uniform(-1, 1, (3, 7, 6)).astype(np.float32)
    d["gb_A"], d["gb_B"] = Ab, Bb
    d["gemm_batched"] = r.gemm_batched(Ab, Bb, None, 1.0, 0.0)

    # -- dequantizers (quant.cpp:47-50,65-73,98-105 and the fp8 forms) --------
    for kind in ("q8", "fp8"):
        d[f"{kind}_row_deq"] = getattr(r, f"{kind}_dequantize_per_row")(d[f"{kind}_row_q"], d[f"{kind}_row_s"])
        d[f"{kind}_col_deq"] = getattr(r, f"{kind}_dequantize_per_col")(d[f"{kind}_col_q"], d[f"{kind}_col_s"])
        d[f"{kind}_tensor_deq"] = getattr(r, f"{kind}_dequantize_per_tensor")(
            d[f"{kind}_tensor_q"], float(d[f"{kind}_tensor_s"]))

    # -- per-token int8 of bf16 rows (config 3's activations): the reference's
    # q8_quantize_per_row (quant.cpp:52-63) on the exact fp32 widening ---------
    g2 = np.random.default_rng(8)
    xb = g2.standard_normal((9, 256)).astype(np.float32)
    xb[0] = 0.0                                             # all-zero row: scale 1
    xb[1] = g2.uniform(-100, 100, 256).astype(np.float32)   # max 127: scale 1, exact ties
    xb[1, :9] = [127.0, 0.5, 1.5, 2.5, -2.5, 63.5, -63.5, -0.5, 126.5]
    xb[2, [7, 100, 201]] = [20.0, -20.0, 20.0]              # +-20 outliers
    xb[3, 5] = np.nan                                       # NaN never wins the max
    xb[4, 17] = -20.0                                       # negative peak
    xb[5] *= 1e-3
    xb[6] *= 1e4
    for row in (7, 8):
        xb[row, g2.integers(0, 256)] = 20.0 if row == 7 else -20.0
    bits = r.f32_to_bf16_n(xb)
    d["q8bf_x"] = bits
    d["q8bf_q"], d["q8bf_s"] = r.q8_quantize_per_row((bits.astype(np.uint32) << 16).view(np.float32))

    # -- the W8A8 epilogue with alpha = 1, beta = 0, rounded to bf16 by the
    # reference's own rule (gemm_quant.cpp:29-49, dtypes.hpp:87-98) -----------
    Aq3, As3 = r.q8_quantize_per_row(g2.standard_normal((16, 96)).astype(np.float32))
    Bq3, Bs3 = r.q8_quantize_per_col((g2.standard_normal((96, 40)) * 0.02).astype(np.float32))
    d["w8bf_Aq"], d["w8bf_As"], d["w8bf_Bq"], d["w8bf_Bs"] = Aq3, As3, Bq3, Bs3
    d["w8bf_C"] = r.f32_to_bf16_n(r.gemm_w8a8(Aq3, Bq3, As3, Bs3, None, 1.0, 0.0))

    # -- ragged pointer-array groups (gemm.cpp:69-75), alpha/beta applied -----
    dims = [(8, 6, 7), (5, 9, 4), (1, 13, 3)]
    for i, (m, k, n) in enumerate(dims):
        d[f"gg_A{i}"] = g2.uniform(-1, 1, (m, k)).astype(np.float32)
        d[f"gg_B{i}"] = g2.uniform(-1, 1, (k, n)).astype(np.float32)
        d[f"gg_C0{i}"] = g2.uniform(-1, 1, (m, n)).astype(np.float32)
    outs = r.gemm_grouped([d[f"gg_A{i}"] for i in range(3)], [d[f"gg_B{i}"] for i in range(3)],
                          [d[f"gg_C0{i}"] for i in range(3)], 0.75, -1.25)
    for i, c in enumerate(outs):
        d[f"gg_C{i}"] = c

    np.savez_compressed(OUT, **d)
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes, {len(d)} arrays)")


if __name__ == "__main__":
    main()
