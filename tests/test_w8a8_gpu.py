"""W8A8 and FP8 GEMMs on the GPU vs the CPU oracle (gemm_quant.cpp:29-49, 87-104).

int32 accumulators must match bit for bit; the fp32 epilogue repeats the
reference's multiply order without fused multiply-add, so fp32 and bf16
outputs are compared bit for bit as well.  FP8 accumulates in fp32 in a
different order than the reference: relative Frobenius <= 1e-4.
"""
import numpy as np
import pytest

from oracle import rel_frobenius
from tests import _data as D

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops(lib):
    from longhornai_amd import ops as _ops
    return _ops


def _quantized(oracle, M, K, N, seed, lo=-1.0, hi=1.0):
    A = D.uniform((M, K), lo, hi, seed)
    B = D.uniform((K, N), lo, hi, seed + 1)
    Aq, As = oracle.q8_quantize_per_row(A)
    Bq, Bs = oracle.q8_quantize_per_col(B)
    return Aq, As, Bq, Bs


SHAPES = [(32, 64, 48), (1, 4096, 4096), (255, 256, 257), (256, 512, 256), (300, 1024, 520),
          (16, 208, 100), (7, 4096, 1000), (2, 48, 17),  # small-size kernel (M <= 16, 16-row blocks)
          (513, 128, 1000), (4, 16, 4),
          (300, 1040, 520),  # K % 128 != 0 over several stages: the tile's clamped A loads meet zero-padded B
          # mid-size kernel (16 < M <= 32, 32 x 32 blocks), then whole or half tiles
          (17, 4096, 1000), (24, 64, 70), (33, 1040, 130), (128, 2048, 2064), (100, 64, 70)]


@pytest.mark.parametrize("M,K,N", SHAPES)
def test_w8a8_i32_bitexact(oracle, ops, M, K, N):
    Aq, _, Bq, _ = _quantized(oracle, M, K, N, seed=M + N)
    want = oracle.gemm_w8a8_i32acc(Aq, Bq)
    Bt = ops.prepack_b8(ops.dev(Bq), K, N)
    got = ops.host(ops.gemm_w8a8_i32(ops.dev(Aq), Bt, M, N, K))
    assert np.array_equal(got, want)


def test_w8a8_i32_extremes(oracle, ops):
    """All +-127 operands: |acc| reaches K*127^2 exactly."""
    M, K, N = 64, 2048, 64
    g = D.rng(5)
    Aq = np.where(g.random((M, K)) < 0.5, -127, 127).astype(np.int8)
    Bq = np.where(g.random((K, N)) < 0.5, -127, 127).astype(np.int8)
    Aq[0, :] = 127
    Bq[:, 0] = 127
    want = oracle.gemm_w8a8_i32acc(Aq, Bq)
    assert want[0, 0] == K * 127 * 127
    Bt = ops.prepack_b8(ops.dev(Bq), K, N)
    got = ops.host(ops.gemm_w8a8_i32(ops.dev(Aq), Bt, M, N, K))
    assert np.array_equal(got, want)


@pytest.mark.parametrize("M,K,N", SHAPES)
@pytest.mark.parametrize("alpha,beta", [(1.0, 0.0), (0.5, 2.0), (1.0, 1.0), (-0.75, -1.5)])
def test_w8a8_f32_bitexact(oracle, ops, M, K, N, alpha, beta):
    Aq, As, Bq, Bs = _quantized(oracle, M, K, N, seed=3 * M + N)
    C0 = D.uniform((M, N), -2, 2, 9)
    want = oracle.gemm_w8a8(Aq, Bq, As, Bs, C0, alpha, beta)
    Bt = ops.prepack_b8(ops.dev(Bq), K, N)
    C = ops.dev(C0)
    ops.gemm_w8a8(ops.dev(Aq), Bt, ops.dev(As), ops.dev(Bs), M, N, K, C, alpha, beta)
    got = ops.host(C)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("M,K,N", [(64, 512, 384), (512, 1024, 512),
                                   (20, 4096, 14336),   # mid-size kernel, 32 x 32 blocks
                                   (96, 1024, 3000),    # 12 tiles: every workgroup a 256 x 128 half tile
                                   (200, 2048, 3000)])  # (and 200 live rows of 256)
def test_w8a8_bf16_bitexact(oracle, ops, M, K, N):
    X = D.to_bf16_bits(oracle, D.with_outliers(D.normal((M, K), 1.0, 11), 0.001, 20.0, 12))
    Aq, As = oracle.q8_quantize_per_row_bf16(X)
    Bq, Bs = oracle.q8_quantize_per_col(D.normal((K, N), 0.02, 13))
    want = oracle.gemm_w8a8_bf16out(Aq, Bq, As, Bs)
    Bt = ops.prepack_b8(ops.dev(Bq), K, N)
    got = ops.host(ops.gemm_w8a8_bf16(ops.dev(Aq), Bt, ops.dev(As), ops.dev(Bs), M, N, K), np.uint16)
    assert np.array_equal(got, want)


def test_w8a8_full_config3_sampled(oracle, ops):
    """Config 3 at full size (M=2048, K=4096, N=14336): the int32 accumulator on
    a seeded sample of 96 rows x 96 columns equals an exact int64 dot product,
    and the bf16 output equals the oracle epilogue on those entries."""
    M, K, N = 2048, 4096, 14336
    X = D.to_bf16_bits(oracle, D.with_outliers(D.normal((M, K), 1.0, 31), 0.001, 20.0, 32))
    Aq, As = oracle.q8_quantize_per_row_bf16(X)
    Bq, Bs = oracle.q8_quantize_per_col(D.normal((K, N), 0.02, 33))
    Bt = ops.prepack_b8(ops.dev(Bq), K, N)
    dA = ops.dev(Aq)
    acc = ops.host(ops.gemm_w8a8_i32(dA, Bt, M, N, K))
    out = ops.host(ops.gemm_w8a8_bf16(dA, Bt, ops.dev(As), ops.dev(Bs), M, N, K), np.uint16)
    g = D.rng(34)
    rows = np.sort(g.choice(M, 96, replace=False))
    cols = np.sort(g.choice(N, 96, replace=False))
    exact = Aq[rows].astype(np.int64) @ Bq[:, cols].astype(np.int64)
    assert np.array_equal(acc[np.ix_(rows, cols)].astype(np.int64), exact)
    sub = oracle.gemm_w8a8_bf16out(np.ascontiguousarray(Aq[rows]), np.ascontiguousarray(Bq[:, cols]),
                                   As[rows], Bs[cols])
    assert np.array_equal(out[np.ix_(rows, cols)], sub)


@pytest.mark.parametrize("M,K,N", [(4096, 4096, 14336), (4000, 1024, 14136), (4000, 512, 14330)])
def test_w8a8_bf16_persistent_tiles(oracle, ops, M, K, N):
    """896 tiles on a 256-CU device run as a persistent launch: 3 rounds of
    256x256 tiles, then the last 128 tiles as 256x128 halves (the second shape
    has partial row and column tiles, and halves wholly past N; the third has
    N % 8 != 0, so every tile takes the edge epilogue).  Every bf16
    output equals the fp32-output kernel's value (one tile per workgroup)
    rounded by the oracle's bf16 rule; sampled entries equal the oracle."""
    X = D.to_bf16_bits(oracle, D.with_outliers(D.normal((M, K), 1.0, 41), 0.001, 20.0, 42))
    Aq, As = oracle.q8_quantize_per_row_bf16(X)
    Bq, Bs = oracle.q8_quantize_per_col(D.normal((K, N), 0.02, 43))
    Bt = ops.prepack_b8(ops.dev(Bq), K, N)
    dA, dAs, dBs = ops.dev(Aq), ops.dev(As), ops.dev(Bs)
    out = ops.host(ops.gemm_w8a8_bf16(dA, Bt, dAs, dBs, M, N, K), np.uint16)
    C = ops.dev(np.zeros((M, N), np.float32))
    ops.gemm_w8a8(dA, Bt, dAs, dBs, M, N, K, C, 1.0, 0.0)
    assert np.array_equal(out, oracle.f32_to_bf16_n(ops.host(C)))
    g = D.rng(44)
    rows = np.sort(g.choice(M, 64, replace=False))
    cols = np.sort(np.concatenate([g.choice(N, 60, replace=False), np.arange(N - 4, N)]))
    sub = oracle.gemm_w8a8_bf16out(np.ascontiguousarray(Aq[rows]), np.ascontiguousarray(Bq[:, cols]),
                                   As[rows], Bs[cols])
    assert np.array_equal(out[np.ix_(rows, cols)], sub)


@pytest.mark.parametrize("M,K,N", [(16, 64, 32), (100, 512, 300), (256, 1024, 256)])
@pytest.mark.parametrize("alpha,beta", [(1.0, 0.0), (0.5, 2.0)])
def test_fp8_matches_oracle(oracle, ops, M, K, N, alpha, beta):
    A = D.uniform((M, K), -1, 1, 50 + M)
    B = D.uniform((K, N), -1, 1, 51 + N)
    a8, sa = oracle.fp8_quantize_per_tensor(A)
    b8, sb = oracle.fp8_quantize_per_tensor(B)
    C0 = D.uniform((M, N), -1, 1, 52)
    want = oracle.gemm_fp8_e4m3(a8, b8, sa, sb, C0, alpha, beta)
    Bt = ops.prepack_b8(ops.dev(b8), K, N)
    C = ops.dev(C0)
    ops.run("lhq_gemm_fp8_e4m3", a8, Bt, np.array([sa], np.float32), np.array([sb], np.float32),
            C, M, N, K, alpha, beta)
    assert rel_frobenius(ops.host(C), want) <= 1e-4


@pytest.mark.parametrize("M,K,N", [
    (300, 1024, 520),   # ragged M and N
    (257, 384, 1000),   # six k stages: a partial last round of buffers
    (512, 4096, 256),
    (129, 128, 64),     # two k stages, fewer than the pipeline's buffers (one tile: two half tiles,
                        # the second wholly past N)
    (2048, 256, 4200),  # 136 tiles: whole 256 x 256 tiles (half tiles only where they fill at most half the CUs)
    # up to 16 rows: the mid-size kernel's 16-row blocks (four waves over K)
    (1, 4096, 1000), (5, 128, 1000), (8, 1024, 520), (16, 2048, 72),
    # then 32 x 32 blocks up to 32 rows, then half tiles
    (17, 1024, 520), (32, 128, 64), (100, 2048, 1000), (128, 4096, 256),
])
@pytest.mark.parametrize("alpha,beta", [(1.0, 0.0), (0.5, 2.0)])
def test_fp8_dma_path(oracle, ops, M, K, N, alpha, beta):
    """K % 128 == 0 runs the mid-size kernel (16x16x32 fp8 MFMAs, K split across
    waves; 16-row blocks up to 16 rows, 32 x 32 blocks up to 32) and the LDS-DMA
    kernel on the 32x32x64 f8f6f4 MFMA above (256 x 128 half tiles where the
    tiles fill at most half the CUs).  A NaN code in A (0x7f) and in B (0xff) make exactly their row /
    column NaN, as in the reference's fp32 loop."""
    A = D.normal((M, K), 1.0, 70 + M)
    B = D.normal((K, N), 0.05, 71 + N)
    a8, sa = oracle.fp8_quantize_per_tensor(A)
    b8, sb = oracle.fp8_quantize_per_tensor(B)
    a8[M // 3, K - 1] = 0x7F
    b8[K // 2, N - 2] = 0xFF
    C0 = D.uniform((M, N), -1, 1, 72)
    want = oracle.gemm_fp8_e4m3(a8, b8, sa, sb, C0, alpha, beta)
    Bt = ops.prepack_b8(ops.dev(b8), K, N)
    C = ops.dev(C0)
    ops.run("lhq_gemm_fp8_e4m3", a8, Bt, np.array([sa], np.float32), np.array([sb], np.float32),
            C, M, N, K, alpha, beta)
    got = ops.host(C)
    nan = np.isnan(want)
    assert nan[M // 3].all() and nan[:, N - 2].all() and nan.sum() == M + N - 1
    assert np.array_equal(np.isnan(got), nan)
    assert rel_frobenius(np.where(nan, 0, got), np.where(nan, 0, want)) <= 1e-4


@pytest.mark.parametrize("M,K,N,batch", [(32, 64, 48, 1), (17, 100, 33, 1), (8, 16, 8, 3)])
@pytest.mark.parametrize("ref", [False, True])
def test_gemm_f32(oracle, ops, M, K, N, batch, ref):
    A = D.uniform((batch, M, K), -1, 1, 60)
    B = D.uniform((batch, K, N), -1, 1, 61)
    C0 = D.uniform((batch, M, N), -1, 1, 62)
    alpha, beta = 0.5, 2.0
    C = ops.dev(C0)
    if batch == 1:
        fn = "lhq_gemm_f32_ref" if ref else "lhq_gemm_f32"
        ops.run(fn, A[0], B[0], C, M, N, K, alpha, beta)
        want = (oracle.gemm_ref if ref else oracle.gemm)(A[0], B[0], C0[0], alpha, beta)[None]
    else:
        if ref:
            pytest.skip("gemm_ref has no batched form")
        ops.run("lhq_gemm_f32_batched", A, B, C, batch, M, N, K, alpha, beta)
        want = oracle.gemm_batched(A, B, C0, alpha, beta)
    assert rel_frobenius(ops.host(C), want) <= 1e-5
