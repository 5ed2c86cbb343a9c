"""Quantizers on the GPU vs the CPU oracle: bit-exact (quant.cpp:12-249).

Codes, scales and dequantized values are compared as raw bits.  Inputs cover
the reference tests' distributions (test_quant.cpp) plus the edge cases the
semantics define: all-zero rows (scale 1), exact rounding ties, values beyond
the clamp, NaN entries (ignored by max, code 0) and the e4m3 flush region.
"""
import numpy as np
import pytest

from tests import _data as D

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops(lib):
    from longhornai_amd import ops as _ops
    return _ops


def _bits(a):
    a = np.asarray(a)
    return a.view(np.uint32) if a.dtype == np.float32 else a


def _eq(got, want):
    assert np.array_equal(_bits(got), _bits(want))


def _rows_input(rows, dim, seed):
    x = D.uniform((rows, dim), -3, 3, seed)
    x[0] = 0.0                                   # all-zero row -> scale 1
    if rows > 2:
        x[1, : min(dim, 8)] = np.array([0.5, 1.5, 2.5, -0.5, -1.5, 127.0, -127.0, 3.0], np.float32)[: min(dim, 8)]
        x[2] = D.uniform((dim,), -1e-3, 1e-3, seed + 1)
        x[2, 0] = np.nan                          # NaN never wins the max; its code is 0
    return x


@pytest.mark.parametrize("rows,dim", [(8, 64), (33, 100), (4, 4096), (1, 1)])
@pytest.mark.parametrize("kind", ["q8", "fp8"])
def test_per_row(oracle, ops, rows, dim, kind):
    x = _rows_input(rows, dim, rows * 7 + dim)
    q_w, s_w = getattr(oracle, f"{kind}_quantize_per_row")(x)
    q = ops.empty((rows, dim), np.int8 if kind == "q8" else np.uint8)
    s = ops.empty((rows,), np.float32)
    ops.run(f"lhq_{kind}_quantize_per_row", x, q, s, rows, dim)
    _eq(ops.host(q), q_w)
    _eq(ops.host(s), s_w)
    d_w = getattr(oracle, f"{kind}_dequantize_per_row")(q_w, s_w)
    d = ops.empty((rows, dim), np.float32)
    ops.run(f"lhq_{kind}_dequantize_per_row", q, s, d, rows, dim)
    _eq(ops.host(d), d_w)


# the vectorised kernel (dim % 8 == 0, short and long rows) and the scalar
# kernel (dim % 8 != 0)
@pytest.mark.parametrize("rows,dim", [(2048, 4096), (2049, 4096), (3, 24), (5, 13), (6, 8192), (7, 4104)])
def test_per_row_bf16(oracle, ops, rows, dim):
    x = D.with_outliers(D.normal((rows, dim), 1.0, 5), 0.001, 20.0, 6)
    x[0] = 0.0
    xb = D.to_bf16_bits(oracle, x)
    q_w, s_w = oracle.q8_quantize_per_row_bf16(xb)
    q = ops.empty((rows, dim), np.int8)
    s = ops.empty((rows,), np.float32)
    ops.run("lhq_q8_quantize_per_row_bf16", xb, q, s, rows, dim)
    _eq(ops.host(q), q_w)
    _eq(ops.host(s), s_w)


# 4 | cols: 16-byte loads; otherwise one column per thread.  Row counts span
# one and many 64-row chunks of the max pass.
@pytest.mark.parametrize("rows,cols", [(16, 32), (4096, 1000), (7, 3), (130, 14336), (65, 6), (200, 1001)])
@pytest.mark.parametrize("kind", ["q8", "fp8"])
def test_per_col(oracle, ops, rows, cols, kind):
    x = D.uniform((rows, cols), -1, 1, rows + cols)
    x[:, 0] = 0.0                                 # all-zero column -> scale 1
    if cols > 2 and rows > 4:
        x[:4, 1] = [np.nan, 0.25, -1.5, 1.0]      # NaN never wins; its code is 0
        x[rows - 1, 2] = 40.0                     # the max in the last row chunk
    q_w, s_w = getattr(oracle, f"{kind}_quantize_per_col")(x)
    q = ops.empty((rows, cols), np.int8 if kind == "q8" else np.uint8)
    s = ops.empty((cols,), np.float32)
    ops.run(f"lhq_{kind}_quantize_per_col", x, q, s, rows, cols)
    _eq(ops.host(q), q_w)
    _eq(ops.host(s), s_w)
    d_w = getattr(oracle, f"{kind}_dequantize_per_col")(q_w, s_w)
    d = ops.empty((rows, cols), np.float32)
    ops.run(f"lhq_{kind}_dequantize_per_col", q, s, d, rows, cols)
    _eq(ops.host(d), d_w)


@pytest.mark.parametrize("n", [1024, 1, 1 << 20, 12345])
@pytest.mark.parametrize("kind", ["q8", "fp8"])
def test_per_tensor(oracle, ops, n, kind):
    x = D.uniform((n,), -3, 3, n)
    if n > 4:
        x[:4] = np.array([0.0, np.nan, 1e-30, -2.5], np.float32)
    q_w, s_w = getattr(oracle, f"{kind}_quantize_per_tensor")(x)
    q = ops.empty((n,), np.int8 if kind == "q8" else np.uint8)
    s = ops.empty((1,), np.float32)
    ops.run(f"lhq_{kind}_quantize_per_tensor", x, q, s, n)
    _eq(ops.host(q), q_w)
    assert ops.host(s).view(np.uint32)[0] == np.float32(s_w).view(np.uint32)
    d = ops.empty((n,), np.float32)
    ops.run(f"lhq_{kind}_dequantize_per_tensor", q, s, d, n)
    _eq(ops.host(d), getattr(oracle, f"{kind}_dequantize_per_tensor")(q_w, s_w))


def test_per_tensor_all_zero(oracle, ops):
    x = np.zeros(4096, np.float32)
    q = ops.empty((4096,), np.int8)
    s = ops.empty((1,), np.float32)
    ops.run("lhq_q8_quantize_per_tensor", x, q, s, 4096)
    assert ops.host(s)[0] == 1.0 and not ops.host(q).any()


@pytest.mark.parametrize("K,N,G", [(64, 16, 32), (8, 4, 4), (256, 48, 128), (4096, 1024, 128), (30, 5, 3)])
def test_q4_groupwise(oracle, ops, K, N, G):
    w = D.uniform((K, N), -1, 1, K + N)
    w[:G, 0] = 0.0  # an all-zero group -> scale 1
    p_w, s_w = oracle.q4_quantize_groupwise(w, G)
    p = ops.empty((K // 2, N), np.uint8)
    s = ops.empty((K // G, N), np.float32)
    ops.run("lhq_q4_quantize_groupwise", w, p, s, K, N, G)
    _eq(ops.host(p), p_w)
    _eq(ops.host(s), s_w)
    d = ops.empty((K, N), np.float32)
    ops.run("lhq_q4_dequantize_groupwise", p, s, d, K, N, G)
    _eq(ops.host(d), oracle.q4_dequantize_groupwise(p_w, s_w, K, N, G))


@pytest.mark.parametrize("K,N,G", [(256, 64, 128), (4096, 512, 128), (64, 8, 32)])
def test_q4a_groupwise(oracle, ops, K, N, G):
    w = D.normal((K, N), 0.02, K * 3 + N)
    w[:G, 0] = 0.0
    w[:G, 1] = 0.5  # one-signed group
    p_w, s_w, z_w = oracle.q4a_quantize_groupwise(w, G)
    p = ops.empty((K // 2, N), np.uint8)
    s = ops.empty((K // G, N), np.int16)
    z = ops.empty((K // G, N), np.uint8)
    ops.run("lhq_q4a_quantize_groupwise", w, p, s, z, K, N, G)
    _eq(ops.host(p), p_w)
    _eq(ops.host(s, np.uint16), s_w)
    _eq(ops.host(z), z_w)
    d = ops.empty((K, N), np.float32)
    ops.run("lhq_q4a_dequantize_groupwise", p, s, z, d, K, N, G)
    _eq(ops.host(d), oracle.q4a_dequantize_groupwise(p_w, s_w, z_w, K, N, G))


def test_per_col_config3_weights(oracle, ops):
    """Config 3's weight quantization at full size (K=4096, N=14336, per
    output channel), with a spike per column at a random row."""
    K, N = 4096, 14336
    w = D.normal((K, N), 0.02, 31)
    w[D.rng(32).integers(0, K, N), np.arange(N)] = 0.5
    q_w, s_w = oracle.q8_quantize_per_col(w)
    q = ops.empty((K, N), np.int8)
    s = ops.empty((N,), np.float32)
    ops.run("lhq_q8_quantize_per_col", w, q, s, K, N)
    _eq(ops.host(q), q_w)
    _eq(ops.host(s), s_w)


def test_per_col_unaligned_rows(oracle, ops):
    """4 | cols but a source 4 bytes past a 16-byte boundary: the scalar
    kernels, same bits."""
    rows, cols = 70, 64
    x = D.uniform((rows, cols), -2, 2, 33)
    buf = ops.dev(np.concatenate([np.zeros(1, np.float32), x.ravel()]))
    src = buf[1:]
    assert src.data_ptr() % 16 == 4
    q = ops.empty((rows, cols), np.int8)
    s = ops.empty((cols,), np.float32)
    ops.run("lhq_q8_quantize_per_col", src, q, s, rows, cols)
    q_w, s_w = oracle.q8_quantize_per_col(x)
    _eq(ops.host(q), q_w)
    _eq(ops.host(s), s_w)


def test_per_col_zero_rows(oracle, ops):
    """rows = 0: every scale is 1 (the reference's max of nothing is 0)."""
    s = ops.dev(np.full(9, 7.0, np.float32))
    q = ops.empty((1,), np.int8)
    ops.run("lhq_q8_quantize_per_col", ops.empty((1,), np.float32), q, s, 0, 9)
    assert (ops.host(s) == 1.0).all()
