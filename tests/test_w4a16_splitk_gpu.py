"""W4A16 with a caller workspace (lhq_gemm_w4a16_bf16_ws) vs the CPU oracle.

At 2..64 rows the tile kernel's output grid cannot fill the GPU, nor at
65..512 rows where it fills at most half the CUs (there with at most
K / (8 M) splits), so K is split across workgroups: each split writes fp32
partial sums to the
workspace and a second kernel adds them in split order.  Checked here: the
three row-block forms (16, 32 and 64 rows per wave; 16-row blocks, and 32-
or 64-row blocks at K >= 16384, with K in two halves inside the workgroup),
ragged M and N, split boundaries inside scale groups, G = 128, 256 and 384,
the workspace-size rules (none, smaller than asked, exactly asked) and
bit-for-bit determinism across calls.  Bars as the other bf16 tests:
relative Frobenius <= 1e-2, and > 99.9% of elements within one bf16 ulp of
the correctly rounded oracle value."""
import numpy as np
import pytest

from oracle import rel_frobenius
from tests import _data as D

pytestmark = pytest.mark.gpu

TOL_BF16 = 1e-2


@pytest.fixture(scope="module")
def ops(lib):
    from longhornai_amd import ops as _ops
    return _ops


def _ulp_close(got, want_f32, oracle, frac=0.999):
    want_b = D.bf16_bits_to_f32(D.to_bf16_bits(oracle, want_f32))
    return (np.abs(got - want_b) <= np.abs(want_b) * 2.0 ** -7 + 1e-30).mean() > frac


def _case(oracle, ops, M, K, N, G, seed):
    A = D.to_bf16_bits(oracle, D.normal((M, K), 1.0, seed))
    p, s, z = oracle.q4a_quantize_groupwise(D.normal((K, N), 0.02, seed + 1), G)
    want = oracle.gemm_w4a16_asym(A, p, s, z, N, G)
    w = ops.prepack_w4_asym(ops.dev(p), ops.dev(s), ops.dev(z), K, N, G)
    return ops.dev(A), w, want


# 2..64 rows on the tile kernel, where the ordinary launch is the tile
# kernel or the weights hold K * N >= 32 Mi values (2..16 rows: at least
# three splits and larger weights the fewer the rows)
@pytest.mark.parametrize("M,K,N,G", [
    (16, 8192, 10240, 128),   # 16-row blocks, 4 splits
    (11, 8192, 10248, 256),   # 16-row blocks, 11 live rows, N % 16 != 0, G = 256
    (4, 16384, 8192, 128),    # 4 rows, K >= 16384
    (17, 4096, 8200, 128),    # 32-row blocks, N % 16 != 0
    (32, 2048, 16400, 256),   # G = 256: two K tiles per scale group
    (48, 2048, 1024, 128),    # 64-row blocks, 48 live rows
    (56, 1152, 2048, 384),    # G = 384: split boundary inside a scale group
    (64, 8192, 1024, 128),    # config 5 K
    (64, 4096, 4104, 128),    # ragged N at 64 rows
    (24, 16384, 2064, 128),   # K >= 16384: 32-row blocks, K halves in the workgroup, odd K tiles per split
    (64, 16384, 1040, 128),   # K >= 16384: 64-row blocks, K halves in the workgroup, ragged N
    (100, 8192, 2048, 128),   # 65..512 rows: two row tiles, 36 live rows in the second, K / (8 M) splits
    (256, 8192, 4104, 128),   # four row tiles, ragged N
    (72, 16384, 1024, 256),   # K halves in the workgroup, G = 256
])
def test_splitk_matches_oracle(oracle, ops, M, K, N, G):
    A, w, want = _case(oracle, ops, M, K, N, G, seed=700 + M + N)
    need = ops.lib().lhq_gemm_w4a16_bf16_workspace_bytes(M, N, K, G)
    assert need > 0 and need % (M * N * 4) == 0, need
    ws = ops.w4a16_bf16_workspace(M, w)
    print(f"split-K M={M} K={K} N={N} G={G}: {need // (M * N * 4)} splits", flush=True)
    got = D.bf16_bits_to_f32(ops.host(ops.gemm_w4a16_bf16_ws(A, w, ws), np.uint16))
    assert rel_frobenius(got, want) <= TOL_BF16
    assert _ulp_close(got, want, oracle)


def test_splitk_deterministic_and_workspace_rules(oracle, ops):
    """Same inputs, same workspace size: identical bits on every call.  A
    workspace smaller than asked runs fewer splits and one of none runs
    unsplit; both stay within the bars."""
    for M, K, N, G in ((24, 4096, 8192, 128), (64, 8192, 2048, 128)):
        _deterministic(oracle, ops, M, K, N, G)


def _deterministic(oracle, ops, M, K, N, G):
    A, w, want = _case(oracle, ops, M, K, N, G, seed=77 + M)
    ws = ops.w4a16_bf16_workspace(M, w)
    outs = [ops.host(ops.gemm_w4a16_bf16_ws(A, w, ws), np.uint16) for _ in range(3)]
    assert all(np.array_equal(outs[0], o) for o in outs[1:])
    small = ops.empty((2 * M * N * 4,), np.uint8)         # room for two splits
    none = ops.gemm_w4a16_bf16_ws(A, w, None)
    for got in (outs[0], ops.host(ops.gemm_w4a16_bf16_ws(A, w, small), np.uint16), ops.host(none, np.uint16)):
        got = D.bf16_bits_to_f32(got)
        assert rel_frobenius(got, want) <= TOL_BF16
        assert _ulp_close(got, want, oracle)


def test_splitk_workspace_bytes_rules(ops):
    def f(M, K, N, G):
        return ops.lib().lhq_gemm_w4a16_bf16_workspace_bytes(M, N, K, G)
    assert f(1, 8192, 8192, 128) == 0        # M = 1: the integer decode kernel
    assert f(4096, 8192, 8192, 128) == 0     # a full grid
    assert f(4, 4096, 4096, 128) == 0        # rows fit in LDS and the columns fill the GPU
    assert f(64, 4096, 8192, 64) == 0        # the tile kernel needs G >= 128
    assert f(64, 4160, 8192, 64) == 0        # (and so K % 128 == 0)
    assert f(0, 8192, 8192, 128) == 0
    assert f(16, 8192, 10240, 128) == 4 * 16 * 10240 * 4   # 16-row blocks, 4 splits
    assert f(16, 8192, 8192, 128) == 0       # one round of the 16-row kernel
    assert f(2, 28672, 8192, 128) == 0       # 2 rows: the 16-row kernel
    assert f(16, 8192, 57344, 128) == 0      # 2 splits would not pay at 16 rows
    assert f(8, 8192, 8192, 128) == 0        # nor K < 16384 at 8 rows or fewer
    assert f(8, 28672, 8192, 128) > 0
    assert f(12, 4096, 4096, 128) == 0       # small weights
    assert f(4, 16384, 4096, 128) == 0       # (up to 8 rows, N < 8192)
    assert f(32, 4096, 4096, 128) == 0       # small weights: the 16-row kernel
    assert f(32, 4096, 8192, 128) > 0
    assert f(64, 8192, 8192, 128) == 8 * 64 * 8192 * 4   # 8 splits of 8 K tiles
    assert f(64, 8192, 14336, 128) == 8 * 64 * 14336 * 4  # two workgroups per CU, 8 K tiles each
    assert f(64, 8192, 28672, 128) == 4 * 64 * 28672 * 4  # 448 workgroups, not 560
    assert f(64, 8192, 57344, 128) == 0      # more than half a CU's worth of column groups
    assert f(128, 8192, 8192, 128) == 8 * 128 * 8192 * 4  # 64 workgroups unsplit: 8 splits (K / (8 M))
    assert f(512, 8192, 8192, 128) == 0      # 256 workgroups unsplit: more than half the CUs
    assert f(512, 4096, 4096, 128) == 0      # K / (8 M) = 1
    assert f(513, 8192, 1024, 128) == 0      # beyond 512 rows


@pytest.mark.parametrize("M,K,N,G", [(4, 4096, 4096, 128), (64, 4160, 1024, 64)])
def test_unsplit_shapes_through_ws_entry(oracle, ops, M, K, N, G):
    """Shapes that need no workspace run the ordinary kernels through the
    workspace entry point too."""
    A, w, want = _case(oracle, ops, M, K, N, G, seed=900 + M)
    assert ops.lib().lhq_gemm_w4a16_bf16_workspace_bytes(M, N, K, G) == 0
    got = D.bf16_bits_to_f32(ops.host(ops.gemm_w4a16_bf16_ws(A, w, None), np.uint16))
    assert rel_frobenius(got, want) <= TOL_BF16
    assert _ulp_close(got, want, oracle)


@pytest.mark.parametrize("K,N", [(8192, 10240), (8192, 8192), (8192, 57344), (28672, 8192), (8192, 28672),
                                 (8192, 14336)])
def test_splitk_config5_m64_sampled(oracle, ops, K, N):
    """Config 5 at M = 64 through the workspace entry point, whole output on
    the GPU, sampled rows x columns against the oracle on column slices."""
    import torch
    M, G = 64, 128
    g = D.rng(1064 + N)
    p = g.integers(0, 256, (K // 2, N), dtype=np.uint8)
    s = oracle.f32_to_f16_n(g.uniform(0.0005, 0.004, (K // G, N)).astype(np.float32))
    z = g.integers(0, 16, (K // G, N), dtype=np.uint8)
    A = D.to_bf16_bits(oracle, g.standard_normal((M, K)).astype(np.float32))
    w = ops.prepack_w4_asym(ops.dev(p), ops.dev(s), ops.dev(z), K, N, G)
    ws = ops.w4a16_bf16_workspace(M, w)
    C = ops.host(ops.gemm_w4a16_bf16_ws(ops.dev(A), w, ws), np.uint16)
    del w, ws
    torch.cuda.empty_cache()
    rows = np.unique(np.concatenate([g.choice(M, 12, replace=False), [0, M - 1]]))
    cols = np.unique(np.concatenate([g.choice(N, 48, replace=False), np.arange(16), np.arange(N - 16, N)]))
    want = oracle.gemm_w4a16_asym(np.ascontiguousarray(A[rows]), np.ascontiguousarray(p[:, cols]),
                                  np.ascontiguousarray(s[:, cols]), np.ascontiguousarray(z[:, cols]), len(cols), G)
    got = D.bf16_bits_to_f32(C[np.ix_(rows, cols)])
    assert rel_frobenius(got, want) <= TOL_BF16
    assert _ulp_close(got, want, oracle, frac=0.99)
