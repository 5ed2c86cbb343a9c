"""The reference's fp32 interface with a caller workspace (lhq_gemm_w4a16_ws;
gemm_w4a16_groupwise, gemm_quant.hpp:47-57 / gemm_quant.cpp:54-82) vs the
CPU oracle.

At 2..64 rows (group size a multiple of 128, K % 128 == 0; at 2..16 rows
only where K * N >= 32 Mi), and at 65..512 rows where the unsplit grid
leaves a CU idle (with at most K / (8 M) splits), K is split across
workgroups: each split writes
fp32 partial sums to the workspace, and a second kernel adds them in split
order and applies alpha / beta as the reference does (beta == 0 never reads
C).  Checked: 16-, 32- and 64-row blocks with ragged M and N, split
boundaries inside scale groups (G = 256, 384), alpha / beta, NaN in C at
beta = 0, the workspace-size rules (none, smaller than asked, exactly asked,
contents irrelevant) and bit-for-bit determinism.  Bar: relative Frobenius
<= 1e-4 (fp32 activations split into bf16 hi + lo on the matrix cores)."""
import numpy as np
import pytest

from oracle import rel_frobenius
from tests import _data as D

pytestmark = pytest.mark.gpu

TOL_F32 = 1e-4


@pytest.fixture(scope="module")
def ops(lib):
    from longhornai_amd import ops as _ops
    return _ops


def _ws_bytes(ops, M, K, N, G):
    return ops.lib().cdll.lhq_gemm_w4a16_workspace_bytes(M, N, K, G)


def _case(oracle, ops, M, K, N, G, seed, alpha=1.0, beta=0.0):
    A = D.uniform((M, K), -1, 1, seed)
    Bp, Bs = oracle.q4_quantize_groupwise(D.uniform((K, N), -1, 1, seed + 1), G)
    C0 = D.uniform((M, N), -1, 1, seed + 2)
    want = oracle.gemm_w4a16_groupwise(A, Bp, Bs, N, G, C0, alpha, beta)
    w = ops.prepack_w4_sym(ops.dev(Bp), ops.dev(Bs), K, N, G)
    return ops.dev(A), w, C0, want


def _run(ops, A, w, C0, alpha, beta, ws_bytes, fill=None):
    import torch
    M = A.shape[0]
    C = ops.dev(C0)
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device="cuda")
    if fill is not None:
        ws.fill_(fill)
    print(f"gemm_w4a16_ws M={M} K={w.K} N={w.N} G={w.G} alpha={alpha} beta={beta} ws={ws_bytes}", flush=True)
    ops.run("lhq_gemm_w4a16_ws", A, w.qweight, w.scales, C, M, w.N, w.K, w.G, alpha, beta,
            ws if ws_bytes else None, ws_bytes)
    return ops.host(C)


@pytest.mark.parametrize("M,K,N,G,alpha,beta", [
    (2, 4096, 8192, 128, 1.0, 0.0),        # 2 rows, K * N = 32 Mi
    (5, 8192, 4104, 256, 0.5, 2.0),        # N % 16 != 0, G = 256, alpha / beta
    (16, 8192, 4096, 128, 1.0, 0.0),       # 16-row blocks
    (16, 2304, 16384, 384, -1.0, 1.0),     # G = 384: split boundaries inside scale groups
    (17, 1024, 1040, 128, 1.0, 0.0),       # 32-row blocks, 17 live rows, ragged N
    (24, 4096, 2048, 128, 2.0, -0.5),
    (32, 2048, 1000, 256, 1.0, 0.0),
    (33, 1152, 512, 128, 1.0, 0.0),        # 64-row blocks, 33 live rows, 9 K tiles
    (48, 4096, 1024, 128, 1.0, 1.0),
    (64, 8192, 512, 128, 0.5, 0.0),        # config 5 K
    (80, 8192, 1024, 128, 1.0, 0.0),       # 65..512 rows: two row tiles, 16 live rows in the second
    (200, 4096, 1536, 256, 0.5, 1.0),      # four row tiles, G = 256, alpha / beta, 2 splits (K / (8 M))
    (130, 16384, 520, 128, 1.0, 0.0),      # ragged N, odd K tiles per split
])
def test_f32_splitk_matches_oracle(oracle, ops, M, K, N, G, alpha, beta):
    A, w, C0, want = _case(oracle, ops, M, K, N, G, seed=2100 + M + K // 128, alpha=alpha, beta=beta)
    n = _ws_bytes(ops, M, K, N, G)
    assert n > 0 and n % (M * N * 4) == 0 and n // (M * N * 4) >= 2   # split
    got = _run(ops, A, w, C0, alpha, beta, n, fill=0x7F)
    err = rel_frobenius(got, want)
    assert err <= TOL_F32, f"rel Frobenius {err:.3e}"


def test_f32_splitk_beta0_ignores_nan_in_c(oracle, ops):
    M, K, N, G = 24, 2048, 768, 128
    A, w, _, want = _case(oracle, ops, M, K, N, G, seed=2300)
    got = _run(ops, A, w, np.full((M, N), np.nan, np.float32), 1.0, 0.0, _ws_bytes(ops, M, K, N, G))
    assert np.isfinite(got).all()
    assert rel_frobenius(got, want) <= TOL_F32


def test_f32_splitk_deterministic_and_workspace_rules(oracle, ops):
    """Same inputs and workspace size: identical bits on every call, whatever
    the workspace held.  A workspace smaller than asked runs fewer splits;
    none runs lhq_gemm_w4a16's kernels, bit for bit."""
    M, K, N, G = 32, 4096, 2048, 128
    A, w, C0, want = _case(oracle, ops, M, K, N, G, seed=2400, alpha=0.75, beta=0.5)
    n = _ws_bytes(ops, M, K, N, G)
    outs = [_run(ops, A, w, C0, 0.75, 0.5, n, fill=f) for f in (0, 0xFF, 0x41)]
    assert all(np.array_equal(outs[0].view(np.uint32), o.view(np.uint32)) for o in outs[1:])
    small = _run(ops, A, w, C0, 0.75, 0.5, 2 * M * N * 4)   # room for two splits
    none = _run(ops, A, w, C0, 0.75, 0.5, 0)
    plain = ops.dev(C0)
    ops.gemm_w4a16(A, w, plain, 0.75, 0.5)
    assert np.array_equal(none.view(np.uint32), ops.host(plain).view(np.uint32))
    for got in (outs[0], small, none):
        assert rel_frobenius(got, want) <= TOL_F32


def test_f32_splitk_workspace_bytes_rules(ops):
    def f(M, K, N, G):
        return _ws_bytes(ops, M, K, N, G)
    assert f(1, 8192, 28672, 128) == 0       # one row: no split
    assert f(513, 8192, 1024, 128) == 0      # beyond 512 rows
    assert f(4096, 8192, 8192, 128) == 0     # a full grid
    assert f(0, 8192, 8192, 128) == 0
    assert f(16, 4096, 4096, 128) == 0       # 2..16 rows with K * N < 32 Mi
    assert f(2, 4096, 4096, 128) == 0
    assert f(2, 4096, 8192, 128) > 0         # K * N = 32 Mi
    assert f(17, 1024, 1024, 128) > 0        # 17..64 rows: always
    assert f(32, 8192, 8192, 64) == 0        # G < 128
    assert f(32, 8320, 8192, 64) == 0        # (and K % 128 != 0)
    # about two workgroups per CU: 112 column groups of 256 at N = 28672 -> 4 splits on 256 CUs
    import torch
    if torch.cuda.get_device_properties(0).multi_processor_count == 256:
        assert f(16, 8192, 28672, 128) == 4 * 16 * 28672 * 4
        assert f(64, 8192, 8192, 128) == 16 * 64 * 8192 * 4   # 32 groups, 16 splits of 4 K tiles
        assert f(128, 8192, 8192, 128) == 8 * 128 * 8192 * 4  # 64 workgroups unsplit, 8 splits (K / (8 M))
        assert f(512, 8192, 8192, 128) == 2 * 512 * 8192 * 4  # 256 workgroups unsplit: 2 splits
        assert f(1024, 8192, 8192, 128) == 0  # 512 workgroups unsplit
        assert f(512, 4096, 4096, 128) == 0   # K / (8 M) = 1


def test_f32_splitk_in_a_captured_hip_graph(oracle, ops):
    """The split (tile kernel + reduce) allocates nothing and records no
    memset: a captured call replayed three times with new activations, C
    reset eagerly between replays (beta = 0.5 reads it), equals the eager
    call bit for bit each time."""
    import torch
    M, K, N, G = 16, 8192, 4096, 128
    A, w, C0, _ = _case(oracle, ops, M, K, N, G, seed=2500, alpha=1.5, beta=0.5)
    n = _ws_bytes(ops, M, K, N, G)
    assert n > 0
    ws = torch.empty(n, dtype=torch.uint8, device="cuda")
    C = ops.dev(C0)
    C0d = ops.dev(C0)
    L = ops.lib().cdll

    def call():
        st = L.lhq_gemm_w4a16_ws(A.data_ptr(), w.qweight.data_ptr(), w.scales.data_ptr(), C.data_ptr(), M, N, K,
                                 G, 1.5, 0.5, ws.data_ptr(), n, ops.stream())
        assert st == 0, ops.lib().last_error()

    call()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        with torch.cuda.graph(g, stream=st):
            call()
    torch.cuda.current_stream().wait_stream(st)
    torch.cuda.synchronize()
    for rep in range(3):
        A.copy_(ops.dev(D.uniform((M, K), -1, 1, 2600 + rep)))
        C.copy_(C0d)
        call()
        want = ops.host(C).copy()
        C.copy_(C0d)
        g.replay()
        torch.cuda.synchronize()
        print(f"fp32 split graph replay {rep}", flush=True)
        assert np.array_equal(ops.host(C).view(np.uint32), want.view(np.uint32)), f"replay {rep}"
