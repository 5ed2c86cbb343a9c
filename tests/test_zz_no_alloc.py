"""The no-allocation W4A16 entry point (lhq_gemm_w4a16_bf16_noalloc) against
the workspace entry point it mirrors (lhq_gemm_w4a16_bf16_ws), through the C
ABI, on the GPU.

The two share the split-K plan, so with the workspace the shape asks for the
outputs must be bit-identical.  Two calls in a row, the second with a smaller
input, check that the static scratch carries nothing from one call into the
next; both outputs are also held to the oracle at the bf16 bar (relative
Frobenius <= 1e-2).  A captured HIP graph of one call is replayed with new
inputs between replays."""
import numpy as np
import pytest

from oracle import rel_frobenius
from tests import _data as D

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops(lib):
    from longhornai_amd import ops as _ops
    return _ops


def _case(oracle, ops, M, K, N, seed):
    A = D.to_bf16_bits(oracle, D.normal((M, K), 1.0, seed))
    p, s, z = oracle.q4a_quantize_groupwise(D.normal((K, N), 0.02, seed + 1), 128)
    w = ops.prepack_w4_asym(ops.dev(p), ops.dev(s), ops.dev(z), K, N, 128)
    return ops.dev(A), w, oracle.gemm_w4a16_asym(A, p, s, z, N, 128)


def test_noalloc_matches_workspace_entry_on_consecutive_calls(oracle, ops):
    # the second call is smaller (fewer rows, shorter K, less scratch), and
    # both split K
    for M, K, N in ((64, 8192, 8192), (24, 4096, 8192)):
        A, w, want = _case(oracle, ops, M, K, N, seed=M + N)
        need = ops.lib().lhq_gemm_w4a16_bf16_workspace_bytes(M, N, K, 128)
        print(f"noalloc M={M} K={K} N={N}: {need} bytes of scratch", flush=True)
        assert need > 0
        ref = ops.host(ops.gemm_w4a16_bf16_ws(A, w, ops.w4a16_bf16_workspace(M, w)), np.uint16)
        got = ops.host(ops.gemm_w4a16_bf16_noalloc(A, w, ops.empty((M, N), np.int16)), np.uint16)
        assert np.array_equal(got, ref)
        assert rel_frobenius(D.bf16_bits_to_f32(got), want) <= 1e-2


def test_noalloc_unsplit_shape(oracle, ops):
    """A shape that needs no scratch (M = 4) runs the ordinary kernels."""
    M, K, N = 4, 4096, 4096
    A, w, want = _case(oracle, ops, M, K, N, seed=5)
    assert ops.lib().lhq_gemm_w4a16_bf16_workspace_bytes(M, N, K, 128) == 0
    got = ops.host(ops.gemm_w4a16_bf16_noalloc(A, w, ops.empty((M, N), np.int16)), np.uint16)
    ref = ops.host(ops.gemm_w4a16_bf16(A, w), np.uint16)
    assert np.array_equal(got, ref)
    assert rel_frobenius(D.bf16_bits_to_f32(got), want) <= 1e-2


def test_noalloc_in_a_captured_hip_graph(oracle, ops):
    """The callers this entry point is for capture it in HIP graphs: a graph
    holding one call (split-K kernel + reduce, no allocation, no memset) is
    replayed three times with new activations written into its input and the
    output cleared eagerly between replays; every replay must equal the
    workspace entry point's eager result for that input, bit for bit."""
    import torch
    M, K, N = 64, 8192, 8192
    A, w, _ = _case(oracle, ops, M, K, N, seed=11)
    assert ops.lib().lhq_gemm_w4a16_bf16_workspace_bytes(M, N, K, 128) > 0
    C = ops.empty((M, N), np.int16)
    ws = ops.w4a16_bf16_workspace(M, w)
    ops.gemm_w4a16_bf16_noalloc(A, w, C)  # first call on the device: the scratch lookup happens here
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            ops.gemm_w4a16_bf16_noalloc(A, w, C)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    for rep in range(3):
        A_new = ops.dev(D.to_bf16_bits(oracle, D.normal((M, K), 1.0, 100 + rep)))
        A.copy_(A_new)
        C.zero_()
        want = ops.host(ops.gemm_w4a16_bf16_ws(A, w, ws), np.uint16)
        g.replay()
        torch.cuda.synchronize()
        print(f"graph replay {rep}", flush=True)
        assert np.array_equal(ops.host(C, np.uint16), want), f"replay {rep}"
