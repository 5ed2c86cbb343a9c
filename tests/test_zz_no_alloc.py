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


def test_noalloc_first_call_under_graph_capture():
    """The first call in a process, where the scratch address is looked up,
    may itself be under graph capture: a fresh process captures its very
    first no-alloc call and replays the graph against the workspace entry
    point (tests/noalloc_capture_first.py)."""
    import os
    import subprocess
    import sys
    script = os.path.join(os.path.dirname(os.path.abspath(__file__)), "noalloc_capture_first.py")
    r = subprocess.run([sys.executable, "-u", script], capture_output=True, text=True, timeout=300)
    print(r.stdout, r.stderr[-2000:], flush=True)
    assert r.returncode == 0 and r.stdout.strip().endswith("ok"), r.stderr[-2000:]


def test_noalloc_caps_a_plan_above_the_scratch(ops):
    """A shape whose split plan asks for more than the 32 MiB scratch (16 rows
    at K = 131072) runs the workspace entry point's plan with a 32 MiB
    workspace: fewer splits, bit-identical results."""
    import torch
    cap = 32 << 20
    M, K, N, G = 16, 131072, 16384, 128
    need = ops.lib().lhq_gemm_w4a16_bf16_workspace_bytes(M, N, K, G)
    print(f"noalloc M={M} K={K} N={N}: plan asks {need} bytes, scratch {cap}", flush=True)
    assert need > cap
    gen = torch.Generator(device="cuda")
    gen.manual_seed(31)
    q, s, z = ops.w4_buffers(K, N, G, True)
    q.copy_(torch.randint(0, 256, q.shape, dtype=torch.uint8, device="cuda", generator=gen))
    s.copy_((torch.rand(s.shape, device="cuda", generator=gen) * 0.001).half().view(torch.int16))
    z.copy_(torch.randint(-2**31, 2**31 - 1, z.shape, dtype=torch.int32, device="cuda", generator=gen))
    w = ops.W4Weights(q, s, z, K, N, G, True)
    A = torch.randn((M, K), device="cuda", generator=gen).to(torch.bfloat16).view(torch.int16)
    ws = ops.empty((cap,), np.uint8)
    ref = ops.host(ops.gemm_w4a16_bf16_ws(A, w, ws), np.uint16)
    full = ops.host(ops.gemm_w4a16_bf16_ws(A, w, ops.empty((need,), np.uint8)), np.uint16)
    for rep in range(2):
        got = ops.host(ops.gemm_w4a16_bf16_noalloc(A, w, ops.empty((M, N), np.int16)), np.uint16)
        assert np.array_equal(got, ref), rep
    # the capped plan is a different split of the same sums: within the bf16 bar of the full one
    assert rel_frobenius(D.bf16_bits_to_f32(got), D.bf16_bits_to_f32(full)) <= 1e-2
    del q, s, z, w, ws
    torch.cuda.empty_cache()
