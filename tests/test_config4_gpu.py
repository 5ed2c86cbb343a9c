"""Benchmark config 4 at its full size on the GPU: the ragged grouped W4A16
GEMM of a Mixtral-style MoE layer (8 experts, 512 tokens routed top-2, so
1024 rows over the device-side group table; moe.cpp:111-123 builds the
table, gemm.cpp:69-75 is the grouped contract), and the two grouped
launches of the quantized expert MLP around it (moe.cpp:150-196):

* the grouped GEMM itself, K = 4096, N = 14336;
* the SwiGLU gate/up launch, H = 4096, I = 14336 (gate and up interleaved
  by column tile, act = bf16(silu(A Wg) * (A Wu)));
* the down projection, K = 14336, N = 4096.

The grouped launches run both ways: without a workspace (one workgroup per
tile) and with one (the persistent launch that splits its left-over tiles
along K).  The GPU computes every output element.  The weights are random codes, fp16
scales and zero points (a GEMM does not care how they were made).  A sample
of rows x columns is checked against the oracle run on the same codes
sliced to those columns (the int4 format is per column, so the slice is
exact): every expert's first and last row plus random rows, and the first
and last 16-column tiles plus random columns.  Bars: relative Frobenius
<= 1e-2 on the bf16 outputs and > 99% of elements within one bf16 ulp of the
correctly rounded oracle value."""
import numpy as np
import pytest

from oracle import rel_frobenius
from tests import _data as D

pytestmark = pytest.mark.gpu

TOL_BF16 = 1e-2
T, E, TOPK, G = 512, 8, 2, 128


@pytest.fixture(scope="module")
def ops(lib):
    from longhornai_amd import ops as _ops
    return _ops


def _codes(oracle, g, K, N):
    p = g.integers(0, 256, (K // 2, N), dtype=np.uint8)
    s = oracle.f32_to_f16_n(g.uniform(0.0005, 0.004, (K // G, N)).astype(np.float32))
    z = g.integers(0, 16, (K // G, N), dtype=np.uint8)
    return p, s, z


def _routing(oracle, seed):
    ids = D.moe_routing(T, E, TOPK, seed)
    off, tok, _ = oracle.moe_dispatch_table(ids, E)
    assert off[-1] == T * TOPK
    return off, tok


def _sample(g, off, N):
    rows = []
    for e in range(E):
        lo, hi = int(off[e]), int(off[e + 1])
        if hi > lo:
            rows += [lo, hi - 1] + list(g.integers(lo, hi, 2))
    cols = np.concatenate([np.arange(16), np.arange(N - 16, N), g.choice(N, 32, replace=False)])
    return np.unique(rows), np.unique(cols)


def _expert_of(off, r):
    return int(np.searchsorted(off, r, side="right") - 1)


def _check(oracle, got, want):
    assert rel_frobenius(got, want) <= TOL_BF16, rel_frobenius(got, want)
    want_b = D.bf16_bits_to_f32(D.to_bf16_bits(oracle, want))
    assert (np.abs(got - want_b) <= np.abs(want_b) * 2.0 ** -7 + 1e-30).mean() > 0.99


def _workspace(ops, name, *dims):
    import torch
    n = getattr(ops.lib().cdll, name)(*dims)
    assert n > 0
    return torch.empty(n, dtype=torch.uint8, device="cuda"), n


def _grouped_launch(oracle, ops, K, N, seed, ws=False):
    """One grouped launch of lhq_gemm_w4a16_bf16_grouped (ws: the persistent
    lhq_gemm_w4a16_bf16_grouped_ws) over config 4's routing; returns (A,
    off, per-expert codes, full output)."""
    import torch
    g = D.rng(seed)
    off, tok = _routing(oracle, seed)
    X = D.to_bf16_bits(oracle, g.standard_normal((T, K)).astype(np.float32))
    A = np.ascontiguousarray(X[tok])
    codes = [_codes(oracle, g, K, N) for _ in range(E)]
    Ws = [ops.prepack_w4_asym(ops.dev(p), ops.dev(s), ops.dev(z), K, N, G) for p, s, z in codes]
    q, s, z = ops.pointer_tables(Ws)
    rows = A.shape[0]
    C = ops.zeros((rows, N), np.int16)
    print(f"config 4 grouped launch K={K} N={N} rows={rows} ws={ws}", flush=True)
    if ws:
        buf, n = _workspace(ops, "lhq_gemm_w4a16_bf16_grouped_workspace_bytes", E, rows, N, K, G)
        ops.run("lhq_gemm_w4a16_bf16_grouped_ws", A, off, q, s, z, C, E, rows, N, K, G, buf, n)
    else:
        ops.run("lhq_gemm_w4a16_bf16_grouped", A, off, q, s, z, C, E, rows, N, K, G)
    out = ops.host(C, np.uint16)
    del Ws, q, s, z, C
    torch.cuda.empty_cache()
    return g, A, off, codes, out


@pytest.mark.parametrize("ws", [False, True], ids=["grid", "persistent"])
@pytest.mark.parametrize("K,N", [(4096, 14336), (14336, 4096)], ids=["gate_shape", "down_shape"])
def test_config4_grouped_full_size(oracle, ops, K, N, ws):
    g, A, off, codes, out = _grouped_launch(oracle, ops, K, N, seed=40 + K // 4096, ws=ws)
    rows, cols = _sample(g, off, N)
    got, want = [], []
    for r in rows:
        p, s, z = codes[_expert_of(off, r)]
        want.append(oracle.gemm_w4a16_asym(A[r:r + 1], np.ascontiguousarray(p[:, cols]),
                                           np.ascontiguousarray(s[:, cols]), np.ascontiguousarray(z[:, cols]),
                                           len(cols), G)[0])
        got.append(D.bf16_bits_to_f32(out[r, cols]))
    _check(oracle, np.array(got), np.array(want))


@pytest.mark.parametrize("ws", [False, True], ids=["grid", "persistent"])
def test_config4_swiglu_gate_up_full_size(oracle, ops, ws):
    import torch
    H, I = 4096, 14336
    g = D.rng(47)
    off, tok = _routing(oracle, 47)
    X = D.to_bf16_bits(oracle, g.standard_normal((T, H)).astype(np.float32))
    A = np.ascontiguousarray(X[tok])
    gate = [_codes(oracle, g, H, I) for _ in range(E)]
    up = [_codes(oracle, g, H, I) for _ in range(E)]
    gu = []
    for (pg, sg, zg), (pu, su, zu) in zip(gate, up):
        wg = ops.prepack_w4_asym(ops.dev(pg), ops.dev(sg), ops.dev(zg), H, I, G)
        wu = ops.prepack_w4_asym(ops.dev(pu), ops.dev(su), ops.dev(zu), H, I, G)
        gu.append(ops.interleave_gate_up(wg, wu))
        del wg, wu
    q, s, z = ops.pointer_tables(gu)
    rows = A.shape[0]
    act = ops.zeros((rows, I), np.int16)
    print(f"config 4 SwiGLU gate/up launch H={H} I={I} rows={rows} ws={ws}", flush=True)
    if ws:
        buf, n = _workspace(ops, "lhq_gemm_w4a16_bf16_grouped_swiglu_workspace_bytes", E, rows, I, H, G)
        ops.run("lhq_gemm_w4a16_bf16_grouped_swiglu_ws", A, off, q, s, z, act, E, rows, I, H, G, buf, n)
    else:
        ops.run("lhq_gemm_w4a16_bf16_grouped_swiglu", A, off, q, s, z, act, E, rows, I, H, G)
    out = ops.host(act, np.uint16)
    del gu, q, s, z, act
    torch.cuda.empty_cache()
    rs, cols = _sample(g, off, I)
    got, want = [], []
    for r in rs:
        e = _expert_of(off, r)
        sl = lambda c: [np.ascontiguousarray(a[:, cols]) for a in c]  # noqa: E731
        gv = oracle.gemm_w4a16_asym(A[r:r + 1], *sl(gate[e]), len(cols), G)
        uv = oracle.gemm_w4a16_asym(A[r:r + 1], *sl(up[e]), len(cols), G)
        want.append(D.bf16_bits_to_f32(oracle.swiglu_bf16(gv, uv))[0])
        got.append(D.bf16_bits_to_f32(out[r, cols]))
    got, want = np.array(got), np.array(want)
    assert rel_frobenius(got, want) <= TOL_BF16, rel_frobenius(got, want)
    # the oracle value is already the bf16 act: compare within one ulp
    assert (np.abs(got - want) <= np.abs(want) * 2.0 ** -7 + 1e-30).mean() > 0.99
