"""W4A16 GEMM on the GPU vs the CPU oracle (gemm_quant.cpp:54-82).

Tolerances (north star): relative Frobenius error <= 1e-4 for fp32 outputs,
<= 1e-2 for bf16 outputs.  The fp32 path is the reference drop-in (fp32
activations, symmetric int4, fp32 scales); the bf16 path is the benchmark
configs' asymmetric int4 with fp16 scales and u4 zero points.
"""
import numpy as np
import pytest

from oracle import rel_frobenius
from tests import _data as D

pytestmark = pytest.mark.gpu

TOL_F32 = 1e-4
TOL_BF16 = 1e-2


@pytest.fixture(scope="module")
def ops(lib):
    from longhornai_amd import ops as _ops
    return _ops


def _sym_case(oracle, ops, M, K, N, G, seed, alpha=1.0, beta=0.0):
    A = D.uniform((M, K), -1, 1, seed)
    W = D.uniform((K, N), -1, 1, seed + 1)
    Bp, Bs = oracle.q4_quantize_groupwise(W, G)
    C0 = D.uniform((M, N), -1, 1, seed + 2)
    want = oracle.gemm_w4a16_groupwise(A, Bp, Bs, N, G, C0, alpha, beta)
    w = ops.prepack_w4_sym(ops.dev(Bp), ops.dev(Bs), K, N, G)
    C = ops.dev(C0)
    ops.gemm_w4a16(ops.dev(A), w, C, alpha, beta)
    got = ops.host(C)
    return got, want


@pytest.mark.parametrize("M,K,N,G", [
    (16, 64, 32, 32),        # test_gemm_quant.cpp:56-57 shape
    (1, 4096, 4096, 128),
    (4, 4096, 11008, 128),
    (16, 11008, 4096, 128),
    (3, 256, 48, 64),
    (17, 512, 100, 32),
    (40, 1024, 272, 256),
    (1, 8192, 28672, 128),   # decode target shape, fp32 API
    (2, 96, 40, 32),         # K not a multiple of the 128-wide tile
    (7, 4160, 72, 64),
    (16, 28672, 64, 128),    # activations too large to stage: generic kernel
    (1, 28672, 512, 128),    # integer decode with 88 KiB of digit planes, two column tiles per wave
])
def test_w4a16_f32_matches_oracle(oracle, ops, M, K, N, G):
    got, want = _sym_case(oracle, ops, M, K, N, G, seed=100 + M + K // 64)
    err = rel_frobenius(got, want)
    assert err <= TOL_F32, f"rel Frobenius {err:.3e}"


@pytest.mark.parametrize("alpha,beta", [(0.5, 2.0), (1.0, 1.0), (-1.25, 0.0), (2.0, -0.5)])
def test_w4a16_f32_alpha_beta(oracle, ops, alpha, beta):
    got, want = _sym_case(oracle, ops, 8, 256, 64, 32, seed=7, alpha=alpha, beta=beta)
    assert rel_frobenius(got, want) <= TOL_F32


def test_w4a16_f32_beta0_ignores_nan_in_c(oracle, ops):
    """apply_beta with beta == 0 writes zeros without reading C (gemm_quant.cpp:15-16)."""
    M, K, N, G = 4, 128, 32, 32
    A = D.uniform((M, K), -1, 1, 1)
    W = D.uniform((K, N), -1, 1, 2)
    Bp, Bs = oracle.q4_quantize_groupwise(W, G)
    want = oracle.gemm_w4a16_groupwise(A, Bp, Bs, N, G)
    w = ops.prepack_w4_sym(ops.dev(Bp), ops.dev(Bs), K, N, G)
    C = ops.dev(np.full((M, N), np.nan, np.float32))
    ops.gemm_w4a16(ops.dev(A), w, C, 1.0, 0.0)
    got = ops.host(C)
    assert np.isfinite(got).all()
    assert rel_frobenius(got, want) <= TOL_F32


# The fp32 interface at 2..32 rows on the tile kernel's 16- and 32-row blocks
# with K split across the waves of a workgroup (where the launch picks it;
# every layout is also run by forcing it in the sweep build): ragged K
# (K parts of unequal length, and an empty last part at Kt = 9 in quarters),
# partial column groups, G = 256, alpha / beta.
@pytest.mark.parametrize("M,K,N,G,alpha,beta", [
    (2, 1024, 96, 128, 1.0, 0.0),
    (5, 1152, 200, 128, 0.5, 2.0),
    (16, 4096, 4096, 128, 1.0, 0.0),
    (16, 8192, 1040, 256, -1.0, 1.0),
    (17, 2304, 272, 128, 1.0, 0.0),
    (24, 1152, 4096, 128, 2.0, -0.5),
    (32, 8192, 2048, 128, 1.0, 0.0),
    # shapes the launch itself sends to the K-split layouts
    (16, 1024, 16384, 128, 1.0, 0.0),      # 16-row blocks, K quarters
    (24, 1152, 16384, 128, 0.5, 1.0),      # 32-row blocks, K quarters, an empty last quarter
    (40, 1024, 20480, 128, 1.0, 0.0),      # two 32-row tiles, K halves
    (20, 2048, 49152, 256, 1.0, 0.0),      # 32-row blocks, K halves, G = 256
])
def test_w4a16_f32_thin_tile(oracle, ops, M, K, N, G, alpha, beta):
    got, want = _sym_case(oracle, ops, M, K, N, G, seed=1700 + M + K // 128, alpha=alpha, beta=beta)
    err = rel_frobenius(got, want)
    assert err <= TOL_F32, f"rel Frobenius {err:.3e}"


# The fp32 interface on the prefill tile kernel (48+ rows, G >= 128, K a
# multiple of 128): fp32 activations split into bf16 hi + lo operands.
@pytest.mark.parametrize("M,K,N,G,alpha,beta", [
    (48, 512, 64, 128, 1.0, 0.0),
    (64, 128, 128, 128, 1.0, 0.0),       # one K tile
    (50, 384, 320, 128, 1.0, 0.0),       # three K tiles (an odd count), 14 dead rows
    (64, 1024, 272, 128, 1.0, 0.0),      # ragged column group
    (130, 2048, 512, 256, 1.0, 0.0),     # ragged row tile (2 rows), G = 256
    (96, 1024, 256, 128, 0.5, 2.0),
    (96, 1024, 256, 128, -1.25, 0.0),
    (256, 8192, 1024, 128, 1.0, 1.0),
])
def test_w4a16_f32_prefill_tile(oracle, ops, M, K, N, G, alpha, beta):
    got, want = _sym_case(oracle, ops, M, K, N, G, seed=300 + M, alpha=alpha, beta=beta)
    err = rel_frobenius(got, want)
    assert err <= TOL_F32, f"rel Frobenius {err:.3e}"


def test_w4a16_f32_prefill_tile_beta0_ignores_nan_in_c(oracle, ops):
    M, K, N, G = 64, 512, 256, 128
    A = D.uniform((M, K), -1, 1, 11)
    W = D.uniform((K, N), -1, 1, 12)
    Bp, Bs = oracle.q4_quantize_groupwise(W, G)
    want = oracle.gemm_w4a16_groupwise(A, Bp, Bs, N, G)
    w = ops.prepack_w4_sym(ops.dev(Bp), ops.dev(Bs), K, N, G)
    C = ops.dev(np.full((M, N), np.nan, np.float32))
    ops.gemm_w4a16(ops.dev(A), w, C, 1.0, 0.0)
    got = ops.host(C)
    assert np.isfinite(got).all()
    assert rel_frobenius(got, want) <= TOL_F32


def test_w4a16_f32_prefill_tile_deterministic(oracle, ops):
    """The fp32 tile path splits each row block into bf16 hi + lo in place in
    LDS and shares the halves between waves: repeated calls on the same
    inputs give the same bits (and stay within the bar), across a full grid
    of workgroups and several K tiles."""
    M, K, N, G = 256, 2048, 2048, 128
    A = D.uniform((M, K), -1, 1, 21)
    W = D.uniform((K, N), -1, 1, 22)
    Bp, Bs = oracle.q4_quantize_groupwise(W, G)
    want = oracle.gemm_w4a16_groupwise(A, Bp, Bs, N, G)
    w = ops.prepack_w4_sym(ops.dev(Bp), ops.dev(Bs), K, N, G)
    Ad = ops.dev(A)
    outs = []
    for _ in range(4):
        C = ops.zeros((M, N), np.float32)
        ops.gemm_w4a16(Ad, w, C, 1.0, 0.0)
        outs.append(ops.host(C))
    assert all(np.array_equal(outs[0].view(np.uint32), o.view(np.uint32)) for o in outs[1:])
    assert rel_frobenius(outs[0], want) <= TOL_F32


def test_w4a16_f32_prefill_config5_sampled(oracle, ops):
    """The fp32 interface at M=4096 on config 5's K=8192, N=28672: whole
    output on the GPU, sampled rows x columns against the oracle."""
    import torch
    M, K, N, G = 4096, 8192, 28672, 128
    g = D.rng(4096 + N)
    Bp = g.integers(0, 256, (K // 2, N), dtype=np.uint8)
    Bs = g.uniform(0.001, 0.01, (K // G, N)).astype(np.float32)
    A = g.uniform(-1, 1, (M, K)).astype(np.float32)
    w = ops.prepack_w4_sym(ops.dev(Bp), ops.dev(Bs), K, N, G)
    C = ops.zeros((M, N), np.float32)
    ops.gemm_w4a16(ops.dev(A), w, C, 1.0, 0.0)
    Ch = ops.host(C)
    del w, C
    torch.cuda.empty_cache()
    rows = np.unique(np.concatenate([g.choice(M, 10, replace=False), [0, 63, 64, M - 1]]))
    cols = np.unique(np.concatenate([g.choice(N, 40, replace=False), np.arange(16), np.arange(N - 16, N)]))
    want = oracle.gemm_w4a16_groupwise(np.ascontiguousarray(A[rows]), np.ascontiguousarray(Bp[:, cols]),
                                       np.ascontiguousarray(Bs[:, cols]), len(cols), G)
    assert rel_frobenius(Ch[np.ix_(rows, cols)], want) <= TOL_F32


def _asym_case(oracle, ops, M, K, N, G, seed):
    A = D.to_bf16_bits(oracle, D.normal((M, K), 1.0, seed))
    W = D.normal((K, N), 0.02, seed + 1)
    p, s, z = oracle.q4a_quantize_groupwise(W, G)
    want_f32 = oracle.gemm_w4a16_asym(A, p, s, z, N, G)
    w = ops.prepack_w4_asym(ops.dev(p), ops.dev(s), ops.dev(z), K, N, G)
    C = ops.gemm_w4a16_bf16(ops.dev(A), w)
    got = D.bf16_bits_to_f32(ops.host(C, np.uint16))
    return got, want_f32


@pytest.mark.parametrize("M,K,N", [
    (1, 4096, 4096), (4, 4096, 11008), (16, 11008, 4096),      # config 2
    (4, 11008, 4096),                                          # 86 KiB of staged activations
    (1, 8192, 10240), (8, 8192, 8192), (1, 28672, 8192),       # config 5 (decode M)
    (1, 8192, 28672),                                          # decode target
    (5, 384, 40),
])
def test_w4a16_bf16_matches_oracle(oracle, ops, M, K, N):
    got, want = _asym_case(oracle, ops, M, K, N, 128, seed=300 + M)
    err = rel_frobenius(got, want)
    # bf16 output rounding alone is ~2^-9 relative; the bound is the north star's.
    assert err <= TOL_BF16, f"rel Frobenius {err:.3e}"
    # and the result must be the correctly rounded value up to one bf16 ulp
    want_b = D.bf16_bits_to_f32(D.to_bf16_bits(oracle, want))
    ulp = np.abs(want_b) * 2.0 ** -7 + 1e-30
    assert (np.abs(got - want_b) <= ulp).mean() > 0.999


CONFIG2 = [(m, k, n) for m in (1, 4, 16) for k, n in ((4096, 4096), (4096, 11008), (11008, 4096))]


@pytest.mark.parametrize("M,K,N", CONFIG2)
def test_w4a16_config2_all_shapes(oracle, ops, M, K, N):
    """Benchmark config 2 (Llama-7B projections, M in {1, 4, 16}) at full size:
    all nine shapes, every output against the oracle."""
    got, want = _asym_case(oracle, ops, M, K, N, 128, seed=900 + M + K)
    assert rel_frobenius(got, want) <= TOL_BF16
    want_b = D.bf16_bits_to_f32(D.to_bf16_bits(oracle, want))
    assert (np.abs(got - want_b) <= np.abs(want_b) * 2.0 ** -7 + 1e-30).mean() > 0.999


CONFIG5_KN = [(8192, 10240), (8192, 8192), (8192, 57344), (28672, 8192)]  # qkv, o, gate_up, down


@pytest.mark.parametrize("M", [1, 8, 64, 4096])
@pytest.mark.parametrize("K,N", CONFIG5_KN)
def test_w4a16_config5_full_sampled(oracle, ops, M, K, N):
    """Benchmark config 5 (Llama-3-70B linears) at full size.  The weights are
    random codes, fp16 scales and zero points (a GEMM does not care how they
    were made); the GPU computes the whole [M, N] output, and a sample of rows
    x columns is checked against the oracle run on the same codes sliced to
    those columns (the int4 format is per column, so the slice is exact)."""
    import torch
    G = 128
    g = D.rng(1000 + M + N)
    p = g.integers(0, 256, (K // 2, N), dtype=np.uint8)
    s = oracle.f32_to_f16_n(g.uniform(0.0005, 0.004, (K // G, N)).astype(np.float32))
    z = g.integers(0, 16, (K // G, N), dtype=np.uint8)
    A = D.to_bf16_bits(oracle, g.standard_normal((M, K)).astype(np.float32))
    w = ops.prepack_w4_asym(ops.dev(p), ops.dev(s), ops.dev(z), K, N, G)
    C = ops.host(ops.gemm_w4a16_bf16(ops.dev(A), w), np.uint16)
    del w
    torch.cuda.empty_cache()
    rows = np.unique(np.concatenate([g.choice(M, min(M, 12), replace=False), [0, M - 1]]))
    cols = np.unique(np.concatenate([g.choice(N, 48, replace=False), [0, N - 1]]))
    want = oracle.gemm_w4a16_asym(np.ascontiguousarray(A[rows]), np.ascontiguousarray(p[:, cols]),
                                  np.ascontiguousarray(s[:, cols]), np.ascontiguousarray(z[:, cols]), len(cols), G)
    got = D.bf16_bits_to_f32(C[np.ix_(rows, cols)])
    assert rel_frobenius(got, want) <= TOL_BF16
    want_b = D.bf16_bits_to_f32(D.to_bf16_bits(oracle, want))
    assert (np.abs(got - want_b) <= np.abs(want_b) * 2.0 ** -7 + 1e-30).mean() > 0.99


@pytest.mark.parametrize("G", [32, 64, 256])
def test_w4a16_bf16_group_sizes(oracle, ops, G):
    got, want = _asym_case(oracle, ops, 3, 1024, 96, G, seed=G)
    assert rel_frobenius(got, want) <= TOL_BF16


@pytest.mark.parametrize("M,K,N,G", [(1, 96, 48, 32), (16, 320, 64, 64), (9, 4160, 136, 64)])
def test_w4a16_bf16_ragged_k(oracle, ops, M, K, N, G):
    """K not a multiple of 128: the padded tail of the last tile must add nothing."""
    got, want = _asym_case(oracle, ops, M, K, N, G, seed=K + M)
    assert rel_frobenius(got, want) <= TOL_BF16


# M = 1 with G = 64 or a multiple of 128 runs the integer-MFMA decode kernel,
# which holds activations as 21-bit fixed point per 128-wide K block.  These
# inputs spread magnitudes over 2^-12 .. 2^12 inside every block and zero a
# whole block, with one and two column tiles per wave (Nt < 1024 and >= 1024,
# odd Nt), G = 64 (also with a ragged last K tile), 128 and 256.
INT8_DECODE_CASES = [
    (1, 4096, 16400, 128),  # K <= 32 tiles with >= 896 column tiles: two waves per workgroup
    (1, 4096, 14336, 128),  # 896 column tiles: the two-wave rule's edge on 256 CUs
    (1, 1024, 272, 64),
    (1, 4160, 72, 64),
    (1, 2048, 16400, 256),
    (1, 640, 48, 64),
]


def _wide_range(M, K, seed):
    x = D.normal((M, K), 1.0, seed) * np.exp2(D.uniform((M, K), -12, 12, seed + 7)).astype(np.float32)
    x[:, 128:256] = 0.0  # one all-zero block per row
    return x.astype(np.float32)


@pytest.mark.parametrize("M,K,N,G", INT8_DECODE_CASES)
def test_w4a16_int8_decode_bf16_wide_range(oracle, ops, M, K, N, G):
    A = D.to_bf16_bits(oracle, _wide_range(M, K, 40 + M))
    p, s, z = oracle.q4a_quantize_groupwise(D.normal((K, N), 0.02, 41 + M), G)
    want = oracle.gemm_w4a16_asym(A, p, s, z, N, G)
    w = ops.prepack_w4_asym(ops.dev(p), ops.dev(s), ops.dev(z), K, N, G)
    got = D.bf16_bits_to_f32(ops.host(ops.gemm_w4a16_bf16(ops.dev(A), w), np.uint16))
    assert rel_frobenius(got, want) <= TOL_BF16


@pytest.mark.parametrize("M,K,N,G", INT8_DECODE_CASES)
def test_w4a16_int8_decode_f32_wide_range(oracle, ops, M, K, N, G):
    A = _wide_range(M, K, 50 + M)
    Bp, Bs = oracle.q4_quantize_groupwise(D.uniform((K, N), -1, 1, 51 + M), G)
    want = oracle.gemm_w4a16_groupwise(A, Bp, Bs, N, G)
    w = ops.prepack_w4_sym(ops.dev(Bp), ops.dev(Bs), K, N, G)
    C = ops.dev(np.zeros((M, N), np.float32))
    ops.gemm_w4a16(ops.dev(A), w, C, 1.0, 0.0)
    assert rel_frobenius(ops.host(C), want) <= TOL_F32


@pytest.mark.parametrize("M,K,N", [(1, 8192, 2048), (1, 4096, 1040)])
def test_w4a16_int8_decode_correctly_rounded(oracle, ops, M, K, N):
    """N(0,1) activations are exact in the fixed-point form: the bf16 output
    is the correctly rounded value up to one ulp."""
    G = 128
    A = D.to_bf16_bits(oracle, D.normal((M, K), 1.0, 61))
    p, s, z = oracle.q4a_quantize_groupwise(D.normal((K, N), 0.02, 62), G)
    want = oracle.gemm_w4a16_asym(A, p, s, z, N, G)
    w = ops.prepack_w4_asym(ops.dev(p), ops.dev(s), ops.dev(z), K, N, G)
    got = D.bf16_bits_to_f32(ops.host(ops.gemm_w4a16_bf16(ops.dev(A), w), np.uint16))
    want_b = D.bf16_bits_to_f32(D.to_bf16_bits(oracle, want))
    ulp = np.abs(want_b) * 2.0 ** -7 + 1e-30
    assert (np.abs(got - want_b) <= ulp).mean() > 0.999


@pytest.mark.parametrize("M", [5, 1])
def test_w4a16_bf16_batched(oracle, ops, M):
    """Uniform batches (grid.z): M=5 runs the bf16 decode kernel, M=1 the
    integer one; each matrix uses its own weights, scales and zeros."""
    import torch
    B, K, N, G = 3, 512, 80, 128
    As, Ws, wants = [], [], []
    for b in range(B):
        A = D.to_bf16_bits(oracle, D.normal((M, K), 1.0, 10 + b))
        p, s, z = oracle.q4a_quantize_groupwise(D.normal((K, N), 0.02, 20 + b), G)
        As.append(A)
        Ws.append(ops.prepack_w4_asym(ops.dev(p), ops.dev(s), ops.dev(z), K, N, G))
        wants.append(oracle.gemm_w4a16_asym(A, p, s, z, N, G))
    A_all = ops.dev(np.stack(As))
    q = torch.cat([w.qweight for w in Ws])
    s = torch.cat([w.scales for w in Ws])
    z = torch.cat([w.zeros for w in Ws])
    C = ops.empty((B, M, N), np.int16)
    ops.run("lhq_gemm_w4a16_bf16_batched", A_all, q, s, z, C, B, M, N, K, G)
    got = D.bf16_bits_to_f32(ops.host(C, np.uint16))
    for b in range(B):
        assert rel_frobenius(got[b], wants[b]) <= TOL_BF16


def _grouped(oracle, ops, T, E, topk, K, N, G, seed, empty_expert=None, one_expert=None,
             bad_tokens=()):
    import torch
    ids = D.moe_routing(T, E, topk, seed)
    if empty_expert is not None:
        ids[ids == empty_expert] = (empty_expert + 1) % E
    if one_expert is not None:  # every row on one expert (top-1 routing)
        ids[:] = one_expert
    off, tok, _ = oracle.moe_dispatch_table(ids, E)
    xf = D.normal((T, K), 1.0, seed + 1)
    for i, t in enumerate(bad_tokens):  # +Inf, -Inf, NaN in turn
        xf[t, (37 * i + 11) % K] = (np.inf, -np.inf, np.nan)[i % 3]
    X = D.to_bf16_bits(oracle, xf)
    A = X[tok]  # dispatched rows, expert-major, token order kept (moe.cpp:124-139)
    P_, S_, Z_ = [], [], []
    for e in range(E):
        p, s, z = oracle.q4a_quantize_groupwise(D.normal((K, N), 0.02, seed + 10 + e), G)
        P_.append(p); S_.append(s); Z_.append(z)
    want = oracle.gemm_w4a16_asym_grouped(A, off, np.stack(P_), np.stack(S_), np.stack(Z_), N, G)
    Ws = [ops.prepack_w4_asym(ops.dev(P_[e]), ops.dev(S_[e]), ops.dev(Z_[e]), K, N, G) for e in range(E)]
    qptr = torch.tensor([w.qweight.data_ptr() for w in Ws], dtype=torch.int64, device="cuda")
    sptr = torch.tensor([w.scales.data_ptr() for w in Ws], dtype=torch.int64, device="cuda")
    zptr = torch.tensor([w.zeros.data_ptr() for w in Ws], dtype=torch.int64, device="cuda")
    rows = A.shape[0]
    C = ops.zeros((rows, N), np.int16)
    ops.run("lhq_gemm_w4a16_bf16_grouped", A, off, qptr, sptr, zptr, C, E, rows, N, K, G)
    got = D.bf16_bits_to_f32(ops.host(C, np.uint16))
    return got, want, off


def test_w4a16_grouped_small(oracle, ops):
    got, want, off = _grouped(oracle, ops, T=37, E=5, topk=2, K=256, N=64, G=128, seed=1)
    assert off[-1] == 74
    assert rel_frobenius(got, want) <= TOL_BF16


@pytest.mark.parametrize("T,E,topk,K,N", [
    (300, 200, 2, 256, 48),    # 200 groups of ~3 rows: the 16-row kernel, 4 steps of 64 groups
    (1750, 70, 2, 256, 64),    # 70 groups of ~50 rows: the tile kernel, 2 steps of 64 groups
])
def test_w4a16_grouped_many_groups(oracle, ops, T, E, topk, K, N):
    """More groups than one wave resolves at once (workgroups find their
    group 64 groups at a time)."""
    got, want, off = _grouped(oracle, ops, T=T, E=E, topk=topk, K=K, N=N, G=128, seed=E)
    assert off[-1] == T * topk
    assert rel_frobenius(got, want) <= TOL_BF16


@pytest.mark.parametrize("T,E,topk,K,N,G", [
    (1, 8, 2, 4096, 256, 128),    # one token over 8 experts (up to 2 rows, G = 128: the integer form)
    (2, 4, 1, 256, 16400, 128),   # two column tiles per workgroup, N % 16 != 0 (2 rows, maybe in one group)
    (1, 8, 2, 14336, 520, 128),   # the MoE down projection's K, N % 16 != 0
    (1, 8, 1, 2048, 4096, 128),   # one row
    (2, 8, 2, 4096, 300, 128),    # 4 rows over 8 groups (the integer form up to groups / 2 rows)
    (3, 8, 2, 1024, 64, 128),     # 6 rows over 8 groups: the bf16 form
    (8, 8, 1, 512, 200, 64),      # G = 64
    (3, 4, 1, 1024, 96, 256),     # G = 256
    (6, 12, 2, 384, 48, 32),      # G = 32, 3 K tiles
    (2, 16, 2, 512, 200, 64),     # G = 64
    (3, 16, 2, 1024, 96, 256),    # G = 256
])
def test_w4a16_grouped_decode(oracle, ops, T, E, topk, K, N, G):
    """At most one row per group on average: the grouped decode kernel, each
    group's rows staged in LDS in blocks of up to 4, or, up to max(2, groups / 2)
    rows in all with G = 128, the integer-MFMA decode with one row per workgroup."""
    got, want, off = _grouped(oracle, ops, T=T, E=E, topk=topk, K=K, N=N, G=G, seed=50 + T)
    assert off[-1] == T * topk <= E
    assert rel_frobenius(got, want) <= TOL_BF16


@pytest.mark.parametrize("T,K,N", [(4, 4096, 300), (2, 14336, 64)])
def test_w4a16_grouped_decode_rows_on_one_group(oracle, ops, T, K, N):
    """All rows on one group, at most groups / 2 rows: the integer-MFMA
    grouped decode streams that group's weights once per row."""
    got, want, off = _grouped(oracle, ops, T=T, E=8, topk=1, K=K, N=N, G=128, seed=70 + T,
                              one_expert=5)
    assert off[5] == 0 and off[6] == T and off[-1] == T
    assert rel_frobenius(got, want) <= TOL_BF16


@pytest.mark.parametrize("N", [
    4000,   # 250 column tiles: eight per workgroup (32 x 16 row blocks >= 384)
    1000,   # 63 column tiles: four per workgroup (16 x 16 >= 256)
])
def test_w4a16_grouped_wide_workgroups(oracle, ops, N):
    """128 rows over 8 groups: the 16-row kernel with several column tiles
    per workgroup, the last workgroup's tiles past Nt clamped and not stored."""
    got, want, off = _grouped(oracle, ops, T=64, E=8, topk=2, K=256, N=N, G=128, seed=21)
    assert off[-1] == 128
    assert rel_frobenius(got, want) <= TOL_BF16


def test_w4a16_dense_four_tiles(oracle, ops):
    """M = 16 whose rows exceed the decode kernel's LDS at N = 32776: the
    16-row kernel with four column tiles per workgroup (513 workgroups)."""
    got, want = _asym_case(oracle, ops, 16, 2304, 32776, 128, 23)
    assert rel_frobenius(got, want) <= TOL_BF16


def test_w4a16_grouped_empty_expert(oracle, ops):
    got, want, off = _grouped(oracle, ops, T=20, E=4, topk=1, K=128, N=48, G=64, seed=3, empty_expert=2)
    assert off[3] == off[2]
    assert rel_frobenius(got, want) <= TOL_BF16


# ---------------------------------------------------------------------------
# Prefill tile kernel (rows > 16, G >= 128, K % 128 == 0): 128 x 128 tiles,
# activations staged in LDS, each weight tile decoded once per 64 rows.
# ---------------------------------------------------------------------------
def _ulp_close(got, want_f32, oracle, frac=0.999):
    want_b = D.bf16_bits_to_f32(D.to_bf16_bits(oracle, want_f32))
    ulp = np.abs(want_b) * 2.0 ** -7 + 1e-30
    return (np.abs(got - want_b) <= ulp).mean() > frac


@pytest.mark.parametrize("M,K,N,G", [
    (48, 256, 48, 128),      # just above the GEMV range
    (64, 1024, 136, 128),    # config 5 M, ragged N (not a multiple of 128)
    (128, 512, 256, 128),    # one full row tile
    (200, 512, 300, 256),    # partial row tile, G spanning two K tiles
    (300, 1024, 512, 128),   # three row tiles
    (129, 768, 130, 384),    # G = 3 K tiles (the __umulhi group index)
    (257, 256, 16, 128),     # a single 16-column tile
    (64, 8192, 256, 128),    # config 5 K
])
def test_w4a16_bf16_prefill_matches_oracle(oracle, ops, M, K, N, G):
    got, want = _asym_case(oracle, ops, M, K, N, G, seed=500 + M + N)
    err = rel_frobenius(got, want)
    assert err <= TOL_BF16, f"rel Frobenius {err:.3e}"
    assert _ulp_close(got, want, oracle)


def test_w4a16_bf16_prefill_batched(oracle, ops):
    import torch
    B, M, K, N, G = 2, 150, 512, 96, 128
    As, Ws, wants = [], [], []
    for b in range(B):
        A = D.to_bf16_bits(oracle, D.normal((M, K), 1.0, 40 + b))
        p, s, z = oracle.q4a_quantize_groupwise(D.normal((K, N), 0.02, 50 + b), G)
        As.append(A)
        Ws.append(ops.prepack_w4_asym(ops.dev(p), ops.dev(s), ops.dev(z), K, N, G))
        wants.append(oracle.gemm_w4a16_asym(A, p, s, z, N, G))
    A_all = ops.dev(np.stack(As))
    q = torch.cat([w.qweight for w in Ws])
    s = torch.cat([w.scales for w in Ws])
    z = torch.cat([w.zeros for w in Ws])
    C = ops.empty((B, M, N), np.int16)
    ops.run("lhq_gemm_w4a16_bf16_batched", A_all, q, s, z, C, B, M, N, K, G)
    got = D.bf16_bits_to_f32(ops.host(C, np.uint16))
    for b in range(B):
        assert rel_frobenius(got[b], wants[b]) <= TOL_BF16
        assert _ulp_close(got[b], wants[b], oracle)


def test_w4a16_grouped_prefill_config4_routing(oracle, ops):
    """Config 4's routing (512 tokens, top-2 of 8 experts, sum M_g = 1024) at full K, reduced N."""
    got, want, off = _grouped(oracle, ops, T=512, E=8, topk=2, K=4096, N=256, G=128, seed=11)
    assert off[-1] == 1024
    assert rel_frobenius(got, want) <= TOL_BF16
    assert _ulp_close(got, want, oracle)


def test_w4a16_grouped_prefill_empty_expert(oracle, ops):
    got, want, off = _grouped(oracle, ops, T=200, E=4, topk=1, K=384, N=80, G=128, seed=5, empty_expert=1)
    assert off[2] == off[1]
    assert rel_frobenius(got, want) <= TOL_BF16
    assert _ulp_close(got, want, oracle)


# Non-finite activations on the C ABI.  The kernels sum x * (q - z) through
# exact group sums that subtract an activation sum (t - (128 + z) * xs, or a
# chain seeded with -144 * sum x, or a block exponent that becomes NaN), so
# a row holding +Inf, -Inf or NaN comes out NaN in every column; every other
# row is unaffected.  (The reference's term-by-term sum, gemm_quant.cpp:78,
# gives +-Inf there, NaN only where a weight is zero; the lh:: drop-in routes
# non-finite host activations to the dequantize + fp32 GEMM path for that.)
NONFINITE_BF16 = [(1, 4096, 2048), (4, 4096, 1024), (16, 4096, 1024), (64, 1024, 512), (256, 1024, 512)]


def _nonfinite_rows(M):
    """(row, value) pairs to plant: one row each of +Inf, -Inf, NaN, and +Inf
    with -Inf together, as many as the rows allow (M = 1: +Inf)."""
    vals = [np.inf, -np.inf, np.nan, "both"]
    return [(r * max(1, M // 4), v) for r, v in enumerate(vals[:max(1, min(4, M))])]


def _check_nonfinite(got, want, bad, tol):
    good = np.setdiff1d(np.arange(got.shape[0]), bad)
    for r in bad:
        assert np.isnan(got[r]).all(), f"row {r}: {np.isfinite(got[r]).sum()} finite outputs"
    if len(good):
        assert np.isfinite(got[good]).all()
        assert rel_frobenius(got[good], want[good]) <= tol


@pytest.mark.parametrize("M,K,N", NONFINITE_BF16)
def test_w4a16_bf16_nonfinite_rows_are_nan(oracle, ops, M, K, N):
    """M=1: the integer decode kernel; 4: the bf16 decode kernel; 16: the
    16-row kernel; 64 / 256: the prefill tile kernel."""
    G = 128
    x = D.normal((M, K), 1.0, 4000 + M)
    bad = []
    for r, v in _nonfinite_rows(M):
        if v == "both":
            x[r, 5], x[r, K - 9] = np.inf, -np.inf
        else:
            x[r, (37 * r + 11) % K] = v
        bad.append(r)
    A = D.to_bf16_bits(oracle, x)
    W = D.normal((K, N), 0.02, 4001)
    p, s, z = oracle.q4a_quantize_groupwise(W, G)
    w = ops.prepack_w4_asym(ops.dev(p), ops.dev(s), ops.dev(z), K, N, G)
    got = D.bf16_bits_to_f32(ops.host(ops.gemm_w4a16_bf16(ops.dev(A), w), np.uint16))
    good = np.setdiff1d(np.arange(M), bad)
    want = np.zeros((M, N), np.float32)
    if len(good):
        want[good] = oracle.gemm_w4a16_asym(np.ascontiguousarray(A[good]), p, s, z, N, G)
    _check_nonfinite(got, want, bad, TOL_BF16)


@pytest.mark.parametrize("T,E,topk,K,N,bad", [
    (2, 8, 2, 4096, 300, (1,)),        # 4 rows: the grouped integer decode
    (3, 8, 2, 1024, 64, (0, 2)),       # 6 rows: the bf16 grouped decode
    (64, 8, 2, 256, 1000, (3, 40, 63)),  # the 16-row kernel
    (300, 4, 1, 256, 256, (0, 150, 299)),  # the tile kernel (~75 rows per group)
])
def test_w4a16_grouped_nonfinite_rows_are_nan(oracle, ops, T, E, topk, K, N, bad):
    """The grouped launches: every dispatched row of a token holding +Inf,
    -Inf or NaN is NaN in every column, the other rows as without them."""
    seed = 90 + T
    got, want, off = _grouped(oracle, ops, T=T, E=E, topk=topk, K=K, N=N, G=128, seed=seed,
                              bad_tokens=bad)
    _, tok, _ = oracle.moe_dispatch_table(D.moe_routing(T, E, topk, seed), E)
    rows = np.flatnonzero(np.isin(tok, bad))
    assert len(rows) == len(bad) * topk
    _check_nonfinite(got, want, rows, TOL_BF16)


@pytest.mark.parametrize("M,K,N", [(1, 4096, 2048), (16, 4096, 1024), (64, 1024, 512)])
def test_w4a16_f32_nonfinite_rows_are_nan(oracle, ops, M, K, N):
    """The fp32 interface: integer decode (M=1), 16-row kernel (16), tile
    kernel with the hi + lo activation split (64)."""
    G = 128
    A = D.uniform((M, K), -1, 1, 4100 + M)
    bad = []
    for r, v in _nonfinite_rows(M):
        if v == "both":
            A[r, 5], A[r, K - 9] = np.inf, -np.inf
        else:
            A[r, (37 * r + 11) % K] = v
        bad.append(r)
    W = D.uniform((K, N), -1, 1, 4101)
    Bp, Bs = oracle.q4_quantize_groupwise(W, G)
    w = ops.prepack_w4_sym(ops.dev(Bp), ops.dev(Bs), K, N, G)
    C = ops.dev(np.zeros((M, N), np.float32))
    ops.gemm_w4a16(ops.dev(A), w, C, 1.0, 0.0)
    got = ops.host(C)
    good = np.setdiff1d(np.arange(M), bad)
    want = np.zeros((M, N), np.float32)
    if len(good):
        want[good] = oracle.gemm_w4a16_groupwise(np.ascontiguousarray(A[good]), Bp, Bs, N, G)
    _check_nonfinite(got, want, bad, TOL_F32)
