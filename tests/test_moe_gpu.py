"""MoE routing and the quantized expert MLP on the GPU vs the CPU oracle
(moe.cpp:102-221; the oracle's MoE functions are pinned against the
reference's own moe.cpp in tests/test_moe_oracle.py).

Bars: dispatch (offsets, token_idx, slot_idx, slot_pos, copied rows) and
combine (fp32 and bf16) bit-exact; the SwiGLU projection and the expert MLP
(bf16 outputs) within relative Frobenius 1e-2, plus a per-element check of
one bf16 unit in the last place for nearly all entries.
"""
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
    ulp = np.abs(want_b) * 2.0 ** -7 + 1e-30
    return (np.abs(got - want_b) <= ulp).mean() > frac


def _routing(T, E, K, seed, kind="uniform"):
    if kind == "repeat":    # ids drawn with replacement: a token may name one expert twice
        return D.rng(seed).integers(0, E, (T, K)).astype(np.int32)
    if kind == "dropped":   # some ids outside [0, E)
        ids = D.rng(seed).integers(-2, E + 2, (T, K)).astype(np.int32)
        return ids
    if kind == "skewed":    # most tokens on expert 0, several experts empty
        ids = D.moe_routing(T, E, K, seed)
        ids[: (3 * T) // 4, 0] = 0
        ids[: (3 * T) // 4, 1:] = np.where(ids[: (3 * T) // 4, 1:] == 0, 1, ids[: (3 * T) // 4, 1:])
        return ids
    return D.moe_routing(T, E, K, seed)


# ---------------------------------------------------------------------------
# dispatch
# ---------------------------------------------------------------------------

DISPATCH_CASES = [
    # T, E, K, H, routing
    (6, 3, 2, 4, "ref"),          # test_moe.cpp:131-170's hand-built table
    (512, 8, 2, 4096, "uniform"),  # benchmark config 4
    (1000, 64, 6, 72, "uniform"),
    (3, 512, 2, 8, "uniform"),     # the most experts the ranking kernel takes
    (37, 16, 4, 5, "uniform"),     # odd H: 2- and 4-byte row copies
    (20000, 8, 2, 16, "uniform"),  # 40000 slots: 40 chunks per wave
    (300, 16, 4, 64, "repeat"),
    (300, 16, 3, 64, "dropped"),
    (257, 32, 2, 40, "skewed"),
    (0, 4, 2, 8, "uniform"),
    # up to 256 slots: the one-launch form
    (1, 8, 2, 4096, "uniform"),   # one decode token
    (2, 8, 2, 4096, "skewed"),
    (40, 16, 3, 64, "dropped"),
    (64, 8, 4, 32, "repeat"),     # exactly 256 slots
    (128, 512, 2, 6, "uniform"),  # 256 slots over the most experts
    (86, 3, 3, 40, "repeat"),     # 258 slots: the two launches
    (2, 100, 70, 8, "repeat"),    # top-70 (past the combine's 64): the two launches
]


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("T,E,K,H,kind", DISPATCH_CASES)
def test_dispatch_bitexact(oracle, ops, T, E, K, H, kind, dtype):
    if kind == "ref":
        ids = np.array([[0, 1], [2, 0], [1, 2], [0, 1], [2, 1], [0, 2]], np.int32)
    else:
        ids = _routing(T, E, K, 1000 + T + E, kind)
    if dtype == "f32":
        hidden = D.normal((T, H), 1.0, 7)
        elem = np.float32
    else:
        hidden = D.rng(7).integers(0, 65536, (T, H), dtype=np.uint16)
        elem = np.uint16
    off, tok, slot, pos, out = oracle.moe_dispatch(hidden, ids.reshape(T, K), E)
    S = T * K
    g_off = ops.zeros((E + 1,), np.int32)
    g_tok, g_slot, g_pos = (ops.zeros((max(S, 1),), np.int32) for _ in range(3))
    g_out = ops.zeros((max(S, 1), H), elem)
    name = "lhq_moe_dispatch_f32" if dtype == "f32" else "lhq_moe_dispatch_bf16"
    ops.run(name, hidden if T else None, ids if T else None, g_off, g_tok, g_slot, g_pos, g_out, T, H, E, K)
    assert np.array_equal(ops.host(g_off), off)
    n = int(off[-1])
    assert np.array_equal(ops.host(g_tok)[:S], tok)
    assert np.array_equal(ops.host(g_slot)[:S], slot)
    assert np.array_equal(ops.host(g_pos)[:S], pos)
    got = ops.host(g_out, elem)[:n]
    assert np.array_equal(got.view(np.uint16 if dtype == "bf16" else np.uint32),
                          out[:n].view(np.uint16 if dtype == "bf16" else np.uint32))


def test_slot_positions_from_reference_layout(oracle, ops):
    T, E, K = 700, 16, 4
    ids = _routing(T, E, K, 77, "dropped")
    _, tok, slot, pos, _ = oracle.moe_dispatch(np.zeros((T, 1), np.float32), ids, E)
    g_pos = ops.zeros((T * K,), np.int32)
    ops.run("lhq_moe_slot_positions", tok, slot, g_pos, T, K)
    assert np.array_equal(ops.host(g_pos), pos)


def test_dispatch_rejects_bad_dims(ops, lib):
    from longhornai_amd.capi import LHQ_ERR_INVALID, LHQ_ERR_UNSUPPORTED
    d = ops.zeros((64,), np.int32)
    P = d.data_ptr()
    assert lib.status("lhq_moe_dispatch_f32", P, P, P, P, P, P, P, 4, 8, 513, 2, ops.stream()) == LHQ_ERR_UNSUPPORTED
    assert lib.status("lhq_moe_dispatch_f32", P, P, P, P, P, P, P, 4, 8, 0, 2, ops.stream()) == LHQ_ERR_INVALID
    assert lib.status("lhq_moe_combine_f32", P, P, P, P, 4, 8, 65, ops.stream()) == LHQ_ERR_UNSUPPORTED


# ---------------------------------------------------------------------------
# combine
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("T,E,K,H,kind", [
    (6, 3, 2, 4, "uniform"),
    (512, 8, 2, 4096, "uniform"),
    (100, 64, 8, 1000, "uniform"),
    (41, 16, 4, 7, "uniform"),      # H % 4 != 0: scalar tail
    (300, 16, 3, 64, "dropped"),
    (300, 16, 4, 2052, "repeat"),
    (1, 2, 2, 5000, "uniform"),      # several column blocks
])
def test_combine_bitexact(oracle, ops, T, E, K, H, kind, dtype):
    ids = _routing(T, E, K, 2000 + T, kind)
    _, tok, slot, pos, _ = oracle.moe_dispatch(np.zeros((T, 1), np.float32), ids, E)
    gates = D.uniform((T, K), 0.0, 1.0, 2001)
    if dtype == "f32":
        y = D.normal((T * K, H), 1.0, 2002)
        want = oracle.moe_combine_f32(y, tok, slot, gates)
        out = ops.zeros((T, H), np.float32)
        ops.run("lhq_moe_combine_f32", y, pos, gates, out, T, H, K)
        assert np.array_equal(ops.host(out).view(np.uint32), want.view(np.uint32))
    else:
        y = D.to_bf16_bits(oracle, D.normal((T * K, H), 1.0, 2002))
        want = oracle.moe_combine_bf16(y, tok, slot, gates)
        out = ops.zeros((T, H), np.uint16)
        ops.run("lhq_moe_combine_bf16", y, pos, gates, out, T, H, K)
        assert np.array_equal(ops.host(out, np.uint16), want)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("T,E,K,H,kind", [
    (512, 8, 2, 4096, "uniform"),   # config 4
    (41, 16, 4, 7, "uniform"),      # H % 4 != 0
    (300, 16, 3, 16384, "dropped"),  # the longest row the fused kernel holds
    (64, 8, 2, 1000, "repeat"),
])
def test_combine_q8_bitexact(oracle, ops, T, E, K, H, kind, dtype):
    """combine + per-token int8 quantization in one kernel == q8_quantize_per_row
    (quant.cpp:52-63) of the fp32 combine; token 0 sums to an all-zero row
    (scale 1) and one expert output holds a NaN (it never wins the max and
    quantizes to 0)."""
    ids = _routing(T, E, K, 6000 + T, kind)
    _, tok, slot, pos, _ = oracle.moe_dispatch(np.zeros((T, 1), np.float32), ids, E)
    gates = D.uniform((T, K), 0.0, 1.0, 6001)
    gates[0] = 0.0
    y = D.normal((T * K, H), 1.0, 6002)
    y[T * K // 2, H // 2] = np.nan
    if dtype == "bf16":
        y = D.to_bf16_bits(oracle, y)
        yf = D.bf16_bits_to_f32(y)
        name = "lhq_moe_combine_q8_bf16"
    else:
        yf = y
        name = "lhq_moe_combine_q8_f32"
    wq, ws = oracle.q8_quantize_per_row(oracle.moe_combine_f32(yf, tok, slot, gates))
    q = ops.zeros((T, H), np.int8)
    sc = ops.zeros((T,), np.float32)
    ops.run(name, y, pos, gates, q, sc, T, H, K)
    assert np.array_equal(ops.host(q), wq)
    assert np.array_equal(ops.host(sc).view(np.uint32), ws.view(np.uint32))
    assert ws[0] == 1.0 and not wq[0].any()


def test_combine_order_is_slot_order(oracle, ops):
    """2^24 + (-2^24) + 1 in expert-major slot order is 1 (top-k order would give 0)."""
    ids = np.array([[2, 0, 1]], np.int32)
    _, tok, slot, pos, _ = oracle.moe_dispatch(np.zeros((1, 1), np.float32), ids, 3)
    y = np.zeros((3, 4), np.float32)
    y[pos[0]] = 1.0
    y[pos[1]] = 2.0 ** 24
    y[pos[2]] = -(2.0 ** 24)
    out = ops.zeros((1, 4), np.float32)
    ops.run("lhq_moe_combine_f32", y, pos, np.ones((1, 3), np.float32), out, 1, 4, 3)
    assert (ops.host(out) == 1.0).all()


# ---------------------------------------------------------------------------
# gate / up interleave, SwiGLU projection, expert MLP
# ---------------------------------------------------------------------------

def _experts(oracle, E, K, N, G, seed):
    qs = [oracle.q4a_quantize_groupwise(D.normal((K, N), 0.02, seed + e), G) for e in range(E)]
    return tuple(np.stack(a) for a in zip(*qs))


def _prepack(ops, stack, K, N, G):
    P_, S_, Z_ = stack
    return [ops.prepack_w4_asym(ops.dev(P_[e]), ops.dev(S_[e]), ops.dev(Z_[e]), K, N, G) for e in range(len(P_))]


def test_interleave_gate_up_layout(oracle, ops):
    K, I, G = 384, 40, 128
    g = _prepack(ops, _experts(oracle, 1, K, I, G, 1), K, I, G)[0]
    u = _prepack(ops, _experts(oracle, 1, K, I, G, 2), K, I, G)[0]
    w = ops.interleave_gate_up(g, u)
    for a, b, c in ((g.qweight, u.qweight, w.qweight), (g.scales, u.scales, w.scales), (g.zeros, u.zeros, w.zeros)):
        Nt = -(-I // 16)
        a, b, c = (ops.host(x).view(np.uint8).reshape(Nt * (2 if x is c else 1), -1) for x in (a, b, c))
        assert np.array_equal(c[0::2], a) and np.array_equal(c[1::2], b)


def _swiglu_case(oracle, ops, T, E, K, H, I, G, seed, kind="uniform"):
    ids = _routing(T, E, K, seed, kind)
    x = D.to_bf16_bits(oracle, D.normal((T, H), 1.0, seed + 1))
    off, tok, _, _, X = oracle.moe_dispatch(x, ids, E)
    gate = _experts(oracle, E, H, I, G, seed + 100)
    up = _experts(oracle, E, H, I, G, seed + 200)
    g = oracle.gemm_w4a16_asym_grouped(X, off, *gate, I, G)
    u = oracle.gemm_w4a16_asym_grouped(X, off, *up, I, G)
    want = D.bf16_bits_to_f32(oracle.swiglu_bf16(g, u))
    gu = [ops.interleave_gate_up(a, b) for a, b in zip(_prepack(ops, gate, H, I, G), _prepack(ops, up, H, I, G))]
    q, s, z = ops.pointer_tables(gu)
    rows = X.shape[0]
    act = ops.zeros((rows, I), np.int16)
    ops.run("lhq_gemm_w4a16_bf16_grouped_swiglu", X, off, q, s, z, act, E, rows, I, H, G)
    n = int(off[-1])
    return D.bf16_bits_to_f32(ops.host(act, np.uint16))[:n], want[:n]


@pytest.mark.parametrize("T,E,K,H,I,G,kind", [
    (37, 5, 2, 256, 64, 128, "uniform"),    # ~15 rows per expert: 16-row kernel
    (20, 4, 1, 128, 72, 64, "skewed"),      # I % 16 != 0, G = 64, empty experts
    (200, 4, 2, 512, 256, 128, "uniform"),  # ~100 rows per expert: 128x128 tile kernel
    (300, 8, 2, 384, 200, 128, "skewed"),   # tile kernel, I % 128 != 0, empty experts
    (512, 8, 2, 1024, 512, 128, "uniform"),  # config 4's routing
    # at most one row per expert on average: the grouped decode kernel
    (1, 8, 2, 4096, 256, 128, "uniform"),   # one token, two experts (the integer-MFMA form)
    (1, 8, 2, 2048, 1000, 128, "uniform"),  # ... I % 16 != 0
    (2, 8, 2, 2048, 300, 128, "skewed"),    # 4 rows, two on expert 0 (integer form)
    (2, 8, 2, 1024, 72, 128, "dropped"),    # integer form, row capacity past offsets[E]
    (5, 8, 1, 512, 72, 64, "uniform"),      # G = 64, I % 16 != 0
    (10, 16, 1, 384, 48, 32, "skewed"),     # 7 rows of one expert: two row blocks; G = 32
    (6, 12, 2, 1024, 40, 256, "dropped"),   # G = 256, ids outside [0, E) dropped
    (4, 16, 2, 512, 72, 128, "skewed"),     # a block of 3 rows
    (8, 16, 1, 256, 48, 64, "skewed"),      # 6 rows of one expert: blocks of 4 and 2; G = 64
    # 16-row kernel with several gate / up pairs per workgroup
    (64, 8, 2, 256, 2024, 128, "uniform"),  # 2 x 127 tiles, four pairs: the last workgroup's 4th lies past the end
    (64, 8, 2, 256, 1000, 128, "uniform"),  # 2 x 63 tiles, two pairs: the last workgroup's 2nd lies past the end
])
def test_grouped_swiglu(oracle, ops, T, E, K, H, I, G, kind):
    got, want = _swiglu_case(oracle, ops, T, E, K, H, I, G, 3000 + T, kind)
    assert rel_frobenius(got, want) <= TOL_BF16
    assert _ulp_close(got, want, oracle, frac=0.99)


@pytest.mark.parametrize("T,E,K,H,I,G", [
    (40, 4, 2, 256, 384, 128),     # 16-row kernels
    (512, 8, 2, 512, 1024, 128),   # config 4's routing on the tile kernels
    (2, 8, 2, 1024, 384, 128),     # 4 rows over 8 experts: the grouped decode kernels
])
def test_expert_mlp(oracle, ops, T, E, K, H, I, G):
    ids = _routing(T, E, K, 4000 + T)
    x = D.to_bf16_bits(oracle, D.normal((T, H), 1.0, 4001))
    off, tok, _, _, X = oracle.moe_dispatch(x, ids, E)
    gate = _experts(oracle, E, H, I, G, 4100)
    up = _experts(oracle, E, H, I, G, 4200)
    down = _experts(oracle, E, I, H, G, 4300)
    want_act, want_y = oracle.moe_expert_mlp_w4a16(X, off, gate, up, down, H, I, G)
    gu = [ops.interleave_gate_up(a, b) for a, b in zip(_prepack(ops, gate, H, I, G), _prepack(ops, up, H, I, G))]
    dw = _prepack(ops, down, I, H, G)
    rows = X.shape[0]
    act = ops.zeros((rows, I), np.int16)
    y = ops.zeros((rows, H), np.int16)
    ops.run("lhq_moe_expert_mlp_w4a16_bf16", X, off, *ops.pointer_tables(gu), *ops.pointer_tables(dw), act, y,
            E, rows, H, I, G)
    n = int(off[-1])
    got_y = D.bf16_bits_to_f32(ops.host(y, np.uint16))[:n]
    assert rel_frobenius(D.bf16_bits_to_f32(ops.host(act, np.uint16))[:n], D.bf16_bits_to_f32(want_act)[:n]) <= TOL_BF16
    assert rel_frobenius(got_y, D.bf16_bits_to_f32(want_y)[:n]) <= TOL_BF16


def test_moe_layer_end_to_end(oracle, ops):
    """dispatch -> expert MLP -> combine with the group table staying on the
    device, vs the oracle's chain."""
    T, E, K, H, I, G = 256, 8, 2, 512, 768, 128
    ids = _routing(T, E, K, 5000)
    gates = D.uniform((T, K), 0.0, 1.0, 5001)
    gates /= gates.sum(1, keepdims=True)
    x = D.to_bf16_bits(oracle, D.normal((T, H), 1.0, 5002))
    gate = _experts(oracle, E, H, I, G, 5100)
    up = _experts(oracle, E, H, I, G, 5200)
    down = _experts(oracle, E, I, H, G, 5300)
    off, tok, slot, _, X = oracle.moe_dispatch(x, ids, E)
    _, y = oracle.moe_expert_mlp_w4a16(X, off, gate, up, down, H, I, G)
    want = D.bf16_bits_to_f32(oracle.moe_combine_bf16(y, tok, slot, gates))

    gu = [ops.interleave_gate_up(a, b) for a, b in zip(_prepack(ops, gate, H, I, G), _prepack(ops, up, H, I, G))]
    dw = _prepack(ops, down, I, H, G)
    S = T * K
    g_off = ops.zeros((E + 1,), np.int32)
    g_tok, g_slot, g_pos = (ops.zeros((S,), np.int32) for _ in range(3))
    g_x = ops.zeros((S, H), np.int16)
    act = ops.zeros((S, I), np.int16)
    g_y = ops.zeros((S, H), np.int16)
    out = ops.zeros((T, H), np.int16)
    ops.run("lhq_moe_dispatch_bf16", x, ids, g_off, g_tok, g_slot, g_pos, g_x, T, H, E, K)
    ops.run("lhq_moe_expert_mlp_w4a16_bf16", g_x, g_off, *ops.pointer_tables(gu), *ops.pointer_tables(dw), act, g_y,
            E, S, H, I, G)
    ops.run("lhq_moe_combine_bf16", g_y, g_pos, gates, out, T, H, K)
    got = D.bf16_bits_to_f32(ops.host(out, np.uint16))
    assert rel_frobenius(got, want) <= TOL_BF16
