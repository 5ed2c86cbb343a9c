"""Pins of the oracle's MoE functions (oracle/lhq_oracle.c: lho_moe_dispatch,
lho_swiglu_bf16, lho_moe_combine_f32/_bf16) -- CPU only.

- the reference's own known answer for dispatch (test_moe.cpp:131-170);
- the reference library (oracle/_ref/libref.so builds moe.cpp) bit for bit:
  dispatch and combine, and the expert MLP within the bf16 bar;
- independent formulations: a stable sort for the dispatch layout, a
  per-token sum in slot order for combine (with values whose sum depends on
  the order), float64 SwiGLU and special values.
"""
import numpy as np
import pytest

from oracle import Oracle, Ref, ref_available, rel_frobenius
from tests import _data as D

need_ref = pytest.mark.skipif(not ref_available(), reason="oracle/_ref not built (reference tree absent)")


@pytest.fixture(scope="module")
def o():
    return Oracle()


def bits(a):
    return np.asarray(a).view(np.uint32)


# ---------------------------------------------------------------------------
# dispatch
# ---------------------------------------------------------------------------

def test_dispatch_reference_known_answer(o):
    """test_moe.cpp:131-170: hand-built routing, T=6, E=3, top-2."""
    ids = np.array([[0, 1], [2, 0], [1, 2], [0, 1], [2, 1], [0, 2]], np.int32)
    hidden = D.normal((6, 4), 1.0, 6100)
    off, tok, slot, pos, out = o.moe_dispatch(hidden, ids, 3)
    assert off[-1] == 12
    assert list(np.diff(off)) == [int((ids == e).sum()) for e in range(3)] == [4, 4, 4]
    assert np.array_equal(out, hidden[tok])


def sort_dispatch(ids, E):
    """The layout as a stable sort of (expert, token, slot) keys."""
    T, K = ids.shape
    keys = sorted((int(ids[t, k]), t, k) for t in range(T) for k in range(K) if 0 <= ids[t, k] < E)
    off = np.zeros(E + 1, np.int32)
    for e, _, _ in keys:
        off[e + 1] += 1
    off = np.cumsum(off).astype(np.int32)
    tok = np.full(T * K, -1, np.int32)
    slot = np.full(T * K, -1, np.int32)
    pos = np.full(T * K, -1, np.int32)
    for p, (e, t, k) in enumerate(keys):
        tok[p], slot[p], pos[t * K + k] = t, k, p
    return off, tok, slot, pos


@pytest.mark.parametrize("T,E,K,seed", [(1, 1, 1, 1), (7, 3, 2, 2), (64, 8, 2, 3), (33, 16, 4, 4), (5, 40, 3, 5)])
def test_dispatch_equals_stable_sort(o, T, E, K, seed):
    ids = D.moe_routing(T, E, K, seed)
    hidden = D.rng(seed).integers(0, 65536, (T, 24), dtype=np.uint16)  # bf16 rows: a copy is a copy
    off, tok, slot, pos, out = o.moe_dispatch(hidden, ids, E)
    want = sort_dispatch(ids, E)
    for got, w in zip((off, tok, slot, pos), want):
        assert np.array_equal(got, w)
    assert np.array_equal(out, hidden[tok])


def test_dispatch_repeated_expert_and_dropped_ids(o):
    """A token may name one expert twice (slot order breaks the tie); ids
    outside [0, E) are dropped and leave -1 past offsets[E]."""
    ids = np.array([[1, 1], [0, 5], [-1, 1], [2, 0]], np.int32)
    off, tok, slot, pos, _ = o.moe_dispatch(np.zeros((4, 2), np.float32), ids, 3)
    want = sort_dispatch(ids, 3)
    for got, w in zip((off, tok, slot, pos), want):
        assert np.array_equal(got, w)
    assert off[-1] == 6 and (tok[6:] == -1).all() and pos[3] == -1 and pos[4] == -1


@need_ref
@pytest.mark.parametrize("T,E,K,H,seed", [(6, 3, 2, 4, 10), (100, 8, 2, 64, 11), (37, 16, 4, 5, 12), (3, 8, 1, 9, 13)])
def test_dispatch_bitexact_vs_reference(o, T, E, K, H, seed):
    ids = D.moe_routing(T, E, K, seed)
    hidden = D.normal((T, H), 1.0, seed)
    off, tok, slot, _, out = o.moe_dispatch(hidden, ids, E)
    roff, rtok, rslot, rout = Ref().moe_dispatch(hidden, ids, E)
    assert np.array_equal(off, roff) and np.array_equal(tok, rtok) and np.array_equal(slot, rslot)
    assert np.array_equal(bits(out), bits(rout))


# ---------------------------------------------------------------------------
# combine
# ---------------------------------------------------------------------------

def test_combine_order_is_slot_order(o):
    """fp32 sums of 2^24, 1, -2^24 depend on the order.  moe.cpp:213-220 adds
    in dispatched-slot order (expert-major), not in top-k order: token 0
    routes k=0 -> expert 2, k=1 -> expert 0, k=2 -> expert 1."""
    ids = np.array([[2, 0, 1]], np.int32)
    off, tok, slot, pos, _ = o.moe_dispatch(np.zeros((1, 1), np.float32), ids, 3)
    y = np.zeros((3, 1), np.float32)
    y[pos[0], 0] = 1.0          # k=0 (expert 2): added last
    y[pos[1], 0] = 2.0 ** 24    # k=1 (expert 0): added first
    y[pos[2], 0] = -(2.0 ** 24)  # k=2 (expert 1): added second
    gates = np.ones((1, 3), np.float32)
    # slot order: 2^24, then -2^24 -> 0, then +1 -> 1.  Top-k order would give
    # 1 + 2^24 = 2^24 (rounded), then -2^24 -> 0.
    assert o.moe_combine_f32(y, tok, slot, gates)[0, 0] == 1.0


@pytest.mark.parametrize("T,E,K,H,seed", [(9, 4, 2, 8, 20), (50, 8, 3, 33, 21)])
def test_combine_per_token_formulation(o, T, E, K, H, seed):
    """The same sum written per token over its slots in position order."""
    ids = D.moe_routing(T, E, K, seed)
    off, tok, slot, pos, _ = o.moe_dispatch(np.zeros((T, 1), np.float32), ids, E)
    y = D.normal((T * K, H), 1.0, seed + 1)
    gates = D.uniform((T, K), 0.0, 1.0, seed + 2)
    got = o.moe_combine_f32(y, tok, slot, gates)
    for t in range(T):
        acc = np.zeros(H, np.float32)
        for k in sorted(range(K), key=lambda k: pos[t * K + k]):
            acc = acc + np.float32(gates[t, k]) * y[pos[t * K + k]]
        assert np.array_equal(bits(got[t]), bits(acc))


@need_ref
@pytest.mark.parametrize("T,E,K,H,seed", [(6, 3, 2, 4, 30), (128, 8, 2, 96, 31), (41, 16, 4, 7, 32)])
def test_combine_bitexact_vs_reference(o, T, E, K, H, seed):
    ids = D.moe_routing(T, E, K, seed)
    off, tok, slot, _, _ = o.moe_dispatch(np.zeros((T, 1), np.float32), ids, E)
    y = D.normal((T * K, H), 1.0, seed + 1)
    gates = D.uniform((T, K), 0.0, 1.0, seed + 2)
    assert np.array_equal(bits(o.moe_combine_f32(y, tok, slot, gates)),
                          bits(Ref().moe_combine(y, off, tok, slot, gates)))


def test_combine_bf16_is_f32_combine_rounded(o):
    T, E, K, H = 40, 8, 2, 20
    ids = D.moe_routing(T, E, K, 40)
    _, tok, slot, _, _ = o.moe_dispatch(np.zeros((T, 1), np.float32), ids, E)
    yb = D.to_bf16_bits(o, D.normal((T * K, H), 1.0, 41))
    gates = D.uniform((T, K), 0.0, 1.0, 42)
    want = o.f32_to_bf16_n(o.moe_combine_f32(D.bf16_bits_to_f32(yb), tok, slot, gates))
    assert np.array_equal(o.moe_combine_bf16(yb, tok, slot, gates), want)


# ---------------------------------------------------------------------------
# SwiGLU and the quantized expert MLP
# ---------------------------------------------------------------------------

def test_swiglu_special_values(o):
    g = np.array([0.0, -0.0, 100.0, -100.0, -1000.0, np.inf, -np.inf, np.nan], np.float32)
    u = np.full(g.shape, 3.0, np.float32)
    a = D.bf16_bits_to_f32(o.swiglu_bf16(g, u))
    assert a[0] == 0.0 and a[1] == 0.0
    assert a[2] == 300.0                     # silu(v) = v for large v
    assert a[3] == 0.0 and a[4] == 0.0       # v / inf -> -0
    assert np.signbit(a[4])
    assert a[5] == np.inf                    # inf / (1 + 0)
    assert np.isnan(a[6]) and np.isnan(a[7])  # -inf / (1 + inf) and NaN


def test_swiglu_vs_float64(o):
    g = D.normal((4096,), 3.0, 50)
    u = D.normal((4096,), 1.0, 51)
    got = D.bf16_bits_to_f32(o.swiglu_bf16(g, u)).astype(np.float64)
    g64, u64 = g.astype(np.float64), u.astype(np.float64)
    want = g64 / (1.0 + np.exp(-g64)) * u64
    # bf16 keeps 8 significant bits: within one unit in the last place
    assert (np.abs(got - want) <= np.abs(want) * 2.0 ** -7 + 1e-30).all()


def _experts(o, E, K, N, G, seed):
    Ps, Ss, Zs, Ws = [], [], [], []
    for e in range(E):
        p, s, z = o.q4a_quantize_groupwise(D.normal((K, N), 0.02, seed + e), G)
        Ps.append(p); Ss.append(s); Zs.append(z); Ws.append(o.q4a_dequantize_groupwise(p, s, z, K, N, G))
    return (np.stack(Ps), np.stack(Ss), np.stack(Zs)), np.stack(Ws)


@need_ref
def test_expert_mlp_vs_reference(o):
    """The quantized expert MLP against the reference's fp32 moe_expert_mlp
    fed the same (dequantized) weights and the same (bf16) inputs; the only
    difference is the bf16 rounding of the activation and of the output."""
    T, E, K, H, I, G = 48, 4, 2, 256, 384, 128
    ids = D.moe_routing(T, E, K, 60)
    x = D.to_bf16_bits(o, D.normal((T, H), 1.0, 61))
    off, tok, _, _, X = o.moe_dispatch(x, ids, E)
    gate, Wg = _experts(o, E, H, I, G, 100)
    up, Wu = _experts(o, E, H, I, G, 200)
    down, Wd = _experts(o, E, I, H, G, 300)
    act, y = o.moe_expert_mlp_w4a16(X, off, gate, up, down, H, I, G)
    want = Ref().moe_expert_mlp(D.bf16_bits_to_f32(X), off, Wg, Wu, Wd)
    assert rel_frobenius(D.bf16_bits_to_f32(y), want) <= 1e-2


def test_expert_mlp_vs_float64(o):
    T, E, K, H, I, G = 20, 3, 2, 128, 256, 64
    ids = D.moe_routing(T, E, K, 70)
    x = D.to_bf16_bits(o, D.normal((T, H), 1.0, 71))
    off, tok, _, _, X = o.moe_dispatch(x, ids, E)
    gate, Wg = _experts(o, E, H, I, G, 400)
    up, Wu = _experts(o, E, H, I, G, 500)
    down, Wd = _experts(o, E, I, H, G, 600)
    _, y = o.moe_expert_mlp_w4a16(X, off, gate, up, down, H, I, G)
    Xf = D.bf16_bits_to_f32(X).astype(np.float64)
    want = np.zeros((T * K, H))
    for e in range(E):
        r = slice(off[e], off[e + 1])
        gp, upj = Xf[r] @ Wg[e], Xf[r] @ Wu[e]
        want[r] = (gp / (1.0 + np.exp(-gp)) * upj) @ Wd[e]
    assert rel_frobenius(D.bf16_bits_to_f32(y), want) <= 1e-2
