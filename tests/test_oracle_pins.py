"""Pins of the CPU oracle (oracle/lhq_oracle.c) -- CPU only.

Three independent kinds of check, so that a plausible slip in the
restatement (a dropped term, a swapped reciprocal/division, a wrong nibble
order, a misplaced rounding) fails at least one:

1. Golden vectors written by the reference's own compiled code
   (tests/golden/ref_vectors.npz, see make_golden.py): bit-exact.
2. The reference library itself (oracle/_ref/libref.so) where it was built:
   bit-exact on many fresh random inputs and on exhaustive conversion tables.
3. Closed forms and independent textbook routines: numpy's IEEE binary16,
   torch's bfloat16 and float8_e4m3fn casts, int64 matrix products,
   float64 matmuls, hand-derived known answers, exhaustive q4_get.
"""
import os

import numpy as np
import pytest

from oracle import ORACLE_SO, Oracle, Ref, ref_available, rel_frobenius
from tests import _data as D

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "ref_vectors.npz")


@pytest.fixture(scope="module")
def o():
    return Oracle(ORACLE_SO)


@pytest.fixture(scope="module")
def g():
    return np.load(GOLDEN, allow_pickle=False)


def bits(a):
    a = np.asarray(a)
    return a.view(np.uint32) if a.dtype == np.float32 else a


def same(a, b):
    return np.array_equal(bits(a), bits(b))


# ---------------------------------------------------------------------------
# 1. golden vectors from the reference build
# ---------------------------------------------------------------------------

def test_golden_decode_tables(o, g):
    assert same(o.e4m3_to_f32_n(np.arange(256, dtype=np.uint8)), g["e4m3_decode"].view(np.float32))
    assert same(o.e5m2_to_f32_n(np.arange(256, dtype=np.uint8)), g["e5m2_decode"].view(np.float32))
    import hashlib
    f16 = o.f16_to_f32_n(np.arange(65536, dtype=np.uint16)).view(np.uint32)
    assert hashlib.sha256(f16.tobytes()).digest() == g["f16_decode_sha256"].tobytes()


def test_golden_encoders(o, g):
    x = g["conv_x"].view(np.float32)
    assert np.array_equal(o.f32_to_f16_n(x), g["conv_f16"])
    assert np.array_equal(o.f32_to_bf16_n(x), g["conv_bf16"])
    assert np.array_equal(o.f32_to_e4m3_n(x), g["conv_e4m3"])
    assert np.array_equal(o.f32_to_e5m2_n(x), g["conv_e5m2"])


def test_golden_quantizers(o, g):
    x = g["q_x"]
    for kind in ("q8", "fp8"):
        q, s = getattr(o, f"{kind}_quantize_per_row")(x)
        assert same(q, g[f"{kind}_row_q"]) and same(s, g[f"{kind}_row_s"])
        q, s = getattr(o, f"{kind}_quantize_per_col")(x)
        assert same(q, g[f"{kind}_col_q"]) and same(s, g[f"{kind}_col_s"])
        q, s = getattr(o, f"{kind}_quantize_per_tensor")(x)
        assert same(q, g[f"{kind}_tensor_q"]) and np.float32(s) == g[f"{kind}_tensor_s"]
    for G in (32, 8, 64):
        p, s = o.q4_quantize_groupwise(g["q4_w"], G)
        assert same(p, g[f"q4_G{G}_p"]) and same(s, g[f"q4_G{G}_s"])
        assert same(o.q4_dequantize_groupwise(p, s, 64, 24, G), g[f"q4_G{G}_deq"])
    p, s = o.q4_quantize_groupwise(g["q4_G3_w"], 3)
    assert same(p, g["q4_G3_p"]) and same(s, g["q4_G3_s"])


def test_golden_gemms(o, g):
    A, B, C0 = g["g_A"], g["g_B"], g["g_C0"]
    Aq, As, Bq, Bs = g["w8_Aq"], g["w8_As"], g["w8_Bq"], g["w8_Bs"]
    for i, (al, be) in enumerate(g["alpha_beta"]):
        al, be = float(al), float(be)
        assert same(o.gemm_w8a8(Aq, Bq, As, Bs, C0, al, be), g[f"w8a8_{i}"])
        assert same(o.gemm(A, B, C0, al, be), g[f"gemm_{i}"])
        assert same(o.gemm_ref(A, B, C0, al, be), g[f"gemm_ref_{i}"])
        assert same(o.gemm_w4a16_groupwise(A, g["w4_Bp"], g["w4_Bs"], 48, 32, C0, al, be), g[f"w4a16_{i}"])
        assert same(o.gemm_fp8_e4m3(g["fp8_A"], g["fp8_B"], float(g["fp8_sa"]), float(g["fp8_sb"]), C0, al, be),
                    g[f"fp8gemm_{i}"])
    assert np.array_equal(o.gemm_w8a8_i32acc(Aq, Bq), g["w8a8_acc"])
    assert same(o.gemm_w4a16_groupwise(g["w4g128_A"], g["w4g128_Bp"], g["w4g128_Bs"], 64, 128), g["w4g128_C"])
    assert same(o.gemm_batched(g["gb_A"], g["gb_B"]), g["gemm_batched"])


# ---------------------------------------------------------------------------
# 2. the compiled reference, on fresh inputs
# ---------------------------------------------------------------------------

need_ref = pytest.mark.skipif(not ref_available(), reason="oracle/_ref not built (reference tree absent)")


@need_ref
def test_ref_conversions_exhaustive(o):
    r = Ref()
    b8 = np.arange(256, dtype=np.uint8)
    assert same(o.e4m3_to_f32_n(b8), r.e4m3_to_f32_n(b8))
    assert same(o.e5m2_to_f32_n(b8), r.e5m2_to_f32_n(b8))
    h = np.arange(65536, dtype=np.uint16)
    assert same(o.f16_to_f32_n(h), r.f16_to_f32_n(h))
    xs = np.random.default_rng(1).integers(0, 2 ** 32, 400000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    for name in ("f32_to_f16_n", "f32_to_bf16_n", "f32_to_e4m3_n", "f32_to_e5m2_n"):
        assert np.array_equal(getattr(o, name)(xs), getattr(r, name)(xs)), name


@need_ref
@pytest.mark.parametrize("seed", range(4))
def test_ref_random_quantizers_and_gemms(o, seed):
    r = Ref()
    gen = np.random.default_rng(100 + seed)
    M, K, N = (int(v) for v in gen.integers(1, 40, 3))
    K = 2 * K
    x = (gen.standard_normal((M, K)) * 10 ** gen.uniform(-3, 2)).astype(np.float32)
    for fn in ("q8_quantize_per_row", "q8_quantize_per_col", "fp8_quantize_per_row", "fp8_quantize_per_col"):
        for u, v in zip(getattr(o, fn)(x), getattr(r, fn)(x)):
            assert same(u, v), fn
    W = gen.uniform(-1, 1, (K, N)).astype(np.float32)
    G = int(gen.choice([d for d in range(1, K + 1) if K % d == 0]))
    p1, s1 = o.q4_quantize_groupwise(W, G)
    p2, s2 = r.q4_quantize_groupwise(W, G)
    assert same(p1, p2) and same(s1, s2)
    C0 = gen.uniform(-1, 1, (M, N)).astype(np.float32)
    al, be = float(gen.uniform(-2, 2)), float(gen.choice([0.0, 1.0, gen.uniform(-2, 2)]))
    assert same(o.gemm_w4a16_groupwise(x, p1, s1, N, G, C0, al, be), r.gemm_w4a16_groupwise(x, p1, s1, N, G, C0, al, be))
    Aq, As = o.q8_quantize_per_row(x)
    Bq, Bs = o.q8_quantize_per_col(W)
    assert same(o.gemm_w8a8(Aq, Bq, As, Bs, C0, al, be), r.gemm_w8a8(Aq, Bq, As, Bs, C0, al, be))
    a8, sa = o.fp8_quantize_per_tensor(x)
    b8, sb = o.fp8_quantize_per_tensor(W)
    assert same(o.gemm_fp8_e4m3(a8, b8, sa, sb, C0, al, be), r.gemm_fp8_e4m3(a8, b8, sa, sb, C0, al, be))
    assert same(o.gemm(x, W, C0, al, be), r.gemm(x, W, C0, al, be))


# ---------------------------------------------------------------------------
# 3. closed forms and independent routines
# ---------------------------------------------------------------------------

def test_f16_matches_numpy_ieee(o):
    """numpy's float32 -> float16 cast is IEEE round-to-nearest-even."""
    gen = np.random.default_rng(3)
    xs = np.concatenate([gen.integers(0, 2 ** 32, 200000, dtype=np.uint64).astype(np.uint32).view(np.float32),
                         np.float32([65504, 65519.996, 65520, 2 ** -24, 2 ** -25, 1.5 * 2 ** -25, 2 ** -26])])
    xs = xs[~np.isnan(xs)]
    with np.errstate(over="ignore"):
        want = xs.astype(np.float16).view(np.uint16)
    assert np.array_equal(o.f32_to_f16_n(xs), want)
    h = np.arange(65536, dtype=np.uint16)
    dec = o.f16_to_f32_n(h)
    ok = ~np.isnan(dec)
    assert same(dec[ok], h.view(np.float16)[ok].astype(np.float32))


def test_bf16_matches_torch(o):
    torch = pytest.importorskip("torch")
    gen = np.random.default_rng(4)
    xs = gen.integers(0, 2 ** 32, 200000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    xs = xs[~np.isnan(xs)]
    want = torch.from_numpy(xs.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(o.f32_to_bf16_n(xs), want)
    nan = np.array([np.float32(np.nan)], np.float32)
    assert o.f32_to_bf16_n(nan)[0] & 0x7fc0 == 0x7fc0


def test_e4m3_decode_closed_form(o):
    """E4M3: bias 7, 3 mantissa bits, subnormals m*2^-9, NaN only at 0x7f/0xff."""
    for b in range(256):
        s = -1.0 if b & 0x80 else 1.0
        e, m = (b >> 3) & 15, b & 7
        v = o.e4m3_to_f32(b)
        if e == 15 and m == 7:
            assert np.isnan(v)
        elif e == 0:
            assert v == s * m * 2.0 ** -9
        else:
            assert v == s * (1 + m / 8) * 2.0 ** (e - 7)


def test_e4m3_encode_vs_torch_and_quirks(o):
    """Inside [2^-9, 448] the encoder is round-to-nearest-even, which torch's
    float8_e4m3fn cast also is; outside it the reference's own rules hold:
    saturate to +-448 (0x7e) above, flush to signed zero below 2^-9."""
    torch = pytest.importorskip("torch")
    gen = np.random.default_rng(5)
    mag = np.exp2(gen.uniform(-9, np.log2(448), 100000)).astype(np.float32)
    xs = np.concatenate([mag, -mag])
    want = torch.from_numpy(xs.copy()).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(o.f32_to_e4m3_n(xs), want)
    assert o.f32_to_e4m3(1000.0) == 0x7e and o.f32_to_e4m3(-1e30) == 0xfe
    assert o.f32_to_e4m3(449.0) == 0x7e
    assert o.f32_to_e4m3(1.5 * 2 ** -10) == 0x00          # RNE would give 0x01; reference flushes
    assert o.f32_to_e4m3(-1.9 * 2 ** -10) == 0x80
    assert o.f32_to_e4m3(2 ** -9) == 0x01
    assert o.f32_to_e4m3(float("nan")) == 0x7f and o.f32_to_e4m3(float("-inf")) == 0xff


def test_e5m2_closed_form(o):
    for b in range(256):
        s = -1.0 if b & 0x80 else 1.0
        e, m = (b >> 2) & 31, b & 3
        v = o.e5m2_to_f32(b)
        if e == 31:
            assert (np.isinf(v) if m == 0 else np.isnan(v))
        elif e == 0:
            assert v == s * m * 2.0 ** -16
        else:
            assert v == s * (1 + m / 4) * 2.0 ** (e - 15)
            assert o.f32_to_e5m2(v) == b          # representable values round-trip
    assert o.f32_to_e5m2(1e6) == 0x7c


def test_q8_known_answers(o):
    # scale = 127/127 = 1: q = rint(x) with ties to even, clamp at +-127
    x = np.array([[127.0, 0.5, 1.5, 2.5, -0.5, -63.5, 63.5, -127.0, 0.0, 3.2]], np.float32)
    q, s = o.q8_quantize_per_row(x)
    assert s[0] == 1.0
    assert q.tolist() == [[127, 0, 2, 2, 0, -64, 64, -127, 0, 3]]
    q, s = o.q8_quantize_per_row(np.zeros((2, 5), np.float32))
    assert (s == 1.0).all() and not q.any()
    q, s = o.q8_quantize_per_col(np.array([[0, 2], [0, -4]], np.float32))
    assert s.tolist() == [1.0, np.float32(4 / 127)] and q.tolist() == [[0, 64], [0, -127]]


def _recip_vs_div_case():
    """x, m with rint(x * (1/(m/127))) != rint(x / (m/127)) in fp32."""
    gen = np.random.default_rng(0)
    for _ in range(200000):
        m = np.float32(gen.uniform(0.5, 2.0))
        s = np.float32(m / np.float32(127))
        inv = np.float32(np.float32(1) / s)
        k = int(gen.integers(1, 126))
        x = np.float32((k + 0.5) * s)
        if abs(x) < m and np.rint(np.float32(x * inv)) != np.rint(np.float32(x / s)):
            return x, m
    raise AssertionError("no distinguishing case found")


def test_q8_row_multiplies_col_divides(o):
    """Per-row quantization multiplies by 1/scale (quant.cpp:57-58); per-column
    divides by the scale (quant.cpp:91); the two differ on this input."""
    x, m = _recip_vs_div_case()
    s = np.float32(m / np.float32(127))
    row = np.array([[m, x]], np.float32)
    q, sr = o.q8_quantize_per_row(row)
    assert sr[0] == s and q[0, 1] == np.rint(np.float32(x * np.float32(np.float32(1) / s)))
    q, sc = o.q8_quantize_per_col(row.T.copy())
    assert sc[0] == s and q[1, 0] == np.rint(np.float32(x / s))
    assert q[1, 0] != o.q8_quantize_per_row(row)[0][0, 1]


def test_q8_invariants(o):
    x = D.normal((64, 300), 3.0, 8)
    for fn, axis in (("q8_quantize_per_row", 1), ("q8_quantize_per_col", 0)):
        q, s = getattr(o, fn)(x)
        assert np.abs(q.astype(int)).max() <= 127 and (q != -128).all()
        sc = s[:, None] if axis == 1 else s[None, :]
        assert (np.abs(q * sc - x) <= sc * 0.5 * (1 + 1e-5)).all()
        amax = np.argmax(np.abs(x), axis=axis)
        peak = q[np.arange(64), amax] if axis == 1 else q[amax, np.arange(300)]
        assert (np.abs(peak) == 127).all()


def test_q4_get_exhaustive(o):
    """Every byte value and both nibbles: low nibble = even k, high = odd k,
    two's-complement sign extension (quant.hpp:68-75)."""
    packed = np.arange(256, dtype=np.uint8).reshape(1, 256)
    for n in range(256):
        lo, hi = n & 15, n >> 4
        assert o.q4_get(packed, 0, n, 256) == (lo - 16 if lo >= 8 else lo)
        assert o.q4_get(packed, 1, n, 256) == (hi - 16 if hi >= 8 else hi)


def test_q4_known_answer_and_packing(o):
    # one group of 4 rows per column; column 0 max 7 -> scale 1
    W = np.array([[7.0, 0.0], [-3.0, 0.0], [2.5, 0.0], [-7.0, 0.0]], np.float32)
    p, s = o.q4_quantize_groupwise(W, 4)
    assert s.tolist() == [[1.0, 1.0]]
    # rows (0,1) -> byte 0: low nibble 7, high nibble -3 (0xd); rows (2,3): 2 (tie -> even), -7 (0x9)
    assert p[:, 0].tolist() == [0xd7, 0x92] and p[:, 1].tolist() == [0, 0]


def test_w8a8_acc_vs_int64_matmul(o):
    gen = np.random.default_rng(9)
    Aq = gen.integers(-127, 128, (13, 200)).astype(np.int8)
    Bq = gen.integers(-127, 128, (200, 17)).astype(np.int8)
    assert np.array_equal(o.gemm_w8a8_i32acc(Aq, Bq), Aq.astype(np.int64) @ Bq.astype(np.int64))
    ones = np.ones((1, 300), np.int8)
    assert o.gemm_w8a8_i32acc(ones, np.full((300, 1), 127, np.int8))[0, 0] == 300 * 127


def test_w8a8_epilogue_order(o):
    """C = ((alpha*a_s)*b_s)*float(acc) with separate roundings: on these
    values the product order matters in fp32."""
    gen = np.random.default_rng(11)
    for _ in range(1000):
        al, a_s, b_s = (np.float32(v) for v in gen.uniform(0.1, 3, 3))
        acc = int(gen.integers(1, 2 ** 20))
        left = np.float32(np.float32(np.float32(al * a_s) * b_s) * np.float32(acc))
        right = np.float32(al * np.float32(a_s * np.float32(b_s * np.float32(acc))))
        if left != right:
            break
    Aq = np.array([[1]], np.int8); Bq = np.array([[1]], np.int8)
    # scale acc through A: choose A = acc as sum of ones
    k = acc
    Aq = np.ones((1, k), np.int8); Bq = np.ones((k, 1), np.int8)
    got = o.gemm_w8a8(Aq, Bq, np.array([a_s]), np.array([b_s]), None, float(al), 0.0)[0, 0]
    assert bits(np.float32(got)) == bits(left) and left != right


def test_w4a16_vs_float64(o):
    """The fp32 restatement stays within fp32 reassociation of an exact
    float64 product of A and the dequantized weights."""
    A = D.uniform((8, 1024), -1, 1, 12)
    W = D.normal((1024, 96), 0.02, 13)
    p, s = o.q4_quantize_groupwise(W, 128)
    Wd = o.q4_dequantize_groupwise(p, s, 1024, 96, 128).astype(np.float64)
    assert rel_frobenius(o.gemm_w4a16_groupwise(A, p, s, 96, 128), A.astype(np.float64) @ Wd) < 1e-6


def test_q4a_closed_forms(o):
    """Asymmetric int4 (build extension, no reference): codes and zeros in
    [0,15], dequant error <= s/2, exact round trip of representable weights."""
    W = D.normal((256, 40), 0.02, 14)
    W[:128, 0] = 0.0
    W[:128, 1] = np.abs(W[:128, 1])               # one-signed group
    p, s, z = o.q4a_quantize_groupwise(W, 128)
    sf = o.f16_to_f32_n(s)
    assert (z <= 15).all() and (sf >= 2 ** -14).all()
    lo, hi = np.minimum(W.reshape(2, 128, 40).min(1), 0), np.maximum(W.reshape(2, 128, 40).max(1), 0)
    Wd = o.q4a_dequantize_groupwise(p, s, z, 256, 40, 128)
    err = np.abs(Wd - W).reshape(2, 128, 40)
    assert (err <= sf[:, None, :] * 0.5 * (1 + 1e-3) + 1e-7).all()
    assert np.all(Wd[:128, 0] == 0)
    # representable weights round-trip exactly: w = (u - z) * s with fp16 s
    gen = np.random.default_rng(15)
    u = gen.integers(0, 16, (128, 8)); u[0] = 0; u[1] = 15
    zz = gen.integers(1, 15, 8)
    sc = o.f16_to_f32_n(o.f32_to_f16_n(gen.uniform(0.001, 0.01, 8).astype(np.float32)))
    Wr = ((u - zz) * sc).astype(np.float32)
    p2, s2, z2 = o.q4a_quantize_groupwise(Wr, 128)
    assert np.allclose(o.q4a_dequantize_groupwise(p2, s2, z2, 128, 8, 128), Wr, rtol=0, atol=1e-3 * sc.max())


def test_w4a16_asym_reduces_to_reference(o):
    """With codes u = q + 8, zero 8, fp16-representable scales and
    bf16-representable activations, the asymmetric GEMM performs the same
    float operations in the same order as gemm_w4a16_groupwise: bit-identical."""
    K, N, G, M = 256, 48, 64, 5
    A = D.to_bf16_bits(o, D.uniform((M, K), -1, 1, 16))
    W = D.uniform((K, N), -1, 1, 17)
    p, s32 = o.q4_quantize_groupwise(W, G)
    s16 = o.f32_to_f16_n(s32)
    s32r = o.f16_to_f32_n(s16)                    # fp16-representable scales
    pu = ((p & 0x0f) ^ 0x08) | ((((p >> 4) & 0x0f) ^ 0x08) << 4)   # q + 8 per nibble
    got = o.gemm_w4a16_asym(A, pu.astype(np.uint8), s16, np.full((K // G, N), 8, np.uint8), N, G)
    want = o.gemm_w4a16_groupwise(D.bf16_bits_to_f32(A), p, s32r, N, G)
    assert same(got, want)


def test_moe_dispatch_table_invariants(o):
    """offsets monotone, offsets[E] = T*topk, counts match the routing,
    token order preserved within an expert (test_moe.cpp:157-163)."""
    ids = D.moe_routing(512, 8, 2, 42)
    off, tok, slot = o.moe_dispatch_table(ids, 8)
    assert off[0] == 0 and off[-1] == 1024 and (np.diff(off) >= 0).all()
    for e in range(8):
        rows = tok[off[e]:off[e + 1]]
        assert len(rows) == (ids == e).sum()
        assert (np.diff(rows) > 0).all()
        assert (ids[rows, slot[off[e]:off[e + 1]]] == e).all()


def test_grouped_equals_per_group_calls(o):
    T, E, K, N, G = 30, 3, 128, 16, 64
    ids = D.moe_routing(T, E, 2, 43)
    off, tok, _ = o.moe_dispatch_table(ids, E)
    A = D.to_bf16_bits(o, D.normal((T, K), 1.0, 44))[tok]
    Ps, Ss, Zs = zip(*[o.q4a_quantize_groupwise(D.normal((K, N), 0.02, 45 + e), G) for e in range(E)])
    got = o.gemm_w4a16_asym_grouped(A, off, np.stack(Ps), np.stack(Ss), np.stack(Zs), N, G)
    for e in range(E):
        sub = o.gemm_w4a16_asym(A[off[e]:off[e + 1]], Ps[e], Ss[e], Zs[e], N, G)
        assert same(got[off[e]:off[e + 1]], sub)


# ---------------------------------------------------------------------------
# 4. the bf16 per-token quantizer, the bf16 W8A8 epilogue, the dequantizers
#    and the ragged group driver: golden vectors, the compiled reference and
#    closed forms
# ---------------------------------------------------------------------------

def test_golden_dequantizers(o, g):
    for kind in ("q8", "fp8"):
        assert same(getattr(o, f"{kind}_dequantize_per_row")(g[f"{kind}_row_q"], g[f"{kind}_row_s"]),
                    g[f"{kind}_row_deq"])
        assert same(getattr(o, f"{kind}_dequantize_per_col")(g[f"{kind}_col_q"], g[f"{kind}_col_s"]),
                    g[f"{kind}_col_deq"])
        assert same(getattr(o, f"{kind}_dequantize_per_tensor")(g[f"{kind}_tensor_q"], float(g[f"{kind}_tensor_s"])),
                    g[f"{kind}_tensor_deq"])


def test_golden_q8_per_row_bf16(o, g):
    """quant.cpp:52-63 on the fp32 widening of bf16 rows: zero row, exact ties
    at scale 1, +-20 outliers, a NaN, a negative peak, tiny and huge rows."""
    q, s = o.q8_quantize_per_row_bf16(g["q8bf_x"])
    assert same(q, g["q8bf_q"]) and same(s, g["q8bf_s"])
    assert g["q8bf_s"][0] == 1.0 and g["q8bf_s"][1] == 1.0
    assert g["q8bf_q"][1, :9].tolist() == [127, 0, 2, 2, -2, 64, -64, 0, 126]


def test_golden_w8a8_bf16out(o, g):
    got = o.gemm_w8a8_bf16out(g["w8bf_Aq"], g["w8bf_Bq"], g["w8bf_As"], g["w8bf_Bs"])
    assert np.array_equal(got, g["w8bf_C"])


def test_golden_gemm_grouped(o, g):
    outs = o.gemm_grouped([g[f"gg_A{i}"] for i in range(3)], [g[f"gg_B{i}"] for i in range(3)],
                          [g[f"gg_C0{i}"] for i in range(3)], 0.75, -1.25)
    for i, c in enumerate(outs):
        assert same(c, g[f"gg_C{i}"])


def _bf16_rows(gen, rows, dim):
    """bf16 bit patterns of per-token rows in the shape of config 3's
    activations: N(0,1) with 0.1% of entries at +-20, plus one row of exact
    ties at scale 1, one all-zero row and one holding a NaN."""
    x = gen.standard_normal((rows, dim)).astype(np.float32)
    n_out = max(1, int(0.001 * x.size))
    pos = gen.choice(x.size, n_out, replace=False)
    x.ravel()[pos] = np.where(gen.random(n_out) < 0.5, -20.0, 20.0)
    x[0] = 0.0
    x[1] = np.round(gen.uniform(-126, 126, dim) * 2) / 2      # halves: ties at scale 1
    x[1, 0] = 127.0
    x[2, dim // 2] = np.nan
    return (x.view(np.uint32) >> 16).astype(np.uint16)


@need_ref
@pytest.mark.parametrize("seed", range(3))
def test_ref_q8_per_row_bf16_and_bf16_epilogue(o, seed):
    r = Ref()
    gen = np.random.default_rng(300 + seed)
    xb = _bf16_rows(gen, 24, int(gen.integers(64, 700)))
    q, s = o.q8_quantize_per_row_bf16(xb)
    qr, sr = r.q8_quantize_per_row(D.bf16_bits_to_f32(xb))
    assert same(q, qr) and same(s, sr)
    K, N = xb.shape[1], int(gen.integers(1, 90))
    Bq, Bs = r.q8_quantize_per_col((gen.standard_normal((K, N)) * 0.02).astype(np.float32))
    want = r.f32_to_bf16_n(r.gemm_w8a8(qr, Bq, sr, Bs, None, 1.0, 0.0))
    assert np.array_equal(o.gemm_w8a8_bf16out(q, Bq, s, Bs), want)


@need_ref
@pytest.mark.parametrize("seed", range(3))
def test_ref_dequantizers_and_grouped(o, seed):
    r = Ref()
    gen = np.random.default_rng(400 + seed)
    x = (gen.standard_normal((int(gen.integers(1, 30)), int(gen.integers(1, 50)))) * 10).astype(np.float32)
    for kind in ("q8", "fp8"):
        q, s = getattr(r, f"{kind}_quantize_per_row")(x)
        assert same(getattr(o, f"{kind}_dequantize_per_row")(q, s), getattr(r, f"{kind}_dequantize_per_row")(q, s))
        q, s = getattr(r, f"{kind}_quantize_per_col")(x)
        assert same(getattr(o, f"{kind}_dequantize_per_col")(q, s), getattr(r, f"{kind}_dequantize_per_col")(q, s))
        q, s = getattr(r, f"{kind}_quantize_per_tensor")(x)
        assert same(getattr(o, f"{kind}_dequantize_per_tensor")(q, s),
                    getattr(r, f"{kind}_dequantize_per_tensor")(q, s))
    dims = [tuple(int(v) for v in gen.integers(0, 20, 3)) for _ in range(4)]
    As = [gen.uniform(-1, 1, (m, k)).astype(np.float32) for m, k, _ in dims]
    Bs = [gen.uniform(-1, 1, (k, n)).astype(np.float32) for _, k, n in dims]
    Cs = [gen.uniform(-1, 1, (m, n)).astype(np.float32) for m, _, n in dims]
    al, be = float(gen.uniform(-2, 2)), float(gen.choice([0.0, 1.0, 0.5]))
    for u, v in zip(o.gemm_grouped(As, Bs, Cs, al, be), r.gemm_grouped(As, Bs, Cs, al, be)):
        assert same(u, v)


def _bf16_recip_vs_div_case():
    """bf16 x, m with rint(x * (1/(m/127))) != rint(x / (m/127)) in fp32."""
    for mb in range(0x3f00, 0x4000):                    # m in [0.5, 2)
        m = np.uint32(mb << 16).view(np.float32)
        s = np.float32(m / np.float32(127))
        inv = np.float32(np.float32(1) / s)
        for xb in range(0x3c00, mb):                    # 0 < x < m
            x = np.uint32(xb << 16).view(np.float32)
            if np.rint(np.float32(x * inv)) != np.rint(np.float32(x / s)):
                return x, m
    raise AssertionError("no distinguishing case found")


def test_q8_per_row_bf16_closed_forms(o):
    """The bf16 per-token quantizer: scale = max|x|/127 (1 for an all-zero
    row), q = rint(x * (1/scale)) -- the reciprocal multiply of
    quant.cpp:57-58, not a division, on a case where the two differ -- ties
    to even, NaN never the max, and equal to the fp32 per-row quantizer on
    the exact widening."""
    x, m = _bf16_recip_vs_div_case()
    row = np.array([[m, x, -x]], np.float32)
    xb = (row.view(np.uint32) >> 16).astype(np.uint16)
    q, s = o.q8_quantize_per_row_bf16(xb)
    scale = np.float32(m / np.float32(127))
    inv = np.float32(np.float32(1) / scale)
    assert s[0] == scale and q[0, 0] == 127
    assert q[0, 1] == np.rint(np.float32(x * inv)) != np.rint(np.float32(x / scale))
    assert q[0, 2] == -q[0, 1]
    ties = np.array([[127.0, 0.5, 1.5, 2.5, -0.5, -1.5, 126.5, np.nan, 0.0]], np.float32)
    q, s = o.q8_quantize_per_row_bf16((ties.view(np.uint32) >> 16).astype(np.uint16))
    assert s[0] == 1.0 and q[0, :7].tolist() == [127, 0, 2, 2, 0, -2, 126] and q[0, 8] == 0
    q, s = o.q8_quantize_per_row_bf16(np.zeros((3, 7), np.uint16))
    assert (s == 1.0).all() and not q.any()
    xb = _bf16_rows(np.random.default_rng(9), 16, 300)
    for a, b in zip(o.q8_quantize_per_row_bf16(xb), o.q8_quantize_per_row(D.bf16_bits_to_f32(xb))):
        assert same(a, b)


def test_w8a8_bf16out_closed_form(o):
    """bf16(((1*a_s)*b_s)*float(acc)), acc from an int64 matmul, the fp32
    products rounded one at a time in that order, then torch's
    round-to-nearest-even bf16 cast."""
    torch = pytest.importorskip("torch")
    gen = np.random.default_rng(10)
    Aq = gen.integers(-127, 128, (7, 333)).astype(np.int8)
    Bq = gen.integers(-127, 128, (333, 29)).astype(np.int8)
    As = gen.uniform(1e-3, 1, 7).astype(np.float32)
    Bs = gen.uniform(1e-4, 1e-2, 29).astype(np.float32)
    acc = (Aq.astype(np.int64) @ Bq.astype(np.int64)).astype(np.float32)
    f = ((np.float32(1) * As)[:, None] * Bs[None, :]).astype(np.float32) * acc
    want = torch.from_numpy(f.astype(np.float32)).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(o.gemm_w8a8_bf16out(Aq, Bq, As, Bs), want)


def test_dequantizers_closed_form(o):
    """dequant = float(q) * scale, one fp32 rounding (quant.cpp:47-50,65-73,98-105)."""
    gen = np.random.default_rng(11)
    q = gen.integers(-127, 128, (5, 9)).astype(np.int8)
    s_row = gen.uniform(0.01, 3, 5).astype(np.float32)
    s_col = gen.uniform(0.01, 3, 9).astype(np.float32)
    assert same(o.q8_dequantize_per_row(q, s_row), q.astype(np.float32) * s_row[:, None])
    assert same(o.q8_dequantize_per_col(q, s_col), q.astype(np.float32) * s_col[None, :])
    assert same(o.q8_dequantize_per_tensor(q.ravel(), 0.37), q.ravel().astype(np.float32) * np.float32(0.37))
    e = gen.integers(0, 256, (5, 9)).astype(np.uint8)
    e[e == 0x7f] = 0; e[e == 0xff] = 0
    ef = o.e4m3_to_f32_n(e)
    assert same(o.fp8_dequantize_per_row(e, s_row), ef * s_row[:, None])
    assert same(o.fp8_dequantize_per_col(e, s_col), ef * s_col[None, :])
    assert same(o.fp8_dequantize_per_tensor(e.ravel(), 0.37), ef.ravel() * np.float32(0.37))


def test_gemm_grouped_is_per_group_gemm(o):
    """gemm.cpp:69-75: group g is gemm(A[g], B[g], C[g], M[g], N[g], K[g]),
    empty groups included, against a float64 product."""
    gen = np.random.default_rng(12)
    dims = [(9, 17, 5), (0, 4, 3), (4, 0, 6), (1, 31, 2)]
    As = [gen.uniform(-1, 1, (m, k)).astype(np.float32) for m, k, _ in dims]
    Bs = [gen.uniform(-1, 1, (k, n)).astype(np.float32) for _, k, n in dims]
    Cs = [gen.uniform(-1, 1, (m, n)).astype(np.float32) for m, _, n in dims]
    outs = o.gemm_grouped(As, Bs, Cs, 1.5, 0.5)
    for a, b, c, out in zip(As, Bs, Cs, outs):
        assert same(out, o.gemm(a, b, c, 1.5, 0.5))
        want = 0.5 * c.astype(np.float64) + 1.5 * (a.astype(np.float64) @ b.astype(np.float64))
        assert np.allclose(out, want, rtol=1e-5, atol=1e-5)


def test_bf16_decode_closed_form(o):
    """bf16 -> fp32 is the 16-bit left shift of the pattern, for all 2^16."""
    h = np.arange(65536, dtype=np.uint16)
    dec = np.array([o.bf16_to_f32(int(b)) for b in h[::257]], np.float32)
    assert same(dec, (h[::257].astype(np.uint32) << 16).view(np.float32))


# ---------------------------------------------------------------------------
# 5. every exported oracle function has a pin
# ---------------------------------------------------------------------------

# lho_* symbol -> the tests that pin it (module-qualified when not in this
# file).  Scalar conversions are pinned through their array forms, which
# call them element by element.
PINS = {
    "lho_f32_to_f16": ["test_golden_encoders", "test_ref_conversions_exhaustive", "test_f16_matches_numpy_ieee"],
    "lho_f16_to_f32": ["test_golden_decode_tables", "test_ref_conversions_exhaustive", "test_f16_matches_numpy_ieee"],
    "lho_f32_to_bf16": ["test_golden_encoders", "test_ref_conversions_exhaustive", "test_bf16_matches_torch"],
    "lho_bf16_to_f32": ["test_bf16_decode_closed_form"],
    "lho_f32_to_e4m3": ["test_golden_encoders", "test_ref_conversions_exhaustive",
                        "test_e4m3_encode_vs_torch_and_quirks"],
    "lho_e4m3_to_f32": ["test_golden_decode_tables", "test_ref_conversions_exhaustive",
                        "test_e4m3_decode_closed_form"],
    "lho_f32_to_e5m2": ["test_golden_encoders", "test_ref_conversions_exhaustive", "test_e5m2_closed_form"],
    "lho_e5m2_to_f32": ["test_golden_decode_tables", "test_ref_conversions_exhaustive", "test_e5m2_closed_form"],
    "lho_f32_to_f16_n": ["test_golden_encoders", "test_f16_matches_numpy_ieee"],
    "lho_f16_to_f32_n": ["test_golden_decode_tables", "test_f16_matches_numpy_ieee"],
    "lho_f32_to_bf16_n": ["test_golden_encoders", "test_bf16_matches_torch"],
    "lho_f32_to_e4m3_n": ["test_golden_encoders", "test_e4m3_encode_vs_torch_and_quirks"],
    "lho_e4m3_to_f32_n": ["test_golden_decode_tables", "test_ref_conversions_exhaustive"],
    "lho_f32_to_e5m2_n": ["test_golden_encoders", "test_ref_conversions_exhaustive"],
    "lho_e5m2_to_f32_n": ["test_golden_decode_tables", "test_ref_conversions_exhaustive"],
    "lho_q8_quantize_per_tensor": ["test_golden_quantizers", "test_ref_dequantizers_and_grouped"],
    "lho_q8_dequantize_per_tensor": ["test_golden_dequantizers", "test_ref_dequantizers_and_grouped",
                                     "test_dequantizers_closed_form"],
    "lho_q8_quantize_per_row": ["test_golden_quantizers", "test_ref_random_quantizers_and_gemms",
                                "test_q8_known_answers", "test_q8_row_multiplies_col_divides", "test_q8_invariants"],
    "lho_q8_dequantize_per_row": ["test_golden_dequantizers", "test_ref_dequantizers_and_grouped",
                                  "test_dequantizers_closed_form"],
    "lho_q8_quantize_per_col": ["test_golden_quantizers", "test_ref_random_quantizers_and_gemms",
                                "test_q8_known_answers", "test_q8_row_multiplies_col_divides", "test_q8_invariants"],
    "lho_q8_dequantize_per_col": ["test_golden_dequantizers", "test_ref_dequantizers_and_grouped",
                                  "test_dequantizers_closed_form"],
    "lho_q4_get": ["test_q4_get_exhaustive"],
    "lho_q4_quantize_groupwise": ["test_golden_quantizers", "test_ref_random_quantizers_and_gemms",
                                  "test_q4_known_answer_and_packing"],
    "lho_q4_dequantize_groupwise": ["test_golden_quantizers", "test_w4a16_vs_float64"],
    "lho_fp8_quantize_per_tensor": ["test_golden_quantizers", "test_ref_random_quantizers_and_gemms"],
    "lho_fp8_dequantize_per_tensor": ["test_golden_dequantizers", "test_ref_dequantizers_and_grouped",
                                      "test_dequantizers_closed_form"],
    "lho_fp8_quantize_per_row": ["test_golden_quantizers", "test_ref_random_quantizers_and_gemms"],
    "lho_fp8_dequantize_per_row": ["test_golden_dequantizers", "test_ref_dequantizers_and_grouped",
                                   "test_dequantizers_closed_form"],
    "lho_fp8_quantize_per_col": ["test_golden_quantizers", "test_ref_random_quantizers_and_gemms"],
    "lho_fp8_dequantize_per_col": ["test_golden_dequantizers", "test_ref_dequantizers_and_grouped",
                                   "test_dequantizers_closed_form"],
    "lho_gemm_w8a8": ["test_golden_gemms", "test_ref_random_quantizers_and_gemms", "test_w8a8_epilogue_order"],
    "lho_gemm_w8a8_i32acc": ["test_golden_gemms", "test_w8a8_acc_vs_int64_matmul"],
    "lho_gemm_w8a8_bf16out": ["test_golden_w8a8_bf16out", "test_ref_q8_per_row_bf16_and_bf16_epilogue",
                              "test_w8a8_bf16out_closed_form"],
    "lho_gemm_w4a16_groupwise": ["test_golden_gemms", "test_ref_random_quantizers_and_gemms",
                                 "test_w4a16_vs_float64"],
    "lho_gemm_fp8_e4m3": ["test_golden_gemms", "test_ref_random_quantizers_and_gemms"],
    "lho_gemm_ref": ["test_golden_gemms"],
    "lho_gemm": ["test_golden_gemms", "test_ref_random_quantizers_and_gemms"],
    "lho_gemm_batched": ["test_golden_gemms"],
    "lho_gemm_grouped": ["test_golden_gemm_grouped", "test_ref_dequantizers_and_grouped",
                         "test_gemm_grouped_is_per_group_gemm"],
    "lho_q8_quantize_per_row_bf16": ["test_golden_q8_per_row_bf16", "test_ref_q8_per_row_bf16_and_bf16_epilogue",
                                     "test_q8_per_row_bf16_closed_forms"],
    # asymmetric int4 / bf16 I/O: no reference counterpart (closed forms and
    # reduction to the reference on the symmetric subset)
    "lho_q4a_quantize_groupwise": ["test_q4a_closed_forms"],
    "lho_q4a_dequantize_groupwise": ["test_q4a_closed_forms", "test_w4a16_asym_reduces_to_reference"],
    "lho_gemm_w4a16_asym": ["test_w4a16_asym_reduces_to_reference"],
    "lho_gemm_w4a16_asym_grouped": ["test_grouped_equals_per_group_calls"],
    # MoE routing (moe.cpp): bit-exact against the compiled reference
    "lho_moe_dispatch": ["test_moe_oracle.py::test_dispatch_reference_known_answer",
                         "test_moe_oracle.py::test_dispatch_bitexact_vs_reference"],
    "lho_moe_dispatch_table": ["test_moe_dispatch_table_invariants",
                               "test_moe_oracle.py::test_dispatch_equals_stable_sort"],
    "lho_swiglu_bf16": ["test_moe_oracle.py::test_swiglu_special_values", "test_moe_oracle.py::test_swiglu_vs_float64",
                        "test_moe_oracle.py::test_expert_mlp_vs_reference"],
    "lho_moe_combine_f32": ["test_moe_oracle.py::test_combine_bitexact_vs_reference",
                            "test_moe_oracle.py::test_combine_order_is_slot_order"],
    "lho_moe_combine_bf16": ["test_moe_oracle.py::test_combine_bf16_is_f32_combine_rounded"],
}


def _oracle_exports():
    import re
    src = open(os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "oracle", "lhq_oracle.c")).read()
    return set(re.findall(r"^EXPORT\b[^(]*?\b(lho_\w+)\s*\(", src, re.M))


def test_every_oracle_export_is_pinned():
    import importlib
    exports = _oracle_exports()
    assert len(exports) > 40
    assert exports - set(PINS) == set(), f"oracle exports without a pin: {sorted(exports - set(PINS))}"
    assert set(PINS) - exports == set(), f"pin table names unknown exports: {sorted(set(PINS) - exports)}"
    this = importlib.import_module(__name__)
    for sym, tests in PINS.items():
        for t in tests:
            mod, name = (t.split("::") if "::" in t else (None, t))
            m = this if mod is None else importlib.import_module("tests." + mod[:-3])
            assert callable(getattr(m, name, None)), f"{sym}: pin {t} does not exist"
