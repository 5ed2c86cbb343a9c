"""CPU parity checkers for the quantized-GEMM path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline
leg import this package.  The product path (``liblonghorn_hip.so`` and the
``lh::`` drop-in) never touches it.

Two checkers share one numpy-level interface:

* ``Oracle`` -- ``liboracle.so``, the C restatement in ``lhq_oracle.c`` of
  the reference functions (quant.cpp, gemm_quant.cpp, gemm.cpp,
  dtypes.hpp), built by ``oracle/Makefile``.
* ``Ref`` -- ``_ref/libref.so``, the reference's own quant/gemm sources
  compiled where they lie (only where the reference tree was present at
  build time; absent on a machine that never had it).
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
# LHO_ORACLE_SO selects another build of the same restatement (the
# sanitizer build, oracle/_asan/liboracle.so).
ORACLE_SO = os.environ.get("LHO_ORACLE_SO") or os.path.join(_HERE, "liboracle.so")
REF_SO = os.path.join(_HERE, "_ref", "libref.so")

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_i = C.c_int
_i64 = C.c_int64
_f = C.c_float

# name -> (restype, argtypes); the same table serves both libraries with the
# "lho_" / "ref_" prefix.
_COMMON = {
    "f32_to_f16": (C.c_uint16, [_f]),
    "f16_to_f32": (_f, [C.c_uint16]),
    "f32_to_bf16": (C.c_uint16, [_f]),
    "bf16_to_f32": (_f, [C.c_uint16]),
    "f32_to_e4m3": (C.c_uint8, [_f]),
    "e4m3_to_f32": (_f, [C.c_uint8]),
    "f32_to_e5m2": (C.c_uint8, [_f]),
    "e5m2_to_f32": (_f, [C.c_uint8]),
    "q8_quantize_per_tensor": (None, [_f32p, _i8p, _f32p, _i64]),
    "q8_dequantize_per_tensor": (None, [_i8p, _f, _f32p, _i64]),
    "q8_quantize_per_row": (None, [_f32p, _i8p, _f32p, _i, _i]),
    "q8_dequantize_per_row": (None, [_i8p, _f32p, _f32p, _i, _i]),
    "q8_quantize_per_col": (None, [_f32p, _i8p, _f32p, _i, _i]),
    "q8_dequantize_per_col": (None, [_i8p, _f32p, _f32p, _i, _i]),
    "q4_quantize_groupwise": (None, [_f32p, _u8p, _f32p, _i, _i, _i]),
    "q4_dequantize_groupwise": (None, [_u8p, _f32p, _f32p, _i, _i, _i]),
    "q4_get": (C.c_int8, [_u8p, _i, _i, _i]),
    "fp8_quantize_per_tensor": (None, [_f32p, _u8p, _f32p, _i64]),
    "fp8_dequantize_per_tensor": (None, [_u8p, _f, _f32p, _i64]),
    "fp8_quantize_per_row": (None, [_f32p, _u8p, _f32p, _i, _i]),
    "fp8_dequantize_per_row": (None, [_u8p, _f32p, _f32p, _i, _i]),
    "fp8_quantize_per_col": (None, [_f32p, _u8p, _f32p, _i, _i]),
    "fp8_dequantize_per_col": (None, [_u8p, _f32p, _f32p, _i, _i]),
    "gemm_w8a8": (None, [_i8p, _i8p, _f32p, _f32p, _f32p, _i, _i, _i, _f, _f]),
    "gemm_w4a16_groupwise": (None, [_f32p, _u8p, _f32p, _f32p, _i, _i, _i, _i, _f, _f]),
    "gemm_fp8_e4m3": (None, [_u8p, _u8p, _f, _f, _f32p, _i, _i, _i, _f, _f]),
    "gemm_ref": (None, [_f32p, _f32p, _f32p, _i, _i, _i, _f, _f]),
    "gemm": (None, [_f32p, _f32p, _f32p, _i, _i, _i, _f, _f]),
    "gemm_batched": (None, [_f32p, _f32p, _f32p, _i, _i, _i, _i, _f, _f]),
    "gemm_grouped": (None, [C.c_void_p, C.c_void_p, C.c_void_p, _i32p, _i32p, _i32p, _i, _f, _f]),
}
_COMMON.update({
    "f32_to_f16_n": (None, [_f32p, _u16p, _i64]),
    "f16_to_f32_n": (None, [_u16p, _f32p, _i64]),
    "f32_to_bf16_n": (None, [_f32p, _u16p, _i64]),
    "f32_to_e4m3_n": (None, [_f32p, _u8p, _i64]),
    "e4m3_to_f32_n": (None, [_u8p, _f32p, _i64]),
    "f32_to_e5m2_n": (None, [_f32p, _u8p, _i64]),
    "e5m2_to_f32_n": (None, [_u8p, _f32p, _i64]),
})
_ORACLE_ONLY = {
    "gemm_w8a8_i32acc": (None, [_i8p, _i8p, _i32p, _i, _i, _i]),
    "gemm_w8a8_bf16out": (None, [_i8p, _i8p, _f32p, _f32p, _u16p, _i, _i, _i]),
    "q8_quantize_per_row_bf16": (None, [_u16p, _i8p, _f32p, _i, _i]),
    "q4a_quantize_groupwise": (None, [_f32p, _u8p, _u16p, _u8p, _i, _i, _i]),
    "q4a_dequantize_groupwise": (None, [_u8p, _u16p, _u8p, _f32p, _i, _i, _i]),
    "gemm_w4a16_asym": (None, [_u16p, _u8p, _u16p, _u8p, _f32p, _i, _i, _i, _i]),
    "gemm_w4a16_asym_grouped": (None, [_u16p, _i32p, _u8p, _u16p, _u8p, _f32p, _i, _i, _i, _i]),
    "moe_dispatch_table": (None, [_i32p, _i, _i, _i, _i32p, _i32p, _i32p]),
    "moe_dispatch": (None, [C.c_void_p, _i64, _i32p, _i, _i, _i, _i32p, _i32p, _i32p, _i32p,
                            C.c_void_p]),
    "swiglu_bf16": (None, [_f32p, _f32p, _u16p, _i64]),
    "moe_combine_f32": (None, [_f32p, _i32p, _i32p, _f32p, _f32p, _i, _i, _i]),
    "moe_combine_bf16": (None, [_u16p, _i32p, _i32p, _f32p, _u16p, _i, _i, _i]),
}
# the reference's MoE functions (moe.hpp:75-102), exported by ref_shim.cpp
_REF_ONLY = {
    "moe_dispatch": (None, [_f32p, _i32p, _i32p, _i32p, _i32p, _f32p, _i, _i, _i, _i]),
    "moe_expert_mlp": (None, [_f32p, _i32p, _f32p, _f32p, _f32p, _f32p, _i, _i, _i]),
    "moe_combine": (None, [_f32p, _i32p, _i32p, _i32p, _f32p, _f32p, _i, _i, _i, _i]),
}


def _bind(so_path: str, prefix: str, table: dict):
    lib = C.CDLL(so_path)
    fns = {}
    for name, (res, args) in table.items():
        fn = getattr(lib, prefix + name)
        fn.restype = res
        fn.argtypes = args
        fns[name] = fn
    return lib, fns


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


class _Checker:
    """numpy-level wrappers; every array result is freshly allocated."""

    def __init__(self, so_path: str, prefix: str, table: dict):
        if not os.path.exists(so_path):
            raise FileNotFoundError(f"{so_path} is not built (run oracle/Makefile)")
        self._lib, self.fn = _bind(so_path, prefix, table)

    # -- scalar conversions ------------------------------------------------
    def f32_to_f16(self, x: float) -> int: return int(self.fn["f32_to_f16"](x))
    def f16_to_f32(self, h: int) -> float: return float(self.fn["f16_to_f32"](h))
    def f32_to_bf16(self, x: float) -> int: return int(self.fn["f32_to_bf16"](x))
    def bf16_to_f32(self, b: int) -> float: return float(self.fn["bf16_to_f32"](b))
    def f32_to_e4m3(self, x: float) -> int: return int(self.fn["f32_to_e4m3"](x))
    def e4m3_to_f32(self, b: int) -> float: return float(self.fn["e4m3_to_f32"](b))
    def f32_to_e5m2(self, x: float) -> int: return int(self.fn["f32_to_e5m2"](x))
    def e5m2_to_f32(self, b: int) -> float: return float(self.fn["e5m2_to_f32"](b))

    # -- vectorised conversions ---------------------------------------------
    def f32_to_bf16_n(self, x):
        x = _c(x, np.float32); y = np.empty(x.shape, np.uint16)
        self.fn["f32_to_bf16_n"](x.ravel(), y.ravel(), x.size)
        return y

    def f32_to_f16_n(self, x):
        x = _c(x, np.float32); y = np.empty(x.shape, np.uint16)
        self.fn["f32_to_f16_n"](x.ravel(), y.ravel(), x.size)
        return y

    def f16_to_f32_n(self, h):
        h = _c(h, np.uint16); y = np.empty(h.shape, np.float32)
        self.fn["f16_to_f32_n"](h.ravel(), y.ravel(), h.size)
        return y

    def f32_to_e4m3_n(self, x):
        x = _c(x, np.float32); y = np.empty(x.shape, np.uint8)
        self.fn["f32_to_e4m3_n"](x.ravel(), y.ravel(), x.size)
        return y

    def e4m3_to_f32_n(self, b):
        b = _c(b, np.uint8); y = np.empty(b.shape, np.float32)
        self.fn["e4m3_to_f32_n"](b.ravel(), y.ravel(), b.size)
        return y

    def f32_to_e5m2_n(self, x):
        x = _c(x, np.float32); y = np.empty(x.shape, np.uint8)
        self.fn["f32_to_e5m2_n"](x.ravel(), y.ravel(), x.size)
        return y

    def e5m2_to_f32_n(self, b):
        b = _c(b, np.uint8); y = np.empty(b.shape, np.float32)
        self.fn["e5m2_to_f32_n"](b.ravel(), y.ravel(), b.size)
        return y

    # -- int8 quantizers (quant.cpp:34-105) --------------------------------
    def q8_quantize_per_tensor(self, x):
        x = _c(x, np.float32); q = np.empty(x.shape, np.int8); s = np.zeros(1, np.float32)
        self.fn["q8_quantize_per_tensor"](x.ravel(), q.ravel(), s, x.size)
        return q, float(s[0])

    def q8_dequantize_per_tensor(self, q, scale):
        q = _c(q, np.int8); d = np.empty(q.shape, np.float32)
        self.fn["q8_dequantize_per_tensor"](q.ravel(), scale, d.ravel(), q.size)
        return d

    def q8_quantize_per_row(self, x):
        x = _c(x, np.float32); r, c = x.shape
        q = np.empty((r, c), np.int8); s = np.empty(r, np.float32)
        self.fn["q8_quantize_per_row"](x, q, s, r, c)
        return q, s

    def q8_dequantize_per_row(self, q, s):
        q = _c(q, np.int8); r, c = q.shape; d = np.empty((r, c), np.float32)
        self.fn["q8_dequantize_per_row"](q, _c(s, np.float32), d, r, c)
        return d

    def q8_quantize_per_col(self, x):
        x = _c(x, np.float32); r, c = x.shape
        q = np.empty((r, c), np.int8); s = np.empty(c, np.float32)
        self.fn["q8_quantize_per_col"](x, q, s, r, c)
        return q, s

    def q8_dequantize_per_col(self, q, s):
        q = _c(q, np.int8); r, c = q.shape; d = np.empty((r, c), np.float32)
        self.fn["q8_dequantize_per_col"](q, _c(s, np.float32), d, r, c)
        return d

    # -- int4 group quantizers (quant.cpp:111-172) --------------------------
    def q4_quantize_groupwise(self, w, G):
        w = _c(w, np.float32); K, N = w.shape
        p = np.zeros((K // 2, N), np.uint8); s = np.empty((K // G, N), np.float32)
        self.fn["q4_quantize_groupwise"](w, p, s, K, N, G)
        return p, s

    def q4_dequantize_groupwise(self, p, s, K, N, G):
        d = np.empty((K, N), np.float32)
        self.fn["q4_dequantize_groupwise"](_c(p, np.uint8), _c(s, np.float32), d, K, N, G)
        return d

    def q4_get(self, p, k, n, N):
        return int(self.fn["q4_get"](_c(p, np.uint8).ravel(), k, n, N))

    # -- fp8 quantizers (quant.cpp:176-249) ---------------------------------
    def fp8_quantize_per_tensor(self, x):
        x = _c(x, np.float32); q = np.empty(x.shape, np.uint8); s = np.zeros(1, np.float32)
        self.fn["fp8_quantize_per_tensor"](x.ravel(), q.ravel(), s, x.size)
        return q, float(s[0])

    def fp8_dequantize_per_tensor(self, q, scale):
        q = _c(q, np.uint8); d = np.empty(q.shape, np.float32)
        self.fn["fp8_dequantize_per_tensor"](q.ravel(), scale, d.ravel(), q.size)
        return d

    def fp8_quantize_per_row(self, x):
        x = _c(x, np.float32); r, c = x.shape
        q = np.empty((r, c), np.uint8); s = np.empty(r, np.float32)
        self.fn["fp8_quantize_per_row"](x, q, s, r, c)
        return q, s

    def fp8_dequantize_per_row(self, q, s):
        q = _c(q, np.uint8); r, c = q.shape; d = np.empty((r, c), np.float32)
        self.fn["fp8_dequantize_per_row"](q, _c(s, np.float32), d, r, c)
        return d

    def fp8_quantize_per_col(self, x):
        x = _c(x, np.float32); r, c = x.shape
        q = np.empty((r, c), np.uint8); s = np.empty(c, np.float32)
        self.fn["fp8_quantize_per_col"](x, q, s, r, c)
        return q, s

    def fp8_dequantize_per_col(self, q, s):
        q = _c(q, np.uint8); r, c = q.shape; d = np.empty((r, c), np.float32)
        self.fn["fp8_dequantize_per_col"](q, _c(s, np.float32), d, r, c)
        return d

    # -- GEMMs (gemm_quant.cpp, gemm.cpp) -----------------------------------
    def gemm_w8a8(self, Aq, Bq, As, Bs, C0=None, alpha=1.0, beta=0.0):
        M, K = Aq.shape; N = Bq.shape[1]
        Cout = np.zeros((M, N), np.float32) if C0 is None else _c(C0, np.float32).copy()
        self.fn["gemm_w8a8"](_c(Aq, np.int8), _c(Bq, np.int8), _c(As, np.float32),
                             _c(Bs, np.float32), Cout, M, N, K, alpha, beta)
        return Cout

    def gemm_w4a16_groupwise(self, A, Bp, Bs, N, G, C0=None, alpha=1.0, beta=0.0):
        A = _c(A, np.float32); M, K = A.shape
        Cout = np.zeros((M, N), np.float32) if C0 is None else _c(C0, np.float32).copy()
        self.fn["gemm_w4a16_groupwise"](A, _c(Bp, np.uint8), _c(Bs, np.float32), Cout,
                                        M, N, K, G, alpha, beta)
        return Cout

    def gemm_fp8_e4m3(self, A8, B8, sa, sb, C0=None, alpha=1.0, beta=0.0):
        M, K = A8.shape; N = B8.shape[1]
        Cout = np.zeros((M, N), np.float32) if C0 is None else _c(C0, np.float32).copy()
        self.fn["gemm_fp8_e4m3"](_c(A8, np.uint8), _c(B8, np.uint8), sa, sb, Cout,
                                 M, N, K, alpha, beta)
        return Cout

    def gemm_ref(self, A, B, C0=None, alpha=1.0, beta=0.0):
        M, K = A.shape; N = B.shape[1]
        Cout = np.zeros((M, N), np.float32) if C0 is None else _c(C0, np.float32).copy()
        self.fn["gemm_ref"](_c(A, np.float32), _c(B, np.float32), Cout, M, N, K, alpha, beta)
        return Cout

    def gemm(self, A, B, C0=None, alpha=1.0, beta=0.0):
        M, K = A.shape; N = B.shape[1]
        Cout = np.zeros((M, N), np.float32) if C0 is None else _c(C0, np.float32).copy()
        self.fn["gemm"](_c(A, np.float32), _c(B, np.float32), Cout, M, N, K, alpha, beta)
        return Cout

    def gemm_batched(self, A, B, C0=None, alpha=1.0, beta=0.0):
        b, M, K = A.shape; N = B.shape[2]
        Cout = np.zeros((b, M, N), np.float32) if C0 is None else _c(C0, np.float32).copy()
        self.fn["gemm_batched"](_c(A, np.float32), _c(B, np.float32), Cout, b, M, N, K,
                                alpha, beta)
        return Cout

    def gemm_grouped(self, As, Bs, C0s=None, alpha=1.0, beta=0.0):
        """Ragged pointer-array groups (gemm.cpp:69-75): one fp32 GEMM per
        (As[g], Bs[g]) pair; returns the list of outputs."""
        As = [_c(a, np.float32) for a in As]
        Bs = [_c(b, np.float32) for b in Bs]
        Cs = [np.zeros((a.shape[0], b.shape[1]), np.float32) if C0s is None else _c(c, np.float32).copy()
              for a, b, c in zip(As, Bs, C0s if C0s is not None else [None] * len(As))]
        ptrs = lambda xs: (C.c_void_p * len(xs))(*[x.ctypes.data for x in xs])  # noqa: E731
        M = np.array([a.shape[0] for a in As], np.int32)
        K = np.array([a.shape[1] for a in As], np.int32)
        N = np.array([b.shape[1] for b in Bs], np.int32)
        self.fn["gemm_grouped"](ptrs(As), ptrs(Bs), ptrs(Cs), M, N, K, len(As), alpha, beta)
        return Cs


class Oracle(_Checker):
    """The C restatement (always available once oracle/Makefile has run)."""

    def __init__(self, so_path: str = ORACLE_SO):
        super().__init__(so_path, "lho_", {**_COMMON, **_ORACLE_ONLY})

    # -- build-side extensions ------------------------------------------------
    def gemm_w8a8_i32acc(self, Aq, Bq):
        M, K = Aq.shape; N = Bq.shape[1]; acc = np.empty((M, N), np.int32)
        self.fn["gemm_w8a8_i32acc"](_c(Aq, np.int8), _c(Bq, np.int8), acc, M, N, K)
        return acc

    def gemm_w8a8_bf16out(self, Aq, Bq, As, Bs):
        M, K = Aq.shape; N = Bq.shape[1]; out = np.empty((M, N), np.uint16)
        self.fn["gemm_w8a8_bf16out"](_c(Aq, np.int8), _c(Bq, np.int8), _c(As, np.float32),
                                     _c(Bs, np.float32), out, M, N, K)
        return out

    def q8_quantize_per_row_bf16(self, xb):
        xb = _c(xb, np.uint16); r, c = xb.shape
        q = np.empty((r, c), np.int8); s = np.empty(r, np.float32)
        self.fn["q8_quantize_per_row_bf16"](xb, q, s, r, c)
        return q, s

    def q4a_quantize_groupwise(self, w, G):
        w = _c(w, np.float32); K, N = w.shape
        p = np.zeros((K // 2, N), np.uint8)
        s = np.empty((K // G, N), np.uint16); z = np.empty((K // G, N), np.uint8)
        self.fn["q4a_quantize_groupwise"](w, p, s, z, K, N, G)
        return p, s, z

    def q4a_dequantize_groupwise(self, p, s, z, K, N, G):
        d = np.empty((K, N), np.float32)
        self.fn["q4a_dequantize_groupwise"](_c(p, np.uint8), _c(s, np.uint16), _c(z, np.uint8),
                                            d, K, N, G)
        return d

    def gemm_w4a16_asym(self, Ab, p, s, z, N, G):
        Ab = _c(Ab, np.uint16); M, K = Ab.shape; Cout = np.empty((M, N), np.float32)
        self.fn["gemm_w4a16_asym"](Ab, _c(p, np.uint8), _c(s, np.uint16), _c(z, np.uint8),
                                   Cout, M, N, K, G)
        return Cout

    def gemm_w4a16_asym_grouped(self, Ab, offsets, p, s, z, N, G):
        Ab = _c(Ab, np.uint16); T, K = Ab.shape; E = len(offsets) - 1
        Cout = np.zeros((T, N), np.float32)
        self.fn["gemm_w4a16_asym_grouped"](Ab, _c(offsets, np.int32), _c(p, np.uint8),
                                           _c(s, np.uint16), _c(z, np.uint8), Cout, E, N, K, G)
        return Cout

    def moe_dispatch_table(self, expert_ids, E):
        ids = _c(expert_ids, np.int32); T, topk = ids.shape
        off = np.empty(E + 1, np.int32)
        tok = np.empty(T * topk, np.int32); slot = np.empty(T * topk, np.int32)
        self.fn["moe_dispatch_table"](ids, T, topk, E, off, tok, slot)
        return off, tok, slot

    def moe_dispatch(self, hidden, expert_ids, E):
        """moe.cpp:102-140 with the row copy; hidden is [T, H] of any dtype
        (rows are copied as bytes).  Returns offsets, token_idx, slot_idx,
        slot_pos and the dispatched rows [T*topk, H]."""
        ids = _c(expert_ids, np.int32); T, topk = ids.shape
        hidden = np.ascontiguousarray(hidden); assert hidden.shape[0] == T
        out = np.zeros((T * topk,) + hidden.shape[1:], hidden.dtype)
        off = np.empty(E + 1, np.int32)
        tok = np.empty(T * topk, np.int32); slot = np.empty(T * topk, np.int32)
        pos = np.empty(T * topk, np.int32)
        rb = hidden.strides[0] if T else 0
        self.fn["moe_dispatch"](hidden.ctypes.data, rb, ids, T, topk, E, off, tok, slot, pos,
                                out.ctypes.data)
        return off, tok, slot, pos, out

    def swiglu_bf16(self, g, u):
        g = _c(g, np.float32); u = _c(u, np.float32); act = np.empty(g.shape, np.uint16)
        self.fn["swiglu_bf16"](g, u, act, g.size)
        return act

    def moe_combine_f32(self, y, token_idx, slot_idx, gates):
        gates = _c(gates, np.float32); T, topk = gates.shape; H = y.shape[1]
        out = np.empty((T, H), np.float32)
        self.fn["moe_combine_f32"](_c(y, np.float32), _c(token_idx, np.int32), _c(slot_idx, np.int32),
                                   gates, out, T, H, topk)
        return out

    def moe_combine_bf16(self, y, token_idx, slot_idx, gates):
        gates = _c(gates, np.float32); T, topk = gates.shape; H = y.shape[1]
        out = np.empty((T, H), np.uint16)
        self.fn["moe_combine_bf16"](_c(y, np.uint16), _c(token_idx, np.int32), _c(slot_idx, np.int32),
                                    gates, out, T, H, topk)
        return out

    def moe_expert_mlp_w4a16(self, X, offsets, gate, up, down, H, I, G):
        """The quantized expert MLP (moe.cpp:150-196 with W4A16 experts, the
        hook of moe.hpp:26-28): per expert, gate and up projections in fp32,
        act = bf16(silu(g) * u), then the down projection, output rounded to
        bf16.  gate / up / down are (packed, scales, zeros) stacks over the
        experts in the lho_q4a layout.  Returns (act, y) as bf16 bits; rows
        past offsets[E] are zero."""
        g = self.gemm_w4a16_asym_grouped(X, offsets, *gate, I, G)
        u = self.gemm_w4a16_asym_grouped(X, offsets, *up, I, G)
        act = self.swiglu_bf16(g, u)
        y = self.gemm_w4a16_asym_grouped(act, offsets, *down, H, G)
        return act, self.f32_to_bf16_n(y)


class Ref(_Checker):
    """The reference's own sources, compiled in oracle/_ref (optional)."""

    def __init__(self, so_path: str = REF_SO):
        super().__init__(so_path, "ref_", {**_COMMON, **_REF_ONLY})

    def moe_dispatch(self, hidden, expert_ids, E):
        ids = _c(expert_ids, np.int32); T, topk = ids.shape
        hidden = _c(hidden, np.float32); H = hidden.shape[1]
        off = np.empty(E + 1, np.int32)
        tok = np.empty(T * topk, np.int32); slot = np.empty(T * topk, np.int32)
        out = np.empty((T * topk, H), np.float32)
        self.fn["moe_dispatch"](hidden, ids, off, tok, slot, out, T, H, E, topk)
        return off, tok, slot, out

    def moe_expert_mlp(self, X, offsets, Wg, Wu, Wd):
        X = _c(X, np.float32); E, H, I = Wg.shape
        y = np.zeros((X.shape[0], H), np.float32)
        self.fn["moe_expert_mlp"](X, _c(offsets, np.int32), _c(Wg, np.float32), _c(Wu, np.float32),
                                  _c(Wd, np.float32), y, H, I, E)
        return y

    def moe_combine(self, y, offsets, token_idx, slot_idx, gates):
        gates = _c(gates, np.float32); T, topk = gates.shape; H = y.shape[1]
        out = np.empty((T, H), np.float32)
        self.fn["moe_combine"](_c(y, np.float32), _c(offsets, np.int32), _c(token_idx, np.int32),
                               _c(slot_idx, np.int32), gates, out, T, H, len(offsets) - 1, topk)
        return out


def ref_available() -> bool:
    return os.path.exists(REF_SO)


# -- helpers shared by tests and bench -----------------------------------------

def bf16_bits_to_f32(b):
    """Exact widening of bf16 bit patterns (uint16) to float32."""
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def rel_frobenius(got, want) -> float:
    """||got - want||_F / ||want||_F in float64 (test_gemm_quant.cpp:14-27's
    relative RMS is the same quantity)."""
    g = np.asarray(got, np.float64); w = np.asarray(want, np.float64)
    den = np.linalg.norm(w.ravel())
    num = np.linalg.norm((g - w).ravel())
    return float(num / den) if den > 0 else float(num)
