"""ctypes binding of ``liblonghorn_hip.so`` (the C ABI in include/longhorn_hip.h).

This is plumbing for the Python tests and ``bench.py``: device memory comes
from torch tensors (``tensor.data_ptr()``), streams from
``torch.cuda.current_stream().cuda_stream``.  Every call checks the returned
status and raises ``LhqError`` with the library's message; there is no
fallback of any kind -- if the library is missing, ``load()`` raises.
"""
from __future__ import annotations

import ctypes as C
import os
import re

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "lib", "liblonghorn_hip.so")
HEADER = os.path.join(os.path.dirname(_HERE), "include", "longhorn_hip.h")

LHQ_OK, LHQ_ERR_INVALID, LHQ_ERR_UNSUPPORTED, LHQ_ERR_HIP = 0, 1, 2, 3

_p = C.c_void_p
_i = C.c_int
_i64 = C.c_int64
_f = C.c_float

# Entry point -> argtypes (restype int unless listed in _RESTYPES).
SIGNATURES = {
    "lhq_status_string": [_i],
    "lhq_last_error": [],
    "lhq_version": [],
    "lhq_q8_quantize_per_tensor": [_p, _p, _p, _i64, _p],
    "lhq_q8_dequantize_per_tensor": [_p, _p, _p, _i64, _p],
    "lhq_q8_quantize_per_row": [_p, _p, _p, _i, _i, _p],
    "lhq_q8_dequantize_per_row": [_p, _p, _p, _i, _i, _p],
    "lhq_q8_quantize_per_row_bf16": [_p, _p, _p, _i, _i, _p],
    "lhq_q8_quantize_per_col": [_p, _p, _p, _i, _i, _p],
    "lhq_q8_dequantize_per_col": [_p, _p, _p, _i, _i, _p],
    "lhq_q4_quantize_groupwise": [_p, _p, _p, _i, _i, _i, _p],
    "lhq_q4_dequantize_groupwise": [_p, _p, _p, _i, _i, _i, _p],
    "lhq_q4a_quantize_groupwise": [_p, _p, _p, _p, _i, _i, _i, _p],
    "lhq_q4a_dequantize_groupwise": [_p, _p, _p, _p, _i, _i, _i, _p],
    "lhq_fp8_quantize_per_tensor": [_p, _p, _p, _i64, _p],
    "lhq_fp8_dequantize_per_tensor": [_p, _p, _p, _i64, _p],
    "lhq_fp8_quantize_per_row": [_p, _p, _p, _i, _i, _p],
    "lhq_fp8_dequantize_per_row": [_p, _p, _p, _i, _i, _p],
    "lhq_fp8_quantize_per_col": [_p, _p, _p, _i, _i, _p],
    "lhq_fp8_dequantize_per_col": [_p, _p, _p, _i, _i, _p],
    "lhq_w4_qweight_bytes": [_i, _i],
    "lhq_w4_scales_bytes": [_i, _i, _i, _i],
    "lhq_w4_zeros_bytes": [_i, _i, _i],
    "lhq_w4_prepack_sym": [_p, _p, _i, _i, _i, _p, _p, _p],
    "lhq_w4_prepack_asym": [_p, _p, _p, _i, _i, _i, _p, _p, _p, _p],
    "lhq_b8_prepacked_bytes": [_i, _i],
    "lhq_b8_prepack": [_p, _i, _i, _p, _p],
    "lhq_gemm_w4a16": [_p, _p, _p, _p, _i, _i, _i, _i, _f, _f, _p],
    "lhq_gemm_w4a16_bf16": [_p, _p, _p, _p, _p, _i, _i, _i, _i, _p],
    "lhq_gemm_w4a16_workspace_bytes": [_i, _i, _i, _i],
    "lhq_gemm_w4a16_ws": [_p, _p, _p, _p, _i, _i, _i, _i, _f, _f, _p, _i64, _p],
    "lhq_gemm_w4a16_bf16_workspace_bytes": [_i, _i, _i, _i],
    "lhq_gemm_w4a16_bf16_ws": [_p, _p, _p, _p, _p, _i, _i, _i, _i, _p, _i64, _p],
    "lhq_gemm_w4a16_bf16_noalloc": [_p, _p, _p, _p, _p, _i, _i, _i, _i, _p],
    "lhq_gemm_w4a16_bf16_batched": [_p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _p],
    "lhq_gemm_w4a16_bf16_grouped": [_p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _p],
    "lhq_gemm_w4a16_bf16_grouped_swiglu": [_p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _p],
    "lhq_gemm_w4a16_bf16_grouped_workspace_bytes": [_i, _i, _i, _i, _i],
    "lhq_gemm_w4a16_bf16_grouped_swiglu_workspace_bytes": [_i, _i, _i, _i, _i],
    "lhq_gemm_w4a16_bf16_grouped_ws": [_p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _p, _i64, _p],
    "lhq_gemm_w4a16_bf16_grouped_swiglu_ws": [_p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _p, _i64, _p],
    "lhq_w4_save": [C.c_char_p, _p, _p, _p, _i, _i, _i, _i, _p],
    "lhq_w4_file_info": [C.c_char_p, _p, _p, _p, _p],
    "lhq_w4_load": [C.c_char_p, _p, _p, _p, _i, _i, _i, _i, _p],
    "lhq_w4_interleave_gate_up": [_p, _p, _p, _p, _p, _p, _i, _i, _i, _p, _p, _p, _p],
    "lhq_moe_dispatch_f32": [_p, _p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _p],
    "lhq_moe_dispatch_bf16": [_p, _p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _p],
    "lhq_moe_slot_positions": [_p, _p, _p, _i, _i, _p],
    "lhq_moe_combine_f32": [_p, _p, _p, _p, _i, _i, _i, _p],
    "lhq_moe_combine_bf16": [_p, _p, _p, _p, _i, _i, _i, _p],
    "lhq_moe_combine_q8_f32": [_p, _p, _p, _p, _p, _i, _i, _i, _p],
    "lhq_moe_combine_q8_bf16": [_p, _p, _p, _p, _p, _i, _i, _i, _p],
    "lhq_moe_expert_mlp_w4a16_bf16": [_p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _p],
    "lhq_moe_expert_mlp_w4a16_bf16_ws": [_p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _p, _i64,
                                         _p],
    "lhq_gemm_w8a8": [_p, _p, _p, _p, _p, _i, _i, _i, _f, _f, _p],
    "lhq_gemm_w8a8_bf16": [_p, _p, _p, _p, _p, _i, _i, _i, _p],
    "lhq_gemm_w8a8_i32": [_p, _p, _p, _i, _i, _i, _p],
    "lhq_gemm_fp8_e4m3": [_p, _p, _p, _p, _p, _i, _i, _i, _f, _f, _p],
    "lhq_gemm_f32": [_p, _p, _p, _i, _i, _i, _f, _f, _p],
    "lhq_gemm_f32_ref": [_p, _p, _p, _i, _i, _i, _f, _f, _p],
    "lhq_gemm_f32_batched": [_p, _p, _p, _i, _i, _i, _i, _f, _f, _p],
    "lhq_selftest_bf16": [_p, _p],
}
# The diagnostics library (include/longhorn_diag.h): matrix-core rate probes.
DIAG_PATH = os.path.join(_HERE, "lib", "liblonghorn_diag.so")
DIAG_HEADER = os.path.join(os.path.dirname(_HERE), "include", "longhorn_diag.h")
DIAG_SIGNATURES = {
    "lhd_last_error": [],
    "lhd_probe_mfma_rate": [_i, _i, _i, _p, _p],
    "lhd_probe_mfma_operands": [_i, _p, _i, _i, _p, _p, _p],
}
_RESTYPES = {
    "lhq_status_string": C.c_char_p,
    "lhq_last_error": C.c_char_p,
    "lhq_w4_qweight_bytes": _i64,
    "lhq_w4_scales_bytes": _i64,
    "lhq_w4_zeros_bytes": _i64,
    "lhq_b8_prepacked_bytes": _i64,
    "lhq_gemm_w4a16_workspace_bytes": _i64,
    "lhq_gemm_w4a16_bf16_workspace_bytes": _i64,
    "lhq_gemm_w4a16_bf16_grouped_workspace_bytes": _i64,
    "lhq_gemm_w4a16_bf16_grouped_swiglu_workspace_bytes": _i64,
}


class LhqError(RuntimeError):
    def __init__(self, fn: str, status: int, msg: str):
        super().__init__(f"{fn} -> status {status}: {msg}")
        self.status = status


def header_symbols(path: str = HEADER, prefix: str = "lhq_") -> list[str]:
    """Every function name declared in include/longhorn_hip.h (or, with
    path=DIAG_HEADER and prefix="lhd_", in include/longhorn_diag.h)."""
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(" + prefix + r"\w+)\s*\(", text)))


class _Lib:
    def __init__(self, path: str):
        if not os.path.exists(path):
            raise FileNotFoundError(
                f"{path} is not built: run `python -c 'import __graft_entry__ as g; g.build()'` "
                "(the HIP backend has no fallback)")
        self.cdll = C.CDLL(path)
        self.path = path
        for name, args in SIGNATURES.items():
            fn = getattr(self.cdll, name)
            fn.argtypes = args
            fn.restype = _RESTYPES.get(name, _i)

    def last_error(self) -> str:
        return self.cdll.lhq_last_error().decode()

    def call(self, name: str, *args) -> int:
        """Call an int-returning entry point and raise on a non-zero status."""
        st = getattr(self.cdll, name)(*args)
        if st != LHQ_OK:
            raise LhqError(name, st, self.last_error())
        return st

    def status(self, name: str, *args) -> int:
        """Call an int-returning entry point and return its status unchecked."""
        return getattr(self.cdll, name)(*args)

    def __getattr__(self, name):
        return getattr(self.cdll, name)


_LIB = None


def load(path: str = LIB_PATH) -> _Lib:
    global _LIB
    if _LIB is None or _LIB.path != path:
        _LIB = _Lib(path)
    return _LIB


class _DiagLib:
    """liblonghorn_diag.so: the matrix-core rate probes (include/longhorn_diag.h)."""

    def __init__(self, path: str):
        if not os.path.exists(path):
            raise FileNotFoundError(
                f"{path} is not built: run `python -c 'import __graft_entry__ as g; g.build()'`")
        self.cdll = C.CDLL(path)
        self.path = path
        for name, args in DIAG_SIGNATURES.items():
            fn = getattr(self.cdll, name)
            fn.argtypes = args
            fn.restype = C.c_char_p if name == "lhd_last_error" else _i

    def last_error(self) -> str:
        return self.cdll.lhd_last_error().decode()

    def call(self, name: str, *args) -> int:
        st = getattr(self.cdll, name)(*args)
        if st != LHQ_OK:
            raise LhqError(name, st, self.last_error())
        return st

    def status(self, name: str, *args) -> int:
        return getattr(self.cdll, name)(*args)


_DIAG = None


def load_diag(path: str = DIAG_PATH) -> _DiagLib:
    global _DIAG
    if _DIAG is None or _DIAG.path != path:
        _DIAG = _DiagLib(path)
    return _DIAG
