"""Torch-tensor helpers over the C ABI, for tests and ``bench.py``.

Torch is only plumbing here: it owns device memory and the current stream.
Every compute call goes through ``liblonghorn_hip.so`` (``capi.load()``), and
a missing library raises -- nothing here computes anything itself.

bf16 / fp16 data travels as raw 16-bit patterns in ``torch.int16`` tensors so
no torch conversion can touch the bits.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

from . import capi

_NP_TO_TORCH = {
    np.dtype(np.float32): torch.float32,
    np.dtype(np.int8): torch.int8,
    np.dtype(np.uint8): torch.uint8,
    np.dtype(np.int16): torch.int16,
    np.dtype(np.int32): torch.int32,
    np.dtype(np.int64): torch.int64,
}
_VIEW = {np.dtype(np.uint16): np.int16, np.dtype(np.uint32): np.int32}


def lib():
    return capi.load()


def stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def dev(a: np.ndarray, device: str = "cuda") -> torch.Tensor:
    """Copy a numpy array to the device, bit for bit (uint16/uint32 via int views)."""
    a = np.ascontiguousarray(a)
    if a.dtype in _VIEW:
        a = a.view(_VIEW[a.dtype])
    return torch.from_numpy(a.copy()).to(device)


def host(t: torch.Tensor, dtype=None) -> np.ndarray:
    a = t.detach().cpu().numpy()
    return a.view(dtype) if dtype is not None else a


def empty(shape, np_dtype, device: str = "cuda") -> torch.Tensor:
    dt = np.dtype(np_dtype)
    dt = np.dtype(_VIEW.get(dt, dt))
    return torch.empty(tuple(shape), dtype=_NP_TO_TORCH[dt], device=device)


def zeros(shape, np_dtype, device: str = "cuda") -> torch.Tensor:
    t = empty(shape, np_dtype, device)
    t.zero_()
    return t


def P(t) -> int:
    return 0 if t is None else t.data_ptr()


def run(name: str, *args) -> None:
    """Call a C-ABI entry point with tensors passed directly.

    Tensors (and numpy arrays, copied to the device here) stay referenced
    until the call has enqueued its kernels; after that, torch's
    stream-ordered allocator cannot hand their memory to later work on the
    same stream before the kernels finish."""
    keep = []
    conv = []
    for a in args:
        if isinstance(a, np.ndarray):
            a = dev(a)
        if isinstance(a, torch.Tensor):
            keep.append(a)
            conv.append(a.data_ptr())
        elif a is None:
            conv.append(0)
        else:
            conv.append(a)
    lib().call(name, *conv, stream())
    del keep


# ---------------------------------------------------------------------------
# Prepacked weights
# ---------------------------------------------------------------------------

@dataclass
class W4Weights:
    """Prepacked int4 weights (layout in include/longhorn_hip.h)."""
    qweight: torch.Tensor
    scales: torch.Tensor
    zeros: torch.Tensor | None
    K: int
    N: int
    G: int
    asym: bool

    @property
    def nbytes(self) -> int:
        n = self.qweight.numel() + self.scales.numel() * self.scales.element_size()
        if self.zeros is not None:
            n += self.zeros.numel() * 4
        return n


def w4_buffers(K: int, N: int, G: int, asym: bool):
    L = lib()
    qb = L.lhq_w4_qweight_bytes(K, N)
    sb = L.lhq_w4_scales_bytes(K, N, G, 1 if asym else 0)
    zb = L.lhq_w4_zeros_bytes(K, N, G) if asym else 0
    if qb <= 0 or sb <= 0:
        raise ValueError(f"bad W4 dims K={K} N={N} G={G}")
    q = empty((qb,), np.uint8)
    s = empty((sb // 2,), np.int16) if asym else empty((sb // 4,), np.float32)
    z = empty((zb // 4,), np.int32) if asym else None
    return q, s, z


def prepack_w4_sym(packed: torch.Tensor, scales: torch.Tensor, K: int, N: int, G: int) -> W4Weights:
    """Reference-layout int4 ([K/2,N] bytes, fp32 [K/G,N] scales) -> prepacked."""
    q, s, _ = w4_buffers(K, N, G, False)
    lib().call("lhq_w4_prepack_sym", P(packed), P(scales), K, N, G, P(q), P(s), stream())
    return W4Weights(q, s, None, K, N, G, False)


def prepack_w4_asym(packed: torch.Tensor, scales_f16: torch.Tensor, zeros_u8: torch.Tensor,
                    K: int, N: int, G: int) -> W4Weights:
    q, s, z = w4_buffers(K, N, G, True)
    lib().call("lhq_w4_prepack_asym", P(packed), P(scales_f16), P(zeros_u8), K, N, G,
               P(q), P(s), P(z), stream())
    return W4Weights(q, s, z, K, N, G, True)


def interleave_gate_up(wg: W4Weights, wu: W4Weights) -> W4Weights:
    """Gate and up projections [K, I] (asymmetric, prepacked) -> one tensor
    with 2 ceil(I/16) interleaved column tiles; N stays I."""
    if (wg.K, wg.N, wg.G, wg.asym) != (wu.K, wu.N, wu.G, wu.asym) or not wg.asym:
        raise ValueError("gate and up must be asymmetric W4 of one shape")
    q = empty((2 * wg.qweight.numel(),), np.uint8)
    s = empty((2 * wg.scales.numel(),), np.int16)
    z = empty((2 * wg.zeros.numel(),), np.int32)
    lib().call("lhq_w4_interleave_gate_up", P(wg.qweight), P(wg.scales), P(wg.zeros), P(wu.qweight),
               P(wu.scales), P(wu.zeros), wg.K, wg.N, wg.G, P(q), P(s), P(z), stream())
    return W4Weights(q, s, z, wg.K, wg.N, wg.G, True)


def pointer_tables(ws: list[W4Weights]):
    """Device arrays of the per-group qweight / scales / zeros pointers."""
    def tab(ts):
        return torch.tensor([t.data_ptr() for t in ts], dtype=torch.int64, device="cuda")
    return tab([w.qweight for w in ws]), tab([w.scales for w in ws]), tab([w.zeros for w in ws])


def prepack_b8(B: torch.Tensor, K: int, N: int) -> torch.Tensor:
    nbytes = lib().lhq_b8_prepacked_bytes(K, N)
    Bt = empty((nbytes,), np.uint8)
    lib().call("lhq_b8_prepack", P(B), K, N, P(Bt), stream())
    return Bt


# ---------------------------------------------------------------------------
# GEMMs
# ---------------------------------------------------------------------------

def gemm_w4a16(A: torch.Tensor, w: W4Weights, C: torch.Tensor | None = None,
               alpha: float = 1.0, beta: float = 0.0) -> torch.Tensor:
    """fp32 A [M,K], symmetric weights, fp32 C (reference semantics)."""
    M = A.shape[0]
    if C is None:
        C = zeros((M, w.N), np.float32)
    lib().call("lhq_gemm_w4a16", P(A), P(w.qweight), P(w.scales), P(C), M, w.N, w.K, w.G,
               alpha, beta, stream())
    return C


def w4a16_bf16_workspace(M: int, w: W4Weights) -> torch.Tensor | None:
    """A device workspace of the size lhq_gemm_w4a16_bf16_ws asks for (None
    when the shape runs without one)."""
    n = lib().lhq_gemm_w4a16_bf16_workspace_bytes(M, w.N, w.K, w.G)
    return empty((n,), np.uint8) if n > 0 else None


def gemm_w4a16_bf16_ws(A: torch.Tensor, w: W4Weights, ws: torch.Tensor | None,
                       C: torch.Tensor | None = None) -> torch.Tensor:
    """gemm_w4a16_bf16 with a workspace (K split across workgroups where the
    output grid is thin)."""
    M = A.shape[0]
    if C is None:
        C = empty((M, w.N), np.int16)
    nbytes = 0 if ws is None else ws.numel() * ws.element_size()
    lib().call("lhq_gemm_w4a16_bf16_ws", P(A), P(w.qweight), P(w.scales), P(w.zeros), P(C),
               M, w.N, w.K, w.G, P(ws), nbytes, stream())
    return C


def gemm_w4a16_bf16_noalloc(A: torch.Tensor, w: W4Weights, C: torch.Tensor) -> torch.Tensor:
    """gemm_w4a16_bf16_ws on the library's static scratch: allocates nothing."""
    M = A.shape[0]
    lib().call("lhq_gemm_w4a16_bf16_noalloc", P(A), P(w.qweight), P(w.scales), P(w.zeros), P(C),
               M, w.N, w.K, w.G, stream())
    return C


def gemm_w4a16_bf16(A: torch.Tensor, w: W4Weights, C: torch.Tensor | None = None) -> torch.Tensor:
    """bf16 A [M,K] (int16 bits), asymmetric weights, bf16 C [M,N] (int16 bits)."""
    M = A.shape[0]
    if C is None:
        C = empty((M, w.N), np.int16)
    lib().call("lhq_gemm_w4a16_bf16", P(A), P(w.qweight), P(w.scales), P(w.zeros), P(C),
               M, w.N, w.K, w.G, stream())
    return C


def gemm_w8a8(Aq, Bt, As, Bs, M, N, K, C=None, alpha=1.0, beta=0.0):
    if C is None:
        C = zeros((M, N), np.float32)
    lib().call("lhq_gemm_w8a8", P(Aq), P(Bt), P(As), P(Bs), P(C), M, N, K, alpha, beta, stream())
    return C


def gemm_w8a8_bf16(Aq, Bt, As, Bs, M, N, K, C=None):
    if C is None:
        C = empty((M, N), np.int16)
    lib().call("lhq_gemm_w8a8_bf16", P(Aq), P(Bt), P(As), P(Bs), P(C), M, N, K, stream())
    return C


def gemm_w8a8_i32(Aq, Bt, M, N, K, C=None):
    if C is None:
        C = empty((M, N), np.int32)
    lib().call("lhq_gemm_w8a8_i32", P(Aq), P(Bt), P(C), M, N, K, stream())
    return C
