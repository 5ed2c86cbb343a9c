"""longhornai_amd -- MI355X (gfx950) backend of LonghornAI's quantized-GEMM path.

* ``csrc/``  hand-written HIP kernels and the C ABI (``include/longhorn_hip.h``),
  built into ``lib/liblonghorn_hip.so``.
* ``cpp/``   the ``lh::`` drop-in headers (``kernels/gemm_quant.hpp``,
  ``kernels/quant.hpp``, ``kernels/gemm.hpp``, ``kernels/dtypes.hpp``) with the
  reference's signatures, built into ``lib/liblonghorn_kernels.so``.
* ``capi``   ctypes binding of the C ABI; ``ops`` torch-tensor helpers (tests
  and bench plumbing).
"""
import os

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_DIR = os.path.join(PKG_DIR, "lib")
HIP_LIB = os.path.join(LIB_DIR, "liblonghorn_hip.so")
KERNELS_LIB = os.path.join(LIB_DIR, "liblonghorn_kernels.so")
