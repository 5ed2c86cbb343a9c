"""C ABI checks that need no GPU: the library loads, exports every entry point
include/longhorn_hip.h declares, and rejects bad arguments on the host with
the documented status codes before any device work is queued."""
import ctypes as C

import pytest

from longhornai_amd import capi


@pytest.fixture(scope="module")
def L():
    return capi.load()


def test_exports_every_declared_symbol(L):
    declared = capi.header_symbols()
    assert len(declared) >= 38
    missing = [s for s in declared if not hasattr(L.cdll, s)]
    assert not missing, missing
    assert set(declared) == set(capi.SIGNATURES), "ctypes table out of sync with the header"


def test_diag_library_exports_its_header_and_product_has_no_probes(L):
    """The matrix-core probes live in liblonghorn_diag.so (longhorn_diag.h),
    not in the product library, and their argument checks run on the host."""
    D = capi.load_diag()
    declared = capi.header_symbols(capi.DIAG_HEADER, "lhd_")
    assert set(declared) == set(capi.DIAG_SIGNATURES), declared
    assert not [s for s in declared if not hasattr(D.cdll, s)]
    assert not [s for s in ("lhq_probe_mfma_rate", "lhq_probe_mfma_operands") if hasattr(L.cdll, s)]
    sink = (C.c_int * 4)()
    assert D.status("lhd_probe_mfma_rate", 8, 1, 1, C.addressof(sink), None) == 1
    assert "kind" in D.last_error()
    assert D.status("lhd_probe_mfma_operands", 0, None, 1, 1, C.addressof(sink), None, None) == 1


def test_status_strings(L):
    assert L.lhq_status_string(0) == b"ok"
    assert L.lhq_status_string(capi.LHQ_ERR_UNSUPPORTED) == b"unsupported configuration"
    assert L.lhq_version() >= 100


def test_size_queries(L):
    # Nt = 28672/16 tiles x Kt = 64 tiles x 1 KiB
    assert L.lhq_w4_qweight_bytes(8192, 28672) == 1792 * 64 * 1024 == 8192 * 28672 // 2
    assert L.lhq_w4_scales_bytes(8192, 28672, 128, 1) == 1792 * 64 * 16 * 2
    assert L.lhq_w4_zeros_bytes(8192, 28672, 128) == 1792 * 8 * 16 * 4
    assert L.lhq_w4_qweight_bytes(64, 32) == 2 * 1 * 1024           # padded to 16 x 128 tiles
    assert L.lhq_b8_prepacked_bytes(4096, 14336) == 14336 * 4096
    assert L.lhq_b8_prepacked_bytes(4, 4) == 256 * 128
    assert L.lhq_w4_scales_bytes(100, 16, 3, 0) == 0               # G does not divide K


FAKE = C.c_void_p(0x1000)  # never dereferenced: validation fails first


@pytest.mark.parametrize("name,args,code", [
    ("lhq_gemm_w4a16", (None, FAKE, FAKE, FAKE, 1, 64, 128, 32, 1.0, 0.0, None), capi.LHQ_ERR_INVALID),
    ("lhq_gemm_w4a16", (FAKE, FAKE, FAKE, FAKE, 1, 64, 128, 48, 1.0, 0.0, None), capi.LHQ_ERR_INVALID),
    ("lhq_gemm_w4a16", (FAKE, FAKE, FAKE, FAKE, 1, 64, 96, 96, 1.0, 0.0, None), capi.LHQ_ERR_UNSUPPORTED),
    ("lhq_gemm_w4a16", (FAKE, FAKE, FAKE, FAKE, 1, 64, 64, 16, 1.0, 0.0, None), capi.LHQ_ERR_UNSUPPORTED),
    ("lhq_gemm_w4a16_bf16", (FAKE, FAKE, FAKE, None, FAKE, 1, 64, 128, 128, None), capi.LHQ_ERR_INVALID),
    ("lhq_gemm_w4a16_bf16", (FAKE, FAKE, FAKE, FAKE, FAKE, -1, 64, 128, 128, None), capi.LHQ_ERR_INVALID),
    ("lhq_gemm_w8a8", (FAKE, FAKE, FAKE, FAKE, FAKE, 4, 4, 4, 1.0, 0.0, None), capi.LHQ_ERR_UNSUPPORTED),
    ("lhq_gemm_w8a8", (FAKE, FAKE, None, FAKE, FAKE, 4, 4, 16, 1.0, 0.0, None), capi.LHQ_ERR_INVALID),
    ("lhq_gemm_w8a8_i32", (FAKE, FAKE, FAKE, 4, 0, 16, None), capi.LHQ_ERR_INVALID),
    ("lhq_w4_prepack_sym", (FAKE, FAKE, 63, 16, 7, FAKE, FAKE, None), capi.LHQ_ERR_INVALID),
    ("lhq_q4_quantize_groupwise", (FAKE, FAKE, FAKE, 64, 16, 48, None), capi.LHQ_ERR_INVALID),
    ("lhq_q8_quantize_per_row", (None, FAKE, FAKE, 4, 4, None), capi.LHQ_ERR_INVALID),
    ("lhq_q8_quantize_per_tensor", (FAKE, FAKE, FAKE, -5, None), capi.LHQ_ERR_INVALID),
    ("lhq_gemm_w4a16_bf16_grouped", (FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, -1, 16, 64, 128, 128, None),
     capi.LHQ_ERR_INVALID),
    ("lhq_gemm_w4a16_bf16_batched", (FAKE, FAKE, FAKE, FAKE, FAKE, 70000, 1, 64, 128, 128, None),
     capi.LHQ_ERR_INVALID),
    ("lhq_gemm_f32", (FAKE, FAKE, FAKE, -1, 4, 4, 1.0, 0.0, None), capi.LHQ_ERR_INVALID),
    # the workspace entry points check their arguments before anything is launched
    ("lhq_gemm_w4a16_ws", (None, FAKE, FAKE, FAKE, 16, 64, 128, 128, 1.0, 0.0, FAKE, 1024, None),
     capi.LHQ_ERR_INVALID),
    ("lhq_gemm_w4a16_ws", (FAKE, FAKE, FAKE, FAKE, 16, 64, 128, 128, 1.0, 0.0, FAKE, -1, None),
     capi.LHQ_ERR_INVALID),
    ("lhq_gemm_w4a16_ws", (FAKE, FAKE, FAKE, FAKE, 16, 64, 96, 96, 1.0, 0.0, FAKE, 1024, None),
     capi.LHQ_ERR_UNSUPPORTED),
    ("lhq_gemm_w4a16_bf16_grouped_ws", (FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 8, 1024, 256, 4096, 128, FAKE, -1,
                                        None), capi.LHQ_ERR_INVALID),
    ("lhq_gemm_w4a16_bf16_grouped_ws", (FAKE, None, FAKE, FAKE, FAKE, FAKE, 8, 1024, 256, 4096, 128, FAKE, 65536,
                                        None), capi.LHQ_ERR_INVALID),
    ("lhq_gemm_w4a16_bf16_grouped_swiglu_ws", (FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, -2, 1024, 256, 4096, 128, FAKE,
                                               65536, None), capi.LHQ_ERR_INVALID),
    ("lhq_moe_expert_mlp_w4a16_bf16_ws", (FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 8, 1024, 4096,
                                          14336, 128, FAKE, -1, None), capi.LHQ_ERR_INVALID),
])
def test_host_validation(L, name, args, code):
    st = L.status(name, *args)
    assert st == code, (st, L.last_error())
    assert L.last_error()


def test_workspace_queries_on_the_host(L):
    """The workspace-size queries are host functions: shapes that never split
    ask for nothing, whatever the device."""
    f32 = L.cdll.lhq_gemm_w4a16_workspace_bytes
    assert f32(1, 28672, 8192, 128) == 0       # one row
    assert f32(4096, 8192, 8192, 128) == 0     # a full grid
    assert f32(513, 8192, 1024, 128) == 0      # beyond 512 rows
    assert f32(16, 4096, 4096, 128) == 0       # 2..16 rows with K * N < 32 Mi
    assert f32(32, 8192, 8192, 64) == 0        # G < 128
    assert f32(16, 8192, 8192, 48) == 0        # a group size the GEMMs reject
    g = L.cdll.lhq_gemm_w4a16_bf16_grouped_workspace_bytes
    assert g(8, 16, 4096, 4096, 128) == 0      # two rows per group: no tile kernel
    assert g(0, 1024, 4096, 4096, 128) == 0
    assert g(8, 1024, 4096, 4096, 64) == 0     # G < 128
    assert g(8, 1024, 4096, 4096, 128) % 65536 == 0


def test_empty_problems_are_noops(L):
    # M == 0 returns OK without touching memory
    assert L.status("lhq_gemm_w4a16_bf16", None, FAKE, FAKE, FAKE, FAKE, 0, 64, 128, 128, None) == 0
    assert L.status("lhq_gemm_w8a8_i32", None, FAKE, FAKE, 0, 16, 16, None) == 0
    assert L.status("lhq_q8_quantize_per_row", FAKE, FAKE, FAKE, 0, 16, None) == 0


def test_dropin_exports_reference_interface():
    """liblonghorn_kernels.so defines every lh:: function of the reference's
    kernel headers (quant.hpp:31-94, gemm_quant.hpp:42-70, gemm.hpp:14-29),
    with the reference's parameter types."""
    import subprocess
    from longhornai_amd import KERNELS_LIB
    out = subprocess.run(["nm", "-D", "-C", "--defined-only", KERNELS_LIB], capture_output=True, text=True,
                         check=True).stdout
    want = [
        "lh::q8_quantize_per_tensor(float const*, signed char*, float*, long)",
        "lh::q8_dequantize_per_tensor(signed char const*, float, float*, long)",
        "lh::q8_quantize_per_row(float const*, signed char*, float*, int, int)",
        "lh::q8_dequantize_per_row(signed char const*, float const*, float*, int, int)",
        "lh::q8_quantize_per_col(float const*, signed char*, float*, int, int)",
        "lh::q8_dequantize_per_col(signed char const*, float const*, float*, int, int)",
        "lh::q4_quantize_groupwise(float const*, unsigned char*, float*, int, int, int)",
        "lh::q4_dequantize_groupwise(unsigned char const*, float const*, float*, int, int, int)",
        "lh::fp8_quantize_per_tensor(float const*, lh::fp8_e4m3*, float*, long)",
        "lh::fp8_dequantize_per_tensor(lh::fp8_e4m3 const*, float, float*, long)",
        "lh::fp8_quantize_per_row(float const*, lh::fp8_e4m3*, float*, int, int)",
        "lh::fp8_dequantize_per_row(lh::fp8_e4m3 const*, float const*, float*, int, int)",
        "lh::fp8_quantize_per_col(float const*, lh::fp8_e4m3*, float*, int, int)",
        "lh::fp8_dequantize_per_col(lh::fp8_e4m3 const*, float const*, float*, int, int)",
        "lh::gemm_w8a8(signed char const*, signed char const*, float const*, float const*, float*, int, int, int, float, float)",
        "lh::gemm_w4a16_groupwise(float const*, unsigned char const*, float const*, float*, int, int, int, int, float, float)",
        "lh::gemm_fp8_e4m3(lh::fp8_e4m3 const*, lh::fp8_e4m3 const*, float, float, float*, int, int, int, float, float)",
        "lh::gemm_ref(float const*, float const*, float*, int, int, int, float, float)",
        "lh::gemm(float const*, float const*, float*, int, int, int, float, float)",
        "lh::gemm_batched(float const*, float const*, float*, int, int, int, int, float, float)",
        "lh::gemm_grouped(float const* const*, float const* const*, float* const*, int const*, int const*, int const*, int, float, float)",
    ]
    missing = [w for w in want if w not in out]
    assert not missing, missing
