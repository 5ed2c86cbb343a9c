"""On-device check of the bf16 conversion instruction the kernels use.

The GEMM and quantizer kernels round fp32 to bf16 with gfx950's
v_cvt_pk_bf16_f32.  The reference's rule (dtypes.hpp:87-98) is round to
nearest even, NaN -> payload kept with the quiet bit set; this test runs the
instruction over all 2^32 fp32 bit patterns and requires it to agree with the
rule on every one (NaNs, infinities, denormals and ties included).
"""
import pytest

pytestmark = pytest.mark.gpu


def test_bf16_convert_matches_reference_rule_exhaustively(lib):
    import torch
    from longhornai_amd import ops
    counts = torch.zeros(2, dtype=torch.int64, device="cuda")
    lib.call("lhq_selftest_bf16", counts.data_ptr(), ops.stream())
    torch.cuda.synchronize()
    non_nan, nan = counts.cpu().tolist()
    assert non_nan == 0 and nan == 0, f"mismatches: {non_nan} non-NaN, {nan} NaN"


def test_mfma_rate_probe_runs_and_rejects_bad_arguments(lib):
    """The matrix-core rate probe (bench.py's ceiling leg): a small launch of
    each kind completes and writes one value per workgroup; an unknown kind
    is refused before any launch."""
    import torch
    from longhornai_amd import ops
    sink = torch.full((16,), -1, dtype=torch.int32, device="cuda")
    for kind in range(8):
        lib.call("lhq_probe_mfma_rate", kind, 16, 8, sink.data_ptr(), ops.stream())
    torch.cuda.synchronize()
    assert lib.status("lhq_probe_mfma_rate", 8, 16, 8, sink.data_ptr(), ops.stream()) != 0
