"""On-device check of the bf16 conversion instruction the kernels use.

The GEMM and quantizer kernels round fp32 to bf16 with gfx950's
v_cvt_pk_bf16_f32.  The reference's rule (dtypes.hpp:87-98) is round to
nearest even, NaN -> payload kept with the quiet bit set; this test runs the
instruction over all 2^32 fp32 bit patterns and requires it to agree with the
rule on every one (NaNs, infinities, denormals and ties included).
"""
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def diag(lib):
    """The diagnostics library (include/longhorn_diag.h) holding the probes."""
    from longhornai_amd import capi
    return capi.load_diag()


def test_bf16_convert_matches_reference_rule_exhaustively(lib):
    import torch
    from longhornai_amd import ops
    counts = torch.zeros(2, dtype=torch.int64, device="cuda")
    lib.call("lhq_selftest_bf16", counts.data_ptr(), ops.stream())
    torch.cuda.synchronize()
    non_nan, nan = counts.cpu().tolist()
    assert non_nan == 0 and nan == 0, f"mismatches: {non_nan} non-NaN, {nan} NaN"


def test_mfma_rate_probe_runs_and_rejects_bad_arguments(diag):
    """The matrix-core rate probe of the diagnostics library (bench.py's
    ceiling leg): a small launch of
    each kind completes and writes one value per workgroup; an unknown kind
    is refused before any launch."""
    import torch
    from longhornai_amd import ops
    sink = torch.full((16,), -1, dtype=torch.int32, device="cuda")
    for kind in range(8):
        diag.call("lhd_probe_mfma_rate", kind, 16, 8, sink.data_ptr(), ops.stream())
    torch.cuda.synchronize()
    assert diag.status("lhd_probe_mfma_rate", 8, 16, 8, sink.data_ptr(), ops.stream()) != 0


def test_mfma_operand_probe_runs_and_rejects_bad_arguments(diag):
    """The matrix-core rate probe on operands from memory (bench.py's
    same-operands figures): every kind completes and writes one value per
    workgroup and two clock counts; the int8 kind's accumulators grow
    linearly in the round count (integer MFMAs are exact) and the k-chain
    kinds reach the same integer sums; an unknown kind
    and a null operand buffer are refused before any launch."""
    import torch
    from longhornai_amd import ops
    gen = torch.Generator(device="cuda")
    gen.manual_seed(5)
    src = torch.randint(0, 256, (32768,), dtype=torch.uint8, device="cuda", generator=gen)
    sink = torch.full((16,), -1, dtype=torch.int32, device="cuda")
    clocks = torch.zeros(32, dtype=torch.int64, device="cuda")
    for kind in range(8):
        diag.call("lhd_probe_mfma_operands", kind, src.data_ptr(), 16, 4, sink.data_ptr(), clocks.data_ptr(),
                 ops.stream())
        torch.cuda.synchronize()
        c = clocks.view(16, 2).cpu()
        assert bool((c[:, 1] > 0).all()) and bool((c[:, 0] > c[:, 1]).all()), c
    sums = []
    for iters in (1, 3):
        diag.call("lhd_probe_mfma_operands", 0, src.data_ptr(), 16, iters, sink.data_ptr(), 0, ops.stream())
        torch.cuda.synchronize()
        sums.append(sink.cpu().tolist())
    assert len(set(sums[0])) == 1 and sums[0][0] != 0
    assert all((3 * a - b) % 2**32 == 0 for a, b in zip(sums[0], sums[1]))
    # the k-chain kinds issue the same products per round (kind 3) or twice
    # them (kind 4): integer sums equal to kind 0's, or double
    for kind, mult in ((3, 1), (4, 2)):
        diag.call("lhd_probe_mfma_operands", kind, src.data_ptr(), 16, 3, sink.data_ptr(), 0, ops.stream())
        torch.cuda.synchronize()
        assert all((mult * b - c) % 2**32 == 0 for b, c in zip(sums[1], sink.cpu().tolist())), kind
    assert diag.status("lhd_probe_mfma_operands", 8, src.data_ptr(), 16, 4, sink.data_ptr(), 0, ops.stream()) != 0
    assert diag.status("lhd_probe_mfma_operands", 0, 0, 16, 4, sink.data_ptr(), 0, ops.stream()) != 0
