// selftest.hip -- on-device check of the conversion instruction the kernels
// rely on (library diagnostics, not part of the reference interface).  The
// matrix-core rate probes live in the separate diagnostics library
// (diag/mfma_probe.hip).
#include <type_traits>

#include "common.hpp"

namespace lhq {
namespace {

// Thread t converts inputs base + 2t and base + 2t + 1 with
// v_cvt_pk_bf16_f32 (pack_bf16x2) and compares each with the reference rule
// (bf16_rule).  counts[0] / counts[1]: mismatches on non-NaN / NaN inputs.
__global__ __launch_bounds__(256) void bf16_selftest_kernel(uint32_t base, unsigned long long* counts) {
    const uint32_t t = blockIdx.x * 256u + threadIdx.x;
    const uint32_t x0 = base + 2u * t, x1 = x0 + 1u;
    const uint32_t hw = pack_bf16x2(__uint_as_float(x0), __uint_as_float(x1));
    const bool bad0 = (hw & 0xffffu) != bf16_rule(x0);
    const bool bad1 = (hw >> 16) != bf16_rule(x1);
    if (bad0) atomicAdd(&counts[(x0 & 0x7fffffffu) > 0x7f800000u ? 1 : 0], 1ull);
    if (bad1) atomicAdd(&counts[(x1 & 0x7fffffffu) > 0x7f800000u ? 1 : 0], 1ull);
}

}  // namespace
}  // namespace lhq

using namespace lhq;

extern "C" int lhq_selftest_bf16(unsigned long long* counts, void* stream) {
    LHQ_REQUIRE(counts, "selftest_bf16: null pointer");
    hipStream_t s = as_stream(stream);
    if (hipMemsetAsync(counts, 0, 2 * sizeof(unsigned long long), s) != hipSuccess)
        return set_error(LHQ_ERR_HIP, "selftest_bf16: memset failed");
    constexpr uint32_t kPer = 1u << 28;  // inputs per launch
    for (uint64_t b = 0; b < (uint64_t{1} << 32); b += kPer) {
        bf16_selftest_kernel<<<kPer / 2 / 256, 256, 0, s>>>(static_cast<uint32_t>(b), counts);
        const int st = check_launch("selftest_bf16");
        if (st != LHQ_OK) return st;
    }
    return LHQ_OK;
}
