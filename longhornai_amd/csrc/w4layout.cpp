// w4layout.cpp -- byte counts of the prepacked W4 layout (w4layout.hpp).
// Host code only: it is also compiled into the sanitizer build of the file
// reader, which has no GPU code.
#include "w4layout.hpp"

#include <cstdint>

#include "longhorn_hip.h"

namespace {

// ceil(a / b) * c * d for non-negative ints, or 0 where the product would
// not fit in int64 (no layout that large can be allocated anyway).
int64_t blocks(int64_t a_ceil, int64_t b, int64_t c) {
    const unsigned __int128 v = static_cast<unsigned __int128>(a_ceil) * b * c;
    return v > static_cast<unsigned __int128>(INT64_MAX) ? 0 : static_cast<int64_t>(v);
}

int64_t ceil_div64(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace

extern "C" {

int64_t lhq_w4_qweight_bytes(int K, int N) {
    if (K <= 0 || N <= 0) return 0;
    return blocks(ceil_div64(N, lhq::kW4TileN), ceil_div64(K, lhq::kW4TileK), lhq::kW4TileBytes);
}

int64_t lhq_w4_scales_bytes(int K, int N, int G, int fp16_scales) {
    if (!lhq::w4_dims_ok(K, N, G)) return 0;
    return blocks(ceil_div64(N, lhq::kW4TileN), K / G, lhq::kW4TileN * (fp16_scales ? 2 : 4));
}

int64_t lhq_w4_zeros_bytes(int K, int N, int G) {
    if (!lhq::w4_dims_ok(K, N, G)) return 0;
    return blocks(ceil_div64(N, lhq::kW4TileN), ceil_div64(K / G, 8), lhq::kW4TileN * 4);
}

}  // extern "C"
