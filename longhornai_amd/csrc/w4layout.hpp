// w4layout.hpp -- geometry of the prepacked W4 weight layout, shared by the
// device code (common.hpp) and the host-only file reader (w4file.cpp).
//
//   qweight  [Nt][Kt][64 lanes][16 B], Nt = ceil(N/16), Kt = ceil(K/128)
//   scales   [Nt][NG][16]  fp32 (symmetric) or fp16 (asymmetric), NG = K/G
//   zeros    [Nt][ceil(NG/8)][16] u32, group g in nibble g % 8 (asymmetric)
// The byte counts are lhq_w4_qweight_bytes / _scales_bytes / _zeros_bytes
// (include/longhorn_hip.h), defined in w4layout.cpp.
#pragma once

namespace lhq {

constexpr int kW4TileN = 16;
constexpr int kW4TileK = 128;
constexpr int kW4TileBytes = 1024;

// The shapes every W4 entry point accepts: K, N, G > 0, K even, G | K
// (the reference's preconditions, quant.hpp:52-59).
inline bool w4_dims_ok(int K, int N, int G) {
    return K > 0 && N > 0 && G > 0 && (K % G) == 0 && (K % 2) == 0;
}

}  // namespace lhq
