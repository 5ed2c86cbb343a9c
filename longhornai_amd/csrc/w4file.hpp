// w4file.hpp -- the prepacked-W4 file format on the host: a safetensors file
// whose header is parsed by a strict JSON subset and checked field by field
// before any byte is trusted.  Host C++17 only (no HIP), so it also builds
// into the sanitizer checker.
//
// File = an 8-byte little-endian header length, a JSON header, then the raw
// tensors.  Tensors: "qweight" U8 [Nt*Kt*1024], "scales" F16 or F32
// [Nt*NG*16], "zeros" U32 [Nt*NG8*16] (asymmetric only).  Metadata (all
// strings, as safetensors requires): format = "lhq-w4-prepacked",
// version = "1", layout = "w4-tile16x128-v1", K, N, group_size, and
// fnv1a64 = 16 hex digits of FNV-1a (64-bit) over the data section.
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

namespace lhq {

struct W4Dims {
    int K = 0, N = 0, G = 0;
    bool asym = false;
    int64_t qbytes = 0, sbytes = 0, zbytes = 0;
};

// A whole file read into memory, parsed and checked.
struct W4File {
    std::vector<uint8_t> bytes;  // the data section
    W4Dims d;
    int64_t q_off = 0, s_off = 0, z_off = 0;
};

// Every function returns LHQ_OK, LHQ_ERR_INVALID or LHQ_ERR_UNSUPPORTED and
// on failure leaves a message in `err`.  None throws.
int w4_dims(const char* who, int K, int N, int G, int fp16_scales, W4Dims& d, std::string& err);
int w4file_read(const char* who, const char* path, W4File& f, std::string& err);
// The header (JSON padded so the data section starts 8-byte aligned) of a
// file holding `d` whose data section hashes to `checksum`.
std::string w4file_header(const W4Dims& d, uint64_t checksum);
uint64_t fnv1a64(const uint8_t* p, size_t n);

}  // namespace lhq
