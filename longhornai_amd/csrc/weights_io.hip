// weights_io.hip -- prepacked W4 weights on disk: the C ABI of the versioned
// safetensors file (host code; the format and its checks are in w4file.cpp).
//
// The reference stores nothing: its int4 weights live in caller memory as
// [K/2, N] bytes plus fp32 scales (quant.hpp:52-59), and its plan lists
// safetensors loaders for later (PLAN.md:326-333).  The GPU layout
// (include/longhorn_hip.h, "prepacked weight layouts") costs a prepack pass
// per matrix; this file keeps the prepacked form so a model loads straight
// into it.
#include <cerrno>
#include <cstdio>
#include <cstring>
#include <memory>
#include <new>
#include <string>
#include <vector>

#include "common.hpp"
#include "w4file.hpp"

using namespace lhq;

extern "C" {

int lhq_w4_save(const char* path, const uint8_t* qweight, const void* scales, const uint32_t* zeros, int K, int N,
                int G, int fp16_scales, void* stream) {
    W4Dims d{};
    std::string err;
    if (int st = w4_dims("w4_save", K, N, G, fp16_scales, d, err)) return set_error(st, "%s", err.c_str());
    LHQ_REQUIRE(path && qweight && scales && (zeros || !d.asym), "w4_save: null pointer");
    try {
        std::vector<uint8_t> data(static_cast<size_t>(d.qbytes + d.sbytes + d.zbytes));
        hipStream_t s = as_stream(stream);
        hipError_t e = hipMemcpyAsync(data.data(), qweight, d.qbytes, hipMemcpyDeviceToHost, s);
        if (e == hipSuccess) e = hipMemcpyAsync(data.data() + d.qbytes, scales, d.sbytes, hipMemcpyDeviceToHost, s);
        if (e == hipSuccess && d.asym)
            e = hipMemcpyAsync(data.data() + d.qbytes + d.sbytes, zeros, d.zbytes, hipMemcpyDeviceToHost, s);
        if (e == hipSuccess) e = hipStreamSynchronize(s);
        if (e != hipSuccess) return set_error(LHQ_ERR_HIP, "w4_save: copy to host: %s", hipGetErrorString(e));
        const std::string h = w4file_header(d, fnv1a64(data.data(), data.size()));
        uint8_t len8[8];
        for (int i = 0; i < 8; ++i) len8[i] = static_cast<uint8_t>(static_cast<uint64_t>(h.size()) >> (8 * i));
        std::unique_ptr<FILE, int (*)(FILE*)> fp(std::fopen(path, "wb"), &std::fclose);
        LHQ_REQUIRE(fp, "w4_save: cannot create %s: %s", path, std::strerror(errno));
        const bool ok = std::fwrite(len8, 1, 8, fp.get()) == 8 &&
                        std::fwrite(h.data(), 1, h.size(), fp.get()) == h.size() &&
                        std::fwrite(data.data(), 1, data.size(), fp.get()) == data.size();
        const int closed = std::fclose(fp.release());
        LHQ_REQUIRE(ok && closed == 0, "w4_save: writing %s failed", path);
    } catch (const std::bad_alloc&) {
        return set_error(LHQ_ERR_INVALID, "w4_save: out of host memory for %lld bytes",
                         static_cast<long long>(d.qbytes + d.sbytes + d.zbytes));
    }
    return LHQ_OK;
}

int lhq_w4_file_info(const char* path, int* K, int* N, int* group_size, int* fp16_scales) {
    W4File f;
    std::string err;
    if (int st = w4file_read("w4_file_info", path, f, err)) return set_error(st, "%s", err.c_str());
    if (K) *K = f.d.K;
    if (N) *N = f.d.N;
    if (group_size) *group_size = f.d.G;
    if (fp16_scales) *fp16_scales = f.d.asym ? 1 : 0;
    return LHQ_OK;
}

int lhq_w4_load(const char* path, uint8_t* qweight, void* scales, uint32_t* zeros, int K, int N, int G,
                int fp16_scales, void* stream) {
    W4File f;
    std::string err;
    if (int st = w4file_read("w4_load", path, f, err)) return set_error(st, "%s", err.c_str());
    LHQ_REQUIRE(f.d.K == K && f.d.N == N && f.d.G == G && f.d.asym == (fp16_scales != 0),
                "w4_load: %s holds K=%d N=%d G=%d %s, the caller asked for K=%d N=%d G=%d %s", path, f.d.K, f.d.N,
                f.d.G, f.d.asym ? "asymmetric" : "symmetric", K, N, G, fp16_scales ? "asymmetric" : "symmetric");
    LHQ_REQUIRE(qweight && scales && (zeros || !f.d.asym), "w4_load: null pointer");
    hipStream_t s = as_stream(stream);
    hipError_t e = hipMemcpyAsync(qweight, f.bytes.data() + f.q_off, f.d.qbytes, hipMemcpyHostToDevice, s);
    if (e == hipSuccess) e = hipMemcpyAsync(scales, f.bytes.data() + f.s_off, f.d.sbytes, hipMemcpyHostToDevice, s);
    if (e == hipSuccess && f.d.asym)
        e = hipMemcpyAsync(zeros, f.bytes.data() + f.z_off, f.d.zbytes, hipMemcpyHostToDevice, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);  // the host copy is freed on return
    if (e != hipSuccess) return set_error(LHQ_ERR_HIP, "w4_load: copy to device: %s", hipGetErrorString(e));
    return LHQ_OK;
}

}  // extern "C"
