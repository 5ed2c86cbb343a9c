// device.cpp -- device buffers and status checks of the lh:: drop-in.
#include "kernels/device.hpp"

#include <hip/hip_runtime_api.h>

#include <cstdio>
#include <cstdlib>

#include "longhorn_hip.h"

namespace lh {
namespace dev {

void fail(const char* what, const char* detail) {
    std::fprintf(stderr, "longhorn (MI355X backend): %s failed: %s\n", what, detail ? detail : "");
    std::fflush(stderr);
    std::abort();
}

void check(int status, const char* what) {
    if (status != LHQ_OK) fail(what, lhq_last_error());
}

static void check_hip(hipError_t e, const char* what) {
    if (e != hipSuccess) fail(what, hipGetErrorString(e));
}

Buffer::Buffer(size_t bytes) : bytes_(bytes) {
    if (bytes_ > 0) check_hip(hipMalloc(&ptr_, bytes_), "hipMalloc");
}

Buffer::~Buffer() {
    if (ptr_) (void)hipFree(ptr_);
}

void Buffer::upload(const void* host, size_t bytes) {
    if (bytes > bytes_) fail("upload", "source larger than the device buffer");
    if (bytes) check_hip(hipMemcpy(ptr_, host, bytes, hipMemcpyHostToDevice), "hipMemcpy H2D");
}

void Buffer::download(void* host, size_t bytes) const {
    if (bytes > bytes_) fail("download", "destination larger than the device buffer");
    if (bytes) check_hip(hipMemcpy(host, ptr_, bytes, hipMemcpyDeviceToHost), "hipMemcpy D2H");
}

void Buffer::zero() {
    if (bytes_) check_hip(hipMemset(ptr_, 0, bytes_), "hipMemset");
}

void upload_pitched(Buffer& dst, size_t pitch, const void* host, size_t row_bytes, size_t rows) {
    if (rows == 0 || row_bytes == 0) return;
    if (pitch < row_bytes || pitch * rows > dst.bytes()) fail("upload_pitched", "pitch too small");
    check_hip(hipMemcpy2D(dst.get(), pitch, host, row_bytes, row_bytes, rows, hipMemcpyHostToDevice),
              "hipMemcpy2D H2D");
}

void* stream() { return nullptr; }

void sync(const char* what) { check_hip(hipDeviceSynchronize(), what); }

}  // namespace dev
}  // namespace lh
