// kernels/device.hpp -- host-side plumbing of the lh:: drop-in library:
// device buffers and status checks around the C ABI (include/longhorn_hip.h).
// Internal to the drop-in; not part of the reference's interface.
#ifndef LONGHORN_MI355X_KERNELS_DEVICE_HPP
#define LONGHORN_MI355X_KERNELS_DEVICE_HPP

#include <cstddef>
#include <cstdint>

namespace lh {
namespace dev {

// Abort with `what` and the detail text (the reference functions return
// void, so a failure cannot be reported to the caller).
[[noreturn]] void fail(const char* what, const char* detail);
// A C-ABI status: LHQ_OK or abort with the library's last error message.
void check(int status, const char* what);

// A device allocation of `bytes` bytes, freed on destruction; zero bytes
// allocates nothing.
class Buffer {
public:
    explicit Buffer(size_t bytes);
    ~Buffer();
    Buffer(const Buffer&) = delete;
    Buffer& operator=(const Buffer&) = delete;
    void* get() const { return ptr_; }
    template <typename T> T* as() const { return static_cast<T*>(ptr_); }
    size_t bytes() const { return bytes_; }
    void upload(const void* host, size_t bytes);    // host -> device
    void download(void* host, size_t bytes) const;  // device -> host
    void zero();

private:
    void* ptr_ = nullptr;
    size_t bytes_ = 0;
};

// Copy `rows` rows of `row_bytes` bytes from host (pitch `row_bytes`) into
// the device buffer at pitch `pitch` (>= row_bytes).
void upload_pitched(Buffer& dst, size_t pitch, const void* host, size_t row_bytes, size_t rows);

// The stream every drop-in call runs on (the null stream) and a full wait.
void* stream();
void sync(const char* what);

}  // namespace dev
}  // namespace lh

#endif  // LONGHORN_MI355X_KERNELS_DEVICE_HPP
