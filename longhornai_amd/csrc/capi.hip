// capi.hip -- status codes and error messages of the C ABI.
//
// The reference's kernels return void and never report errors
// (gemm_quant.hpp:42-70, quant.hpp:31-94).  The device backend must: every
// entry point validates its arguments on the host before any launch and
// returns an LHQ_* status, with a per-thread message for the last failure.
#include <cstdarg>
#include <cstdio>

#include "common.hpp"

namespace lhq {

namespace {
thread_local char g_last_error[512] = "";
}

int set_error(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
    return code;
}

// Launch errors (bad configuration, missing code object) surface through
// hipGetLastError immediately after the launch.
int check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return set_error(LHQ_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
    return LHQ_OK;
}

}  // namespace lhq

extern "C" {

const char* lhq_status_string(int status) {
    switch (status) {
        case LHQ_OK: return "ok";
        case LHQ_ERR_INVALID: return "invalid argument";
        case LHQ_ERR_UNSUPPORTED: return "unsupported configuration";
        case LHQ_ERR_HIP: return "HIP runtime error";
        default: return "unknown status";
    }
}

const char* lhq_last_error(void) { return lhq::g_last_error; }

int lhq_version(void) { return 100; /* 0.1.0 */ }

}  // extern "C"
