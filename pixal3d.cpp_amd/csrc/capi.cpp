// Error reporting and version for the pxs C ABI.

#include "pxs_common.h"

#include <string>

namespace pxs {
namespace {
thread_local std::string g_last_error;
} // namespace

void set_error(const std::string & message) { g_last_error = message; }

int fail(int code, const std::string & message) noexcept {
    try {
        g_last_error = message;
    } catch (...) {
        g_last_error.clear();  // out of host memory: the code alone reports it
    }
    return code;
}

int fail_workspace(const char * what) noexcept {
    try {
        return fail(PXS_ERR_ARG, std::string(what) + ": workspace must be 256-byte aligned");
    } catch (...) {
        return fail(PXS_ERR_ARG, std::string());
    }
}

int check_hip(hipError_t status, const char * what) {
    if (status == hipSuccess) return PXS_OK;
    return fail(PXS_ERR_HIP, std::string(what) + ": " + hipGetErrorString(status));
}

int check_launch(const char * what) { return check_hip(hipGetLastError(), what); }

} // namespace pxs

extern "C" {

const char * pxs_last_error(void) { return pxs::g_last_error.c_str(); }

int pxs_version(void) { return 1; }

} // extern "C"
