// Version, status strings and the per-thread error message of the C ABI.
#include <stdarg.h>
#include <stdio.h>

#include <hip/hip_runtime.h>

#include "crumpet_common.h"
#include "crumpet_hip.h"

namespace crumpet {

namespace {
thread_local char g_last_error[512] = "";
}

void set_last_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
}

int fail(int status, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
    return status;
}

int check_launch(const char* what) {
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) {
        return fail(CRUMPET_ERR_HIP, "%s: HIP launch failed: %s", what, hipGetErrorString(err));
    }
    return CRUMPET_OK;
}

}  // namespace crumpet

extern "C" const char* crumpet_version(void) { return "0.1.0"; }

extern "C" const char* crumpet_last_error(void) { return crumpet::g_last_error; }

extern "C" const char* crumpet_status_string(int status) {
    switch (status) {
        case CRUMPET_OK: return "CRUMPET_OK";
        case CRUMPET_ERR_INVALID_ARGUMENT: return "CRUMPET_ERR_INVALID_ARGUMENT";
        case CRUMPET_ERR_UNSUPPORTED: return "CRUMPET_ERR_UNSUPPORTED";
        case CRUMPET_ERR_HIP: return "CRUMPET_ERR_HIP";
        default: return "CRUMPET_ERR_UNKNOWN";
    }
}
