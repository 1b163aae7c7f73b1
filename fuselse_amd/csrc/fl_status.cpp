// Error reporting for the C ABI: every entry point returns an int status and
// leaves a human-readable message for the calling thread.
#include "fl_status.hpp"

#include <stdarg.h>
#include <stdio.h>

#include "../../include/fuselse_amd.h"

namespace {
thread_local char g_msg[512] = "";
}

namespace fl {

int set_error(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_msg, sizeof(g_msg), fmt, ap);
    va_end(ap);
    return code;
}

int ok() {
    g_msg[0] = '\0';
    return FL_OK;
}

int launch_status(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(FL_ELAUNCH, "%s: kernel launch failed: %s", what, hipGetErrorString(e));
    return ok();
}

}  // namespace fl

extern "C" const char* fl_last_error(void) { return g_msg; }

extern "C" int fl_abi_version(void) { return FL_ABI_VERSION; }
