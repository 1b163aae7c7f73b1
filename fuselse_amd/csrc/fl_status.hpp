// Status codes and the per-thread error message behind the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define FL_OK 0
#define FL_EINVAL 1
#define FL_ELAUNCH 2
#define FL_ERANGE 3

namespace fl {

// Records a message for fl_last_error() and returns code.
int set_error(int code, const char* fmt, ...);
// Clears the message and returns FL_OK.
int ok();
// Maps the launch status of the kernels just enqueued to a return code.
int launch_status(const char* what);

}  // namespace fl

#define FL_CHECK(cond, ...)                                  \
    do {                                                     \
        if (!(cond)) return fl::set_error(FL_EINVAL, __VA_ARGS__); \
    } while (0)
