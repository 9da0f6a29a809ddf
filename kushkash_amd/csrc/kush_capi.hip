// C-ABI plumbing shared by every entry point: error codes and the last error message.
// The entry points themselves live next to their kernels (kush_write.hip, kush_decode.hip,
// kush_rotate.hip, kush_unpack.hip) and are declared in include/kushkash_amd.h.
#include <stdarg.h>
#include <stdio.h>

#include "kush_common.h"

namespace {
thread_local char g_err[512] = "";
}

int kush_fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

// Launches are asynchronous: this reports configuration errors (bad grid, missing code object)
// without synchronizing, so entry points stay usable under stream capture.
int kush_check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return kush_fail(-3, "%s: %s (%s)", what, hipGetErrorName(e), hipGetErrorString(e));
    return 0;
}

extern "C" const char* kush_last_error(void) { return g_err; }

// Bumped when an entry point's signature or meaning changes.
extern "C" int kush_abi_version(void) { return 8; }
