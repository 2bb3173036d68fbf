// Host-only parts of the C ABI: error state, version, device query.
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>

#include "common.h"

namespace swann {

static thread_local char g_err[1024] = "";

void set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
}

void clear_error() { g_err[0] = '\0'; }

}  // namespace swann

extern "C" {

const char* swann_last_error(void) { return swann::g_err; }

const char* swann_version(void) { return "swann_amd 0.1.0 gfx950"; }

int swann_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    return n;
}

}  // extern "C"
