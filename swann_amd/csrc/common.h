// Internal helpers shared by the HIP translation units of libswann_amd.
#pragma once

#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdlib.h>
#include <stdio.h>

#include "swann_amd.h"

namespace swann {

// Thread-local message of the last failed call (swann_last_error).
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
void clear_error();

// MI355X dispatches workgroup b to XCD (b % 8).  Give each XCD one contiguous
// range of logical ids instead, so the J branches of a query -- which share
// the query's distance table, claims and bound -- run under one L2.
constexpr int kNumXcd = 8;

__device__ __forceinline__ int64_t xcd_remap(int64_t b, int64_t nblocks) {
    if (nblocks < kNumXcd) return b;
    const int64_t per = nblocks / kNumXcd, extra = nblocks % kNumXcd;
    const int64_t x = b % kNumXcd, k = b / kNumXcd;
    return x * per + (x < extra ? x : extra) + k;
}

// Launch-error check after a kernel launch.
inline int launch_status(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error("%s: launch failed: %s", what, hipGetErrorString(e));
        return SWANN_E_LAUNCH;
    }
    return SWANN_OK;
}

inline bool is_pow2(int64_t x) { return x > 0 && (x & (x - 1)) == 0; }

// A test hook: true when the environment variable is set to a non-zero value
// (used to run an alternative code path on the same inputs).
inline bool getenv_flag(const char* name) {
    const char* e = getenv(name);
    return e && *e && *e != '0';
}

inline int pow2_at_least(int x, int lo, int cap) {
    int n = lo;
    while (n < x && n < cap) n <<= 1;
    return n;
}

}  // namespace swann

#define SWANN_REQUIRE(cond, ...)              \
    do {                                      \
        if (!(cond)) {                        \
            ::swann::set_error(__VA_ARGS__);  \
            return SWANN_E_INVALID;           \
        }                                     \
    } while (0)
