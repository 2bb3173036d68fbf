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

// Switches that select an alternative code path of the same computation,
// for tests that run every path on the same inputs and for diagnosis; set
// through swann_set_option (include/swann_amd.h, which lists each one and
// its values).  Every one defaults to the production path; the library reads
// no environment variable.
enum Option {
    kOptSearchBlock,     // advance workgroup size: 0 chosen per batch, or 64 | 256 | 1024
    kOptPruneSimt,       // 1: the prune's Gram on fp32 SIMT instead of MFMA
    kOptPruneF32,        // 1: fp32 rows' prune Gram on fp32 MFMA instead of split fp16 planes
    kOptSweepSym,        // -1 by size, 0 one-sided, 1 symmetric (from 2 row panels)
    kOptSweepWaves,      // 16 or 8 waves a direct-load sweep workgroup
    kOptSweepRowscale,   // 1: an fp32 corpus's screen plane always row-scaled
    kOptSweepRegstage,   // 1: the register-staged sweep instead of direct loads
    kOptSweepSymFcap,    // 0, or the room of a row's second list (forces its overflow)
    kOptSweepNoseed,     // 1: the symmetric sweep without locality order and seeds
    kOptSweepOrder,      // 1: the seeded sweep on the locality-ordered copy; 0: in row order
    kOptSweepRepairMax,  // overflowed panels repaired one at a time (more: all at once)
    kOptCount
};
int option(Option o);
inline bool option_on(Option o) { return option(o) != 0; }

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
