// The MFMA rate the chip sustains, measured: every wave keeps four
// independent chains of v_mfma_f32_32x32x16_f16 busy on register operands (no
// memory traffic), four waves to a SIMD on every CU.  The candidate sweep's
// roofline is quoted against the published dense fp16 peak (2.5 PFLOP/s at
// 2.4 GHz); under a sustained MFMA load the chip holds a lower clock, and this
// is the rate it then delivers.  Measurement only: nothing on the search or
// build path calls it.
#include <hip/hip_runtime.h>

#include "common.h"

namespace {

typedef _Float16 pf16x8 __attribute__((ext_vector_type(8)));
typedef float pf32x16 __attribute__((ext_vector_type(16)));

__global__ __launch_bounds__(256) void mfma_probe_kernel(int iters, float* sink) {
    const int lane = threadIdx.x & 63;
    pf16x8 a, b;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        a[i] = (_Float16)(0.001f * (lane + i));
        b[i] = (_Float16)(0.002f * (lane - i));
    }
    pf32x16 c0 = {}, c1 = {}, c2 = {}, c3 = {};
    for (int it = 0; it < iters; ++it) {
        c0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c0, 0, 0, 0);
        c1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(b, a, c1, 0, 0, 0);
        c2 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, a, c2, 0, 0, 0);
        c3 = __builtin_amdgcn_mfma_f32_32x32x16_f16(b, b, c3, 0, 0, 0);
    }
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < 16; ++e) s += c0[e] + c1[e] + c2[e] + c3[e];
    if (s == 1234.5f) sink[0] = s;      // keeps the chains live; never true in practice
}

}  // namespace

extern "C" int64_t swann_mfma_probe_flop(int iters, int blocks) {
    return (int64_t)blocks * 4 * iters * 4 * (2 * 32 * 32 * 16);
}

extern "C" int swann_mfma_probe(int iters, int blocks, float* sink, void* stream) {
    swann::clear_error();
    SWANN_REQUIRE(iters >= 1 && blocks >= 1, "mfma probe: iters and blocks must be >= 1");
    SWANN_REQUIRE(sink, "mfma probe: sink is NULL");
    hipLaunchKernelGGL(mfma_probe_kernel, dim3((unsigned)blocks), dim3(256), 0,
                       (hipStream_t)stream, iters, sink);
    if (hipGetLastError() != hipSuccess) {
        swann::set_error("mfma probe: launch failed");
        return SWANN_E_LAUNCH;
    }
    return SWANN_OK;
}
