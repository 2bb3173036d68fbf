// Sign codes for the search's pre-filter.
//
// The reference consumes them (swann/csrc/local_search.cu:205-243: bit b of
// word w stands for dimension 32w + b, set meaning +1 around the corpus mean;
// alpha scales the code back to the corpus's units) and loads them from
// codes_<name>.npy / alpha_<name>.npy / mu_<name>.npy (swann/_engine.py:320-337),
// but does not ship the builder.  This one follows the consumer's estimator:
//   mu[t]    = mean over rows of x[r, t]       (double sums, rounded to fp32)
//   bit      = x[r, t] - mu[t] > 0             (fp32 difference)
//   alpha[r] = sum_t |x[r, t] - mu[t]| / dim   (double sum, rounded to fp32)
//
// Two HBM passes over X: column sums (row chunks in parallel, partials in a
// workspace, folded in chunk order so the mean does not depend on timing),
// then one wave per row writing its words and alpha.  Both are bandwidth
// bound; at 1M x 1536 fp16 that is 2 x 3.1 GB.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "common.h"

namespace swann {
namespace {

constexpr int kColBlock = 256;
constexpr int kChunks = 256;

template <typename XT>
__device__ __forceinline__ float ldx(const XT* p) { return (float)*p; }

template <typename XT>
__global__ __launch_bounds__(kColBlock) void col_partial(const XT* __restrict__ X, int64_t n,
                                                         int dim, int64_t rows_per,
                                                         double* __restrict__ part) {
    const int c = blockIdx.x * kColBlock + threadIdx.x;
    const int chunk = blockIdx.y;
    if (c >= dim) return;
    const int64_t r0 = (int64_t)chunk * rows_per;
    int64_t r1 = r0 + rows_per;
    if (r1 > n) r1 = n;
    double s = 0.0;
    for (int64_t r = r0; r < r1; ++r) s += (double)ldx(X + r * dim + c);
    part[(int64_t)chunk * dim + c] = s;
}

__global__ __launch_bounds__(kColBlock) void col_final(const double* __restrict__ part,
                                                       int nchunk, int dim, int64_t n,
                                                       float* __restrict__ mu) {
    const int c = blockIdx.x * kColBlock + threadIdx.x;
    if (c >= dim) return;
    double s = 0.0;
    for (int k = 0; k < nchunk; ++k) s += part[(int64_t)k * dim + c];
    mu[c] = (float)(s / (double)n);
}

// One wave per row; lane l owns words l, l + 64, ...
template <typename XT>
__global__ __launch_bounds__(256) void code_rows(const XT* __restrict__ X, int64_t n, int dim,
                                                 int cwords, const float* __restrict__ mu,
                                                 int32_t* __restrict__ codes,
                                                 float* __restrict__ alpha) {
    const int lane = threadIdx.x & 63;
    const int64_t r = (int64_t)xcd_remap(blockIdx.x, gridDim.x) * 4 + (threadIdx.x >> 6);
    if (r >= n) return;
    const XT* x = X + r * dim;
    double l1 = 0.0;
    for (int w = lane; w < cwords; w += 64) {
        unsigned bits = 0u;
        const int t0 = w * 32;
        for (int b = 0; b < 32; ++b) {
            const int t = t0 + b;
            if (t >= dim) break;
            const float df = ldx(x + t) - mu[t];
            if (df > 0.f) bits |= (1u << b);
            l1 += (double)fabsf(df);
        }
        codes[r * cwords + w] = (int32_t)bits;
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) l1 += __shfl_down(l1, off, 64);
    if (lane == 0) alpha[r] = (float)(l1 / (double)dim);
}

int nchunks_for(int64_t n) { return n < kChunks ? (int)n : kChunks; }

}  // namespace
}  // namespace swann

using namespace swann;

extern "C" {

int64_t swann_codes_workspace_size(int64_t n, int dim) {
    if (n <= 0 || dim <= 0) return 0;
    return (int64_t)nchunks_for(n) * dim * (int64_t)sizeof(double);
}

int swann_build_codes(const void* X, int x_dtype, int64_t n, int dim, const float* mu_in,
                      int32_t* codes, float* alpha, float* mu_out, void* workspace,
                      void* stream) {
    clear_error();
    SWANN_REQUIRE(n > 0 && dim > 0, "X must be a non-empty [n, dim] matrix");
    SWANN_REQUIRE(x_dtype == SWANN_DTYPE_F32 || x_dtype == SWANN_DTYPE_F16,
                  "X: float32 or float16");
    SWANN_REQUIRE(X && codes && alpha && mu_out, "build_codes: a required pointer is NULL");
    SWANN_REQUIRE(mu_in || workspace, "build_codes: computing the mean needs the workspace");
    hipStream_t st = (hipStream_t)stream;
    const int cwords = (dim + 31) / 32;
    const unsigned cblocks = (unsigned)((dim + kColBlock - 1) / kColBlock);
    if (mu_in) {
        if (mu_in != mu_out) {
            const hipError_t e = hipMemcpyAsync(mu_out, mu_in, sizeof(float) * (size_t)dim,
                                                hipMemcpyDeviceToDevice, st);
            if (e != hipSuccess) return launch_status("build_codes (copy mu)");
        }
    } else {
        const int nchunk = nchunks_for(n);
        const int64_t rows_per = (n + nchunk - 1) / nchunk;
        double* part = static_cast<double*>(workspace);
        if (x_dtype == SWANN_DTYPE_F32)
            col_partial<float><<<dim3(cblocks, nchunk), kColBlock, 0, st>>>(
                static_cast<const float*>(X), n, dim, rows_per, part);
        else
            col_partial<_Float16><<<dim3(cblocks, nchunk), kColBlock, 0, st>>>(
                static_cast<const _Float16*>(X), n, dim, rows_per, part);
        col_final<<<cblocks, kColBlock, 0, st>>>(part, nchunk, dim, n, mu_out);
    }
    const int64_t nb = (n + 3) / 4;
    SWANN_REQUIRE(nb <= (int64_t)INT32_MAX, "too many rows for one launch");
    if (x_dtype == SWANN_DTYPE_F32)
        code_rows<float><<<(unsigned)nb, 256, 0, st>>>(static_cast<const float*>(X), n, dim,
                                                       cwords, mu_out, codes, alpha);
    else
        code_rows<_Float16><<<(unsigned)nb, 256, 0, st>>>(static_cast<const _Float16*>(X), n,
                                                          dim, cwords, mu_out, codes, alpha);
    return launch_status("build_codes");
}

}  // extern "C"
