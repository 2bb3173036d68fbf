// Seed selection: the E nearest catalogue rows per query (swann/_select.py:93-128).
//
// Two kernels: a tiled fp32 distance GEMM that writes the distance matrix
// D[q, p] (1 - <q,v> for IP; |v|^2 - 2<q,v> + |q|^2 for L2, the reference's
// formulas) into a caller-owned workspace, and a per-row top-E that sorts
// (distance, index) pairs in LDS and keeps the E smallest, ascending.  The
// reference folds slices of 8192 columns into a running best; the result is
// the exact top-E either way.
#include <float.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "common.h"

namespace swann {
namespace {

constexpr int kTM = 64, kTN = 64, kTK = 16;   // GEMM tile
constexpr int kTopBuf = 4096;                 // pairs held in LDS by the top-E kernel
constexpr int kTopBlock = 256;

__device__ __forceinline__ bool lt(float da, int ia, float db, int ib) {
    return (da < db) || (da == db && ia < ib);
}

// Squared norms of rows (only the L2 metric needs them).
__global__ __launch_bounds__(256) void row_norms(const float* __restrict__ A, int64_t n, int dim,
                                                 float* __restrict__ out) {
    const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (r >= n) return;
    const float* a = A + r * dim;
    float s = 0.f;
    for (int t = lane; t < dim; t += 64) s = __builtin_fmaf(a[t], a[t], s);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
    if (lane == 0) out[r] = s;
}

// D[m, n] = f(<A_m, B_n>) for A [M, dim], B [N, dim], both row-major.
__global__ __launch_bounds__(256) void dist_gemm(const float* __restrict__ A,
                                                 const float* __restrict__ B, int64_t M, int64_t N,
                                                 int dim, int metric,
                                                 const float* __restrict__ an,
                                                 const float* __restrict__ bn,
                                                 float* __restrict__ Dm) {
    __shared__ float As[kTK][kTM + 4];
    __shared__ float Bs[kTK][kTN + 4];
    const int tid = threadIdx.x;
    const int tx = tid & 15, ty = tid >> 4;           // 16 x 16 threads, 4 x 4 outputs each
    const int64_t m0 = (int64_t)blockIdx.y * kTM, n0 = (int64_t)blockIdx.x * kTN;
    float acc[4][4] = {};
    // loader: 256 threads x 4 elements = one 64 x 16 tile
    const int lr = tid >> 2, lk = (tid & 3) * 4;
    for (int k0 = 0; k0 < dim; k0 += kTK) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int k = k0 + lk + e;
            const int64_t am = m0 + lr, bnn = n0 + lr;
            As[lk + e][lr] = (am < M && k < dim) ? A[am * dim + k] : 0.f;
            Bs[lk + e][lr] = (bnn < N && k < dim) ? B[bnn * dim + k] : 0.f;
        }
        __syncthreads();
#pragma unroll
        for (int k = 0; k < kTK; ++k) {
            float a[4], b[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) a[i] = As[k][ty * 4 + i];
#pragma unroll
            for (int j = 0; j < 4; ++j) b[j] = Bs[k][tx * 4 + j];
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_fmaf(a[i], b[j], acc[i][j]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int64_t m = m0 + ty * 4 + i;
        if (m >= M) continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int64_t nn = n0 + tx * 4 + j;
            if (nn >= N) continue;
            const float s = acc[i][j];
            Dm[m * N + nn] = metric == SWANN_METRIC_IP ? 1.0f - s : (bn[nn] - 2.0f * s) + an[m];
        }
    }
}

// Bitonic sort of kTopBuf (d, i) pairs in LDS, ascending.
__device__ void lds_sort(float* sd, int* si, int n) {
    for (int size = 2; size <= n; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int i = threadIdx.x; i < n; i += kTopBlock) {
                const int j = i ^ stride;
                if (j > i) {
                    const bool up = ((i & size) == 0);
                    if (up != lt(sd[i], si[i], sd[j], si[j])) {
                        const float td = sd[i]; sd[i] = sd[j]; sd[j] = td;
                        const int ti = si[i]; si[i] = si[j]; si[j] = ti;
                    }
                }
            }
            __syncthreads();
        }
    }
}

// Row top-E of Dm [M, N]: out_idx/out_dist [M, E], ascending by (d, index).
__global__ __launch_bounds__(kTopBlock) void row_topk(const float* __restrict__ Dm, int64_t M,
                                                     int64_t N, int E, int32_t* __restrict__ oi,
                                                     float* __restrict__ od) {
    __shared__ float sd[kTopBuf];
    __shared__ int si[kTopBuf];
    const int64_t r = blockIdx.x;
    const float* row = Dm + r * N;
    int keep = 0;                       // running best held in [0, keep)
    int64_t c0 = 0;
    while (c0 < N) {
        const int64_t take = (N - c0) < (int64_t)(kTopBuf - keep) ? (N - c0) : (kTopBuf - keep);
        int fill = keep + (int)take;
        int n = 2;
        while (n < fill) n <<= 1;
        for (int i = keep + threadIdx.x; i < n; i += kTopBlock) {
            const int64_t c = c0 + (i - keep);
            const bool real = i < fill;
            sd[i] = real ? row[c] : INFINITY;
            si[i] = real ? (int)c : INT32_MAX;
        }
        __syncthreads();
        lds_sort(sd, si, n);
        c0 += take;
        keep = fill < E ? fill : E;
    }
    for (int e = threadIdx.x; e < E; e += kTopBlock) {
        const bool ok = e < keep;
        oi[r * E + e] = ok ? si[e] : -1;
        if (od) od[r * E + e] = ok ? sd[e] : INFINITY;
    }
}

}  // namespace
}  // namespace swann

using namespace swann;

extern "C" {

int64_t swann_select_workspace_size(int64_t nq, int64_t P) {
    // distance matrix + both norm vectors, each 256-byte aligned
    const int64_t a = ((nq * P * 4 + 255) / 256) * 256;
    const int64_t b = ((nq * 4 + 255) / 256) * 256;
    const int64_t c = ((P * 4 + 255) / 256) * 256;
    return a + b + c;
}

int swann_select_nearest(const float* Q, int64_t nq, int dim, const float* Vp, int64_t P, int E,
                         int metric, int32_t* out_idx, float* out_dist, void* workspace,
                         void* stream) {
    clear_error();
    SWANN_REQUIRE(metric == SWANN_METRIC_IP || metric == SWANN_METRIC_L2,
                  "metric must be 0 (ip) or 1 (l2)");
    SWANN_REQUIRE(nq >= 0 && P >= 1 && dim >= 1, "select: need nq >= 0, P >= 1, dim >= 1");
    SWANN_REQUIRE(E >= 1 && E <= kTopBuf / 2, "select: E must be in 1..%d", kTopBuf / 2);
    SWANN_REQUIRE(E <= P, "select: E (%d) exceeds the catalogue size (%lld)", E, (long long)P);
    SWANN_REQUIRE(nq <= INT32_MAX && (P + kTN - 1) / kTN <= INT32_MAX &&
                      (nq + kTM - 1) / kTM <= 65535,
                  "select: batch of %lld queries too large for one call", (long long)nq);
    if (nq == 0) return SWANN_OK;
    SWANN_REQUIRE(Q && Vp && out_idx && workspace, "select: a required pointer is NULL");
    hipStream_t st = (hipStream_t)stream;
    char* ws = (char*)workspace;
    float* Dm = (float*)ws;
    float* qn = (float*)(ws + ((nq * P * 4 + 255) / 256) * 256);
    float* vn = (float*)((char*)qn + ((nq * 4 + 255) / 256) * 256);
    if (metric == SWANN_METRIC_L2) {
        hipLaunchKernelGGL(row_norms, dim3((unsigned)((nq + 3) / 4)), dim3(256), 0, st, Q, nq, dim,
                           qn);
        hipLaunchKernelGGL(row_norms, dim3((unsigned)((P + 3) / 4)), dim3(256), 0, st, Vp, P, dim,
                           vn);
    }
    dim3 grid((unsigned)((P + kTN - 1) / kTN), (unsigned)((nq + kTM - 1) / kTM));
    hipLaunchKernelGGL(dist_gemm, grid, dim3(256), 0, st, Q, Vp, nq, P, dim, metric, qn, vn, Dm);
    int rc = launch_status("select gemm");
    if (rc) return rc;
    hipLaunchKernelGGL(row_topk, dim3((unsigned)nq), dim3(kTopBlock), 0, st, Dm, nq, P, E, out_idx,
                       out_dist);
    return launch_status("select top-E");
}

}  // extern "C"
