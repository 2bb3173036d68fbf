// Seed selection: the E nearest catalogue rows per query (swann/_select.py:93-128).
//
// Two steps: a tiled fp32 distance GEMM that writes the distance matrix
// D[q, p] (1 - <q,v> for IP; |v|^2 - 2<q,v> + |q|^2 for L2, the reference's
// formulas) into a caller-owned workspace, and a per-row top-E, ascending by
// (distance, index).  The reference folds slices of 8192 columns into a
// running best; the result is the exact top-E either way.
//
// Small batches would leave most of the chip idle: a batch of 8 against a
// 4096-entry catalogue is 64 GEMM tiles.  There the K dimension is split so
// the grid has >= 1024 workgroups, partial dot products go to the workspace,
// and a finishing pass sums them in split order and applies the formula.
// The top-E keeps a row of up to 16384 distances in the registers of 1024
// threads and finds the E-th smallest by a 4-pass radix select over the
// distances' order-preserving 32-bit keys (LDS histograms), then sorts only
// the E survivors; longer rows use the chunked bitonic kernel.
#include <float.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>
#include <mutex>

#include "common.h"

namespace swann {
namespace {

constexpr int kTM = 64, kTN = 64, kTK = 16;   // GEMM tile
constexpr int kTopBuf = 4096;                 // pairs held in LDS by the top-E kernel
constexpr int kTopBlock = 256;
constexpr int kRadBlock = 1024, kRadPer = 16; // radix top-E: rows of up to 16384
constexpr int kRadMaxE = 2048;
constexpr int kMaxSplit = 16;

// K splits for a grid of `tiles` workgroups: enough for >= 1024 workgroups.
int split_for(int64_t tiles) {
    if (tiles >= 256) return 1;
    int64_t s = (1024 + tiles - 1) / tiles;
    return (int)(s < kMaxSplit ? s : kMaxSplit);
}

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

// D[m, n] = f(<A_m, B_n>) for A [M, dim], B [N, dim], both row-major.  With
// `kper` < dim, workgroup z covers k in [z*kper, (z+1)*kper) and writes the
// raw partial dot product to Dm + z*M*N (finished by split_finish).
__global__ __launch_bounds__(256) void dist_gemm(const float* __restrict__ A,
                                                 const float* __restrict__ B, int64_t M, int64_t N,
                                                 int dim, int metric,
                                                 const float* __restrict__ an,
                                                 const float* __restrict__ bn,
                                                 float* __restrict__ Dm, int kper) {
    __shared__ float As[kTK][kTM + 4];
    __shared__ float Bs[kTK][kTN + 4];
    const int tid = threadIdx.x;
    const int tx = tid & 15, ty = tid >> 4;           // 16 x 16 threads, 4 x 4 outputs each
    const int64_t m0 = (int64_t)blockIdx.y * kTM, n0 = (int64_t)blockIdx.x * kTN;
    float acc[4][4] = {};
    // loader: 256 threads x 4 elements = one 64 x 16 tile
    const int lr = tid >> 2, lk = (tid & 3) * 4;
    const int kb = blockIdx.z * kper;
    const int ke = (kb + kper < dim) ? kb + kper : dim;
    for (int k0 = kb; k0 < ke; k0 += kTK) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int k = k0 + lk + e;
            const int64_t am = m0 + lr, bnn = n0 + lr;
            As[lk + e][lr] = (am < M && k < ke) ? A[am * dim + k] : 0.f;
            Bs[lk + e][lr] = (bnn < N && k < ke) ? B[bnn * dim + k] : 0.f;
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
            if (kper < dim)
                Dm[(int64_t)blockIdx.z * M * N + m * N + nn] = s;
            else
                Dm[m * N + nn] = metric == SWANN_METRIC_IP ? 1.0f - s : (bn[nn] - 2.0f * s) + an[m];
        }
    }
}

// Sum the S partial dot products in split order, then the distance formula.
__global__ __launch_bounds__(256) void split_finish(const float* __restrict__ part, int S,
                                                    int64_t M, int64_t N, int metric,
                                                    const float* __restrict__ an,
                                                    const float* __restrict__ bn,
                                                    float* __restrict__ Dm) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= M * N) return;
    float s = part[i];
    for (int z = 1; z < S; ++z) s += part[(int64_t)z * M * N + i];
    const int64_t m = i / N, nn = i - m * N;
    Dm[i] = metric == SWANN_METRIC_IP ? 1.0f - s : (bn[nn] - 2.0f * s) + an[m];
}

// Order-preserving key of a distance (-0 folded onto +0, so equal distances
// have equal keys); larger keys sort later.
__device__ __forceinline__ unsigned dkey(float d) {
    const unsigned u = __float_as_uint(d + 0.0f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Row top-E for rows of N <= kRadBlock*kRadPer: radix select of the E-th key,
// then a bitonic sort of the E survivors by (d, index).
__global__ __launch_bounds__(kRadBlock) void row_topk_radix(const float* __restrict__ Dm,
                                                           int64_t N, int E,
                                                           int32_t* __restrict__ oi,
                                                           float* __restrict__ od) {
    __shared__ unsigned hist[256];
    __shared__ unsigned s_bucket, s_before;
    __shared__ int s_nsel, s_wcnt[kRadBlock / 64], s_ebase;
    __shared__ float sd[kRadMaxE];
    __shared__ int si[kRadMaxE];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t r = blockIdx.x;
    const float* row = Dm + r * N;
    unsigned key[kRadPer];
#pragma unroll
    for (int i = 0; i < kRadPer; ++i) {
        const int64_t c = tid + (int64_t)i * kRadBlock;
        key[i] = c < N ? dkey(row[c]) : 0xFFFFFFFFu;
    }
    // ---- the E-th smallest key, 8 bits at a time from the top ----
    unsigned prefix = 0u, pmask = 0u;
    int need = E;                       // how many to take from the current bucket
    for (int pass = 0; pass < 4; ++pass) {
        const int shift = 24 - 8 * pass;
        if (tid < 256) hist[tid] = 0u;
        __syncthreads();
#pragma unroll
        for (int i = 0; i < kRadPer; ++i)
            if ((key[i] & pmask) == prefix) atomicAdd(&hist[(key[i] >> shift) & 255u], 1u);
        __syncthreads();
        if (wave == 0) {
            unsigned h[4], run = 0u;
#pragma unroll
            for (int j = 0; j < 4; ++j) { h[j] = hist[lane * 4 + j]; run += h[j]; }
            unsigned incl = run;        // inclusive scan of lane totals
#pragma unroll
            for (int off = 1; off < 64; off <<= 1) {
                const unsigned o = __shfl_up(incl, off, 64);
                if (lane >= off) incl += o;
            }
            unsigned before = incl - run;
            const bool mine = before < (unsigned)need && incl >= (unsigned)need;
            if (mine) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    if (before + h[j] >= (unsigned)need) { s_bucket = lane * 4 + j; s_before = before; break; }
                    before += h[j];
                }
            }
        }
        __syncthreads();
        prefix |= s_bucket << shift;
        pmask |= 0xFFu << shift;
        need -= (int)s_before;
        __syncthreads();
    }
    const unsigned T = prefix;          // keys < T: all taken; keys == T: the `need` lowest indices
    if (tid == 0) { s_nsel = 0; s_ebase = 0; }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kRadPer; ++i) {
        if (key[i] < T) {
            const int pos = atomicAdd(&s_nsel, 1);
            const int c = tid + i * kRadBlock;
            sd[pos] = row[c]; si[pos] = c;
        }
    }
    __syncthreads();
    const int nless = s_nsel;           // == E - need
    // ties at T in index order (c = tid + i*kRadBlock: i-major, then tid)
    for (int i = 0; i < kRadPer; ++i) {
        // padding slots (c >= N) carry the largest key and the largest
        // indices: never taken, even when a NaN distance ties them
        const bool eq = key[i] == T && tid + i * kRadBlock < N;
        const uint64_t m = __ballot(eq);
        if (lane == 0) s_wcnt[wave] = __builtin_popcountll(m);
        __syncthreads();
        int base = s_ebase;
        for (int w = 0; w < wave; ++w) base += s_wcnt[w];
        const int rank = base + __builtin_popcountll(m & ((1ull << lane) - 1ull));
        if (eq && rank < need) {
            const int c = tid + i * kRadBlock;
            sd[nless + rank] = row[c]; si[nless + rank] = c;
        }
        __syncthreads();
        if (tid == 0) {
            int tot = 0;
            for (int w = 0; w < kRadBlock / 64; ++w) tot += s_wcnt[w];
            s_ebase += tot;
        }
        __syncthreads();
        if (s_ebase >= need) break;     // uniform: every later tie ranks >= need
    }
    // ---- sort the E survivors by (d, index) ----
    int n = 1;
    while (n < E) n <<= 1;
    for (int i = E + tid; i < n; i += kRadBlock) { sd[i] = INFINITY; si[i] = INT32_MAX; }
    __syncthreads();
    for (int size = 2; size <= n; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int i = tid; i < n; i += kRadBlock) {
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
    for (int e = tid; e < E; e += kRadBlock) {
        oi[r * E + e] = si[e];
        if (od) od[r * E + e] = sd[e];
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

// ---- the fixed workspace of swann_select_nearest_noalloc -------------------
// One array per GPU in the library's own device memory, reserved when the
// code object loads on that device and held until the process ends, so the
// no-alloc entry point never calls an allocator.  In host code `scratch` only
// names the symbol; its address on a device comes from hipGetSymbolAddress,
// looked up once per device (with that device current) and cached.
constexpr int64_t kScratchBytes = SWANN_SELECT_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch[kMaxDevices];
std::mutex g_scratch_mu;

int scratch_address(void** out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) {
        set_error("select (no-alloc): hipGetDevice failed: %s", hipGetErrorString(e));
        return SWANN_E_NODEVICE;
    }
    if (dev < 0 || dev >= kMaxDevices) {
        set_error("select (no-alloc): device %d out of range", dev);
        return SWANN_E_UNSUPPORTED;
    }
    void* p = g_scratch[dev].load(std::memory_order_acquire);
    if (!p) {
        std::lock_guard<std::mutex> lock(g_scratch_mu);
        p = g_scratch[dev].load(std::memory_order_relaxed);
        if (!p) {
            e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
            if (e != hipSuccess || !p) {
                set_error("select (no-alloc): hipGetSymbolAddress(scratch) failed on device %d: %s",
                          dev, hipGetErrorString(e));
                return SWANN_E_LAUNCH;
            }
            g_scratch[dev].store(p, std::memory_order_release);
        }
    }
    *out = p;
    return SWANN_OK;
}
}  // namespace

static int select_run(const float* Q, int64_t nq, int dim, const float* Vp, int64_t P, int E,
                      int metric, int32_t* out_idx, float* out_dist, void* workspace,
                      void* stream) {
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
    const int64_t tiles = ((P + kTN - 1) / kTN) * ((nq + kTM - 1) / kTM);
    int S = split_for(tiles);
    int kper = dim;
    if (S > 1) {
        kper = (dim + S - 1) / S;
        kper = ((kper + kTK - 1) / kTK) * kTK;
        S = (dim + kper - 1) / kper;
    }
    dim3 grid((unsigned)((P + kTN - 1) / kTN), (unsigned)((nq + kTM - 1) / kTM), (unsigned)S);
    if (S > 1) {
        float* part = (float*)((char*)vn + ((P * 4 + 255) / 256) * 256);
        hipLaunchKernelGGL(dist_gemm, grid, dim3(256), 0, st, Q, Vp, nq, P, dim, metric, qn, vn,
                           part, kper);
        hipLaunchKernelGGL(split_finish, dim3((unsigned)((nq * P + 255) / 256)), dim3(256), 0, st,
                           part, S, nq, P, metric, qn, vn, Dm);
    } else {
        hipLaunchKernelGGL(dist_gemm, grid, dim3(256), 0, st, Q, Vp, nq, P, dim, metric, qn, vn,
                           Dm, dim);
    }
    int rc = launch_status("select gemm");
    if (rc) return rc;
    if (P <= (int64_t)kRadBlock * kRadPer && E <= kRadMaxE)
        hipLaunchKernelGGL(row_topk_radix, dim3((unsigned)nq), dim3(kRadBlock), 0, st, Dm, P, E,
                           out_idx, out_dist);
    else
        hipLaunchKernelGGL(row_topk, dim3((unsigned)nq), dim3(kTopBlock), 0, st, Dm, nq, P, E,
                           out_idx, out_dist);
    return launch_status("select top-E");
}


extern "C" {

int64_t swann_select_workspace_size(int64_t nq, int64_t P) {
    // distance matrix + both norm vectors + (small batches) the split-K
    // partials, each 256-byte aligned
    const int64_t a = ((nq * P * 4 + 255) / 256) * 256;
    const int64_t b = ((nq * 4 + 255) / 256) * 256;
    const int64_t c = ((P * 4 + 255) / 256) * 256;
    const int S = split_for(((P + kTN - 1) / kTN) * ((nq + kTM - 1) / kTM));
    const int64_t d = S > 1 ? (int64_t)S * a : 0;
    return a + b + c + d;
}

int swann_select_nearest(const float* Q, int64_t nq, int dim, const float* Vp, int64_t P, int E,
                         int metric, int32_t* out_idx, float* out_dist, void* workspace,
                         void* stream) {
    clear_error();
    return select_run(Q, nq, dim, Vp, P, E, metric, out_idx, out_dist, workspace, stream);
}

int swann_select_nearest_noalloc(const float* Q, int64_t nq, int dim, const float* Vp, int64_t P,
                                 int E, int metric, int32_t* out_idx, float* out_dist,
                                 void* stream) {
    clear_error();
    SWANN_REQUIRE(nq >= 0 && P >= 1, "select: need nq >= 0, P >= 1");
    const int64_t need = swann_select_workspace_size(nq, P);
    SWANN_REQUIRE(need <= kScratchBytes,
                  "select (no-alloc): %lld queries x %lld catalogue rows need %lld bytes of "
                  "workspace; the built-in scratch holds %lld (use swann_select_nearest with a "
                  "workspace of swann_select_workspace_size bytes)",
                  (long long)nq, (long long)P, (long long)need, (long long)kScratchBytes);
    if (nq == 0) return select_run(Q, nq, dim, Vp, P, E, metric, out_idx, out_dist, nullptr,
                                   stream);
    void* ws = nullptr;
    const int rc = scratch_address(&ws);
    if (rc) return rc;
    return select_run(Q, nq, dim, Vp, P, E, metric, out_idx, out_dist, ws, stream);
}

}  // extern "C"
