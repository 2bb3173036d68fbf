// Candidate sweep on MFMA: exact top-C neighbours of every row (swann/build.py:28-43)
// as a dense contraction on gfx950 matrix cores with the top-C selection fused
// into the tile epilogue, so the n^2 scores never reach HBM.
//
// Operands are 16-bit rows of X, read K-contiguous for both sides of
// S = X_rows . X_cols^T:
//   * an fp16 corpus is used as is: fp16 x fp16 products are exact in fp32 and
//     accumulate in fp32, so the scores are as good as an fp32 GEMM's;
//   * an fp32 corpus is split per row into hi = fp16(x / s) and
//     lo = fp16((x / s - hi) * 2^11) with s a power of two (exact scaling), and
//     s_a s_b (hi.hi + 2^-11 (hi.lo + lo.hi)) carries ~22 significant bits --
//     fp32-grade scores from three fp16 MFMA terms.
// Workgroup: 256 threads = 4 waves in 2 x 2, tile 128 rows x 128 columns, each
// wave 64 x 64 = 2 x 2 blocks of v_mfma_f32_32x32x16_f16, K step 32, the next
// K tile prefetched into registers while the current one is consumed.
// Epilogue per tile: score -> distance by the reference formula, test against
// the row's running threshold (LDS), append survivors to the row's buffer;
// rows near capacity are compacted to their C best (wave-level exact select).
#include <float.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "common.h"

namespace swann {
namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kBM = 128, kBN = 128, kBK = 32;
constexpr int kPad = 8;                       // fp16 elements of padding per LDS row
constexpr int kLdsRow = kBK + kPad;           // 40 halves = 80 bytes
constexpr float kSelf = 3.4e38f;

__device__ __forceinline__ uint32_t fkey(float f) {
    const uint32_t b = __float_as_uint(f);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float funkey(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

__device__ __forceinline__ float dist_formula(float dot, float na, float nb, int metric) {
    if (metric == SWANN_METRIC_IP) return 1.0f - dot;
    const float v = (nb - 2.0f * dot) + na;
    return v < 0.f ? 0.f : v;
}

// ---------------------------------------------------------------------------
// fp32 rows -> (hi, lo, scale); fp16 rows -> norms only.
__global__ __launch_bounds__(256) void split_rows(const float* __restrict__ X, int64_t n, int dim,
                                                  _Float16* __restrict__ hi,
                                                  _Float16* __restrict__ lo,
                                                  float* __restrict__ scale,
                                                  float* __restrict__ norm) {
    const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (r >= n) return;
    const float* x = X + r * dim;
    float m = 0.f, s2 = 0.f;
    for (int t = lane; t < dim; t += 64) {
        const float v = x[t];
        m = fmaxf(m, fabsf(v));
        s2 = __builtin_fmaf(v, v, s2);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        m = fmaxf(m, __shfl_xor(m, off, 64));
        s2 += __shfl_xor(s2, off, 64);
    }
    // s = 2^e with m / s <= 1 (exact division by a power of two)
    int e = 0;
    if (m > 0.f) { frexpf(m, &e); }
    const float s = ldexpf(1.0f, e);
    const float inv = ldexpf(1.0f, -e);
    for (int t = lane; t < dim; t += 64) {
        const float v = x[t] * inv;
        const _Float16 h = (_Float16)v;
        hi[r * dim + t] = h;
        lo[r * dim + t] = (_Float16)((v - (float)h) * 2048.0f);
    }
    if (lane == 0) { scale[r] = s; norm[r] = s2; }
}

__global__ __launch_bounds__(256) void norms_f16(const _Float16* __restrict__ X, int64_t n,
                                                 int dim, float* __restrict__ norm,
                                                 float* __restrict__ scale) {
    const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (r >= n) return;
    float s2 = 0.f;
    for (int t = lane; t < dim; t += 64) { const float v = (float)X[r * dim + t]; s2 = __builtin_fmaf(v, v, s2); }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) s2 += __shfl_xor(s2, off, 64);
    if (lane == 0) { norm[r] = s2; scale[r] = 1.0f; }
}

// ---------------------------------------------------------------------------
struct MfmaSweepArgs {
    const _Float16* hi; const _Float16* lo; const float* scale; const float* xn;
    int64_t n; int dim; int metric; int C; int cap;
    float* bkey; int32_t* bid; int32_t* bcnt;
};

// Wave-cooperative compaction of one row's buffer to its C best (exact:
// threshold by bitwise search, ties kept in index order).
__device__ void compact_row_w(float* key, int32_t* id, int cnt, int C, float* thr_out,
                              int* cnt_out) {
    const int lane = threadIdx.x & 63;
    constexpr int R = 16;                      // cap <= 1024
    uint32_t u[R];
#pragma unroll
    for (int t = 0; t < R; ++t) {
        const int i = t * 64 + lane;
        u[t] = i < cnt ? fkey(key[i]) : 0xffffffffu;
    }
    uint32_t lo = 0, hi = 0xffffffffu;
    while (lo < hi) {
        const uint32_t mid = lo + ((hi - lo) >> 1);
        int c = 0;
#pragma unroll
        for (int t = 0; t < R; ++t) c += (t * 64 + lane < cnt && u[t] <= mid) ? 1 : 0;
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) c += __shfl_xor(c, off, 64);
        if (c >= C) hi = mid; else lo = mid + 1;
    }
    const uint32_t T = lo;
    int nlt = 0;
#pragma unroll
    for (int t = 0; t < R; ++t) nlt += (t * 64 + lane < cnt && u[t] < T) ? 1 : 0;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) nlt += __shfl_xor(nlt, off, 64);
    int eq_left = C - nlt;
    int w = 0;
    const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
#pragma unroll
    for (int t = 0; t < R; ++t) {
        const int i = t * 64 + lane;
        const bool in = i < cnt;
        const bool is_lt = in && u[t] < T;
        const bool is_eq = in && u[t] == T;
        const uint64_t meq = __ballot(is_eq);
        const int eq_rank = __popcll(meq & below);
        const bool keep = is_lt || (is_eq && eq_rank < eq_left);
        const uint64_t mk = __ballot(keep);
        const int kid = in ? id[i] : 0;
        const float kk = in ? key[i] : 0.f;
        if (keep) {
            const int dst = w + __popcll(mk & below);
            key[dst] = kk;
            id[dst] = kid;
        }
        w += __popcll(mk);
        const int used = __popcll(meq);
        eq_left -= used < eq_left ? used : eq_left;
    }
    if (lane == 0) { *thr_out = funkey(T); *cnt_out = w; }
}

template <int NTERM>
__global__ __launch_bounds__(256) void sweep_mfma_kernel(MfmaSweepArgs a) {
    constexpr int NT = (NTERM == 1) ? 1 : 2;          // operand planes: hi (and lo)
    __shared__ __align__(16) _Float16 sA[NT][kBM * kLdsRow];
    __shared__ __align__(16) _Float16 sB[NT][kBN * kLdsRow];
    __shared__ float thr[kBM];
    __shared__ int cnt[kBM];
    __shared__ float rnorm[kBM], rscale[kBM];
    __shared__ int need;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;          // wave's 64 x 64 quadrant
    const int64_t n = a.n;
    const int dim = a.dim;
    // XCD-aware: consecutive row tiles share an XCD (and its L2 copy of the columns)
    const int64_t ntile = (n + kBM - 1) / kBM;
    const int64_t r0 = xcd_remap(blockIdx.x, ntile) * kBM;

    if (tid < kBM) {
        const int64_t r = r0 + tid;
        thr[tid] = INFINITY;
        cnt[tid] = 0;
        rnorm[tid] = r < n ? a.xn[r] : 0.f;
        rscale[tid] = r < n ? a.scale[r] : 1.f;
    }
    if (tid == 0) need = 0;
    __syncthreads();

    // loader: 128 rows x 64 bytes per plane = 512 chunks of 16 B, 2 per thread
    const int c0i = tid, c1i = tid + 256;
    const int lr0 = c0i >> 2, lp0 = (c0i & 3) * 8;
    const int lr1 = c1i >> 2, lp1 = (c1i & 3) * 8;

    for (int64_t cb = 0; cb < n; cb += kBN) {
        f32x16 acc[2][2], accx[2][2];
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                acc[i][j] = (f32x16){};
                accx[i][j] = (f32x16){};
            }
        f16x8 ga[NT][2], gb[NT][2];
        auto gload = [&](int k0) {
#pragma unroll
            for (int p = 0; p < NT; ++p) {
                const _Float16* M = p == 0 ? a.hi : a.lo;
                const int64_t ra0 = r0 + lr0, ra1 = r0 + lr1;
                const int64_t rb0 = cb + lr0, rb1 = cb + lr1;
                const f16x8 z = {};
                ga[p][0] = (ra0 < n && k0 + lp0 < dim) ? *reinterpret_cast<const f16x8*>(M + ra0 * dim + k0 + lp0) : z;
                ga[p][1] = (ra1 < n && k0 + lp1 < dim) ? *reinterpret_cast<const f16x8*>(M + ra1 * dim + k0 + lp1) : z;
                gb[p][0] = (rb0 < n && k0 + lp0 < dim) ? *reinterpret_cast<const f16x8*>(M + rb0 * dim + k0 + lp0) : z;
                gb[p][1] = (rb1 < n && k0 + lp1 < dim) ? *reinterpret_cast<const f16x8*>(M + rb1 * dim + k0 + lp1) : z;
            }
        };
        gload(0);
        for (int k0 = 0; k0 < dim; k0 += kBK) {
#pragma unroll
            for (int p = 0; p < NT; ++p) {
                *reinterpret_cast<f16x8*>(&sA[p][lr0 * kLdsRow + lp0]) = ga[p][0];
                *reinterpret_cast<f16x8*>(&sA[p][lr1 * kLdsRow + lp1]) = ga[p][1];
                *reinterpret_cast<f16x8*>(&sB[p][lr0 * kLdsRow + lp0]) = gb[p][0];
                *reinterpret_cast<f16x8*>(&sB[p][lr1 * kLdsRow + lp1]) = gb[p][1];
            }
            __syncthreads();
            if (k0 + kBK < dim) gload(k0 + kBK);       // next tile in flight during the MFMAs
#pragma unroll
            for (int ks = 0; ks < kBK; ks += 16) {
                f16x8 fa[NT][2], fb[NT][2];
                const int kof = ks + (lane >> 5) * 8;
#pragma unroll
                for (int p = 0; p < NT; ++p)
#pragma unroll
                    for (int i = 0; i < 2; ++i) {
                        const int ar = wm * 64 + i * 32 + (lane & 31);
                        const int br = wn * 64 + i * 32 + (lane & 31);
                        fa[p][i] = *reinterpret_cast<const f16x8*>(&sA[p][ar * kLdsRow + kof]);
                        fb[p][i] = *reinterpret_cast<const f16x8*>(&sB[p][br * kLdsRow + kof]);
                    }
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[0][i], fb[0][j],
                                                                          acc[i][j], 0, 0, 0);
                        if constexpr (NTERM == 3) {
                            accx[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
                                fa[0][i], fb[1][j], accx[i][j], 0, 0, 0);
                            accx[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
                                fa[1][i], fb[0][j], accx[i][j], 0, 0, 0);
                        }
                    }
            }
            __syncthreads();
        }
        // ---- epilogue: distances, threshold test, append ----
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int cl = wn * 64 + j * 32 + (lane & 31);
            const int64_t c = cb + cl;
            const bool cok = c < n;
            const float cn = cok ? a.xn[c] : 0.f;
            const float cs = cok ? a.scale[c] : 1.f;
#pragma unroll
            for (int i = 0; i < 2; ++i) {
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int rl = wm * 64 + i * 32 + (e >> 2) * 8 + (lane >> 5) * 4 + (e & 3);
                    const int64_t r = r0 + rl;
                    if (!cok || r >= n) continue;
                    float dot;
                    if constexpr (NTERM == 3)
                        dot = rscale[rl] * cs * (acc[i][j][e] + accx[i][j][e] * (1.0f / 2048.0f));
                    else
                        dot = acc[i][j][e];
                    const float d = (c == r) ? kSelf : dist_formula(dot, rnorm[rl], cn, a.metric);
                    if (d < thr[rl]) {
                        const int p = atomicAdd(&cnt[rl], 1);
                        a.bkey[r * a.cap + p] = d;
                        a.bid[r * a.cap + p] = (int32_t)c;
                    }
                }
            }
        }
        __syncthreads();
        if (tid < kBM && cnt[tid] > a.cap - kBN) atomicOr(&need, 1);
        __syncthreads();
        if (need) {
            for (int rl = wave; rl < kBM; rl += 4) {
                const int64_t r = r0 + rl;
                if (r < n && cnt[rl] > a.cap - kBN)
                    compact_row_w(a.bkey + r * a.cap, a.bid + r * a.cap, cnt[rl], a.C, &thr[rl],
                                  &cnt[rl]);
            }
            __syncthreads();
            if (tid == 0) need = 0;
            __syncthreads();
        }
    }
    if (tid < kBM && r0 + tid < n) a.bcnt[r0 + tid] = cnt[tid];
}

inline int64_t al256(int64_t b) { return ((b + 255) / 256) * 256; }

}  // namespace

// Workspace layout for the MFMA sweep (bytes), after the row buffers.
int64_t sweep_mfma_extra_bytes(int64_t n, int dim, int x_dtype) {
    const int64_t planes = x_dtype == SWANN_DTYPE_F16 ? 0 : 2;
    return al256(n * 4) * 2 + planes * al256(n * (int64_t)dim * 2);
}

int sweep_mfma_cap(int C) {
    int cap = C + 640;
    return cap > 1024 ? 1024 : cap;
}

// Runs the MFMA sweep into the row buffers (bkey/bid/bcnt); the caller sorts.
int sweep_mfma_run(const void* X, int x_dtype, int64_t n, int dim, int metric, int C, int cap,
                   float* bkey, int32_t* bid, int32_t* bcnt, char* extra, hipStream_t st) {
    float* xn = (float*)extra; extra += al256(n * 4);
    float* scale = (float*)extra; extra += al256(n * 4);
    const _Float16* hi;
    const _Float16* lo = nullptr;
    if (x_dtype == SWANN_DTYPE_F16) {
        hi = (const _Float16*)X;
        hipLaunchKernelGGL(norms_f16, dim3((unsigned)((n + 3) / 4)), dim3(256), 0, st, hi, n, dim,
                           xn, scale);
    } else {
        _Float16* h = (_Float16*)extra; extra += al256(n * (int64_t)dim * 2);
        _Float16* l = (_Float16*)extra;
        hipLaunchKernelGGL(split_rows, dim3((unsigned)((n + 3) / 4)), dim3(256), 0, st,
                           (const float*)X, n, dim, h, l, scale, xn);
        hi = h;
        lo = l;
    }
    MfmaSweepArgs a{hi, lo, scale, xn, n, dim, metric, C, cap, bkey, bid, bcnt};
    const unsigned grid = (unsigned)((n + kBM - 1) / kBM);
    if (x_dtype == SWANN_DTYPE_F16)
        hipLaunchKernelGGL(sweep_mfma_kernel<1>, dim3(grid), dim3(256), 0, st, a);
    else
        hipLaunchKernelGGL(sweep_mfma_kernel<3>, dim3(grid), dim3(256), 0, st, a);
    return launch_status("sweep (mfma)");
}

}  // namespace swann
