// Seed selection: the E nearest catalogue rows per query (swann/_select.py:93-128).
//
// Two steps: a tiled fp32 distance GEMM that writes the distance matrix
// D[q, p] (1 - <q,v> for IP; |v|^2 - 2<q,v> + |q|^2 for L2, the reference's
// formulas) into a caller-owned workspace, and a per-row top-E, ascending by
// (distance, index).  The reference folds slices of 8192 columns into a
// running best; the result is the exact top-E either way.
//
// Batches of up to 8 queries read the catalogue once in a wave-per-rows
// product (dist_gemv).  Larger batches that would still leave most of the
// chip idle (64 queries against a 4096-entry catalogue are 64 GEMM tiles)
// split the K dimension so the grid has >= 1024 workgroups: partial dot
// products go to the workspace, and a finishing pass sums them in split
// order and applies the formula.
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

// Order-preserving key of a distance: -0 folded onto +0, so equal distances
// have equal keys; every NaN takes the largest key, so it ranks after every
// number (as torch.topk ranks NaN) and the order is total.
__device__ __forceinline__ unsigned dkey(float d) {
    if (d != d) return 0xFFFFFFFFu;
    const unsigned u = __float_as_uint(d + 0.0f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// (distance, index) order: on numbers the plain comparison; a NaN after
// every number, NaNs by index.  Total, so a sorting network run on it keeps
// every element once and sorts the padding (pad_d(), INT32_MAX) last.
__device__ __forceinline__ bool lt(float da, int ia, float db, int ib) {
    const unsigned ka = dkey(da), kb = dkey(db);
    return ka < kb || (ka == kb && ia < ib);
}

// The distance of a padding entry: a NaN, which with index INT32_MAX ranks
// after every real entry.
__device__ __forceinline__ float pad_d() { return __int_as_float(0x7fffffff); }

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

// Small batches (nq <= kGvMaxQ): D[m, p] for every query m against catalogue
// rows p, the catalogue read once.  A wave takes kGvRows consecutive rows
// (one: a 4096-row catalogue is 4096 waves, with eight 16-byte loads of the
// row in flight a lane); lane l sums the 4-float blocks l, l + 64, ... of
// each row against each query, which the workgroup stages in LDS
// kGvLds / NQ dimensions at a time; then the wave folds each sum.  For l2 the
// row's |v|^2 is summed on the way.  The 64 x 64 tiles of dist_gemm would
// spend 63 of 64 products on padding at batch 1 and read the catalogue
// through 16 split-K passes.  (Measured at 4096 x 4096 with the top-E: 1
// row and 8 waves a workgroup beat 2 or 4 rows a wave and 4 waves.)
constexpr int kGvRows = 1, kGvWaves = 8, kGvMaxQ = 8;
constexpr int kGvLds = 8192;                  // staged query floats (32 KB)

template <int NQ>
__global__ __launch_bounds__(kGvWaves * 64) void dist_gemv(const float* __restrict__ Q,
                                                           const float* __restrict__ V, int nq,
                                                           int64_t P, int dim, int metric,
                                                           const float* __restrict__ qn,
                                                           float* __restrict__ Dm) {
    constexpr int KC = kGvLds / NQ;           // dimensions staged a pass
    __shared__ __align__(16) float qs[kGvLds];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t p0 = ((int64_t)blockIdx.x * kGvWaves + wave) * kGvRows;
    const bool vec = (dim & 3) == 0 && ((uintptr_t)V & 15) == 0;
    const bool qvec = (dim & 3) == 0 && ((uintptr_t)Q & 15) == 0;
    float acc[kGvRows][NQ], vv[kGvRows];
#pragma unroll
    for (int r = 0; r < kGvRows; ++r) {
        vv[r] = 0.f;
#pragma unroll
        for (int m = 0; m < NQ; ++m) acc[r][m] = 0.f;
    }
    // rows past P read row P - 1 (their sums are never written)
    const float* vr[kGvRows];
#pragma unroll
    for (int r = 0; r < kGvRows; ++r) vr[r] = V + (p0 + r < P ? p0 + r : P - 1) * (int64_t)dim;
    for (int k0 = 0; k0 < dim; k0 += KC) {
        const int kc = dim - k0 < KC ? dim - k0 : KC;
        __syncthreads();                      // the last pass's reads of qs are done
        if (qvec) {
            // 16-byte loads, four in flight a thread
            const int nv = NQ * (kc >> 2);
#pragma unroll 4
            for (int i = tid; i < nv; i += kGvWaves * 64) {
                const int m = i / (kc >> 2), t = (i - m * (kc >> 2)) << 2;
                const float4 v = m < nq ? *reinterpret_cast<const float4*>(Q + (int64_t)m * dim + k0 + t)
                                        : make_float4(0.f, 0.f, 0.f, 0.f);
                *reinterpret_cast<float4*>(&qs[m * KC + t]) = v;
            }
        } else {
            for (int i = tid; i < NQ * kc; i += kGvWaves * 64) {
                const int m = i / kc, t = i - m * kc;
                qs[m * KC + t] = m < nq ? Q[(int64_t)m * dim + k0 + t] : 0.f;
            }
        }
        __syncthreads();
        if (vec) {
#pragma unroll 8
            for (int t = lane * 4; t < kc; t += 256) {
                float4 x[kGvRows];
#pragma unroll
                for (int r = 0; r < kGvRows; ++r)
                    x[r] = *reinterpret_cast<const float4*>(vr[r] + k0 + t);
#pragma unroll
                for (int m = 0; m < NQ; ++m) {
                    const float4 q = *reinterpret_cast<const float4*>(&qs[m * KC + t]);
#pragma unroll
                    for (int r = 0; r < kGvRows; ++r) {
                        float s = acc[r][m];
                        s = __builtin_fmaf(x[r].x, q.x, s);
                        s = __builtin_fmaf(x[r].y, q.y, s);
                        s = __builtin_fmaf(x[r].z, q.z, s);
                        acc[r][m] = __builtin_fmaf(x[r].w, q.w, s);
                    }
                }
                if (metric == SWANN_METRIC_L2) {
#pragma unroll
                    for (int r = 0; r < kGvRows; ++r) {
                        float s = vv[r];
                        s = __builtin_fmaf(x[r].x, x[r].x, s);
                        s = __builtin_fmaf(x[r].y, x[r].y, s);
                        s = __builtin_fmaf(x[r].z, x[r].z, s);
                        vv[r] = __builtin_fmaf(x[r].w, x[r].w, s);
                    }
                }
            }
        } else {
            for (int t = lane; t < kc; t += 64) {
                float x[kGvRows];
#pragma unroll
                for (int r = 0; r < kGvRows; ++r) x[r] = vr[r][k0 + t];
#pragma unroll
                for (int m = 0; m < NQ; ++m) {
                    const float q = qs[m * KC + t];
#pragma unroll
                    for (int r = 0; r < kGvRows; ++r) acc[r][m] = __builtin_fmaf(x[r], q, acc[r][m]);
                }
#pragma unroll
                for (int r = 0; r < kGvRows; ++r) vv[r] = __builtin_fmaf(x[r], x[r], vv[r]);
            }
        }
    }
    // fold every sum over the wave (each lane ends with every total); lane
    // r * NQ + m writes D[m, p0 + r]
    float out = 0.f;
#pragma unroll
    for (int r = 0; r < kGvRows; ++r) {
        float n2 = vv[r];
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) n2 += __shfl_xor(n2, off, 64);
#pragma unroll
        for (int m = 0; m < NQ; ++m) {
            float s = acc[r][m];
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
            if (lane == r * NQ + m)
                out = metric == SWANN_METRIC_IP ? 1.0f - s
                                                : (n2 - 2.0f * s) + (m < nq ? qn[m] : 0.f);
        }
    }
    const int r = lane / NQ, m = lane - r * NQ;
    if (lane < kGvRows * NQ && m < nq && p0 + r < P) Dm[(int64_t)m * P + p0 + r] = out;
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
    // slots i < nper hold keys (column tid + i * kRadBlock); the loops below
    // visit only those, and skip the padding columns c >= N
    const int nper = (int)((N + kRadBlock - 1) / kRadBlock);
    unsigned key[kRadPer];
#pragma unroll
    for (int i = 0; i < kRadPer; ++i) {
        const int64_t c = tid + (int64_t)i * kRadBlock;
        key[i] = (i < nper && c < N) ? dkey(row[c]) : 0xFFFFFFFFu;
    }
    // ---- the E-th smallest key, 8 bits at a time from the top ----
    unsigned prefix = 0u, pmask = 0u;
    int need = E;                       // how many to take from the current bucket
    for (int pass = 0; pass < 4; ++pass) {
        const int shift = 24 - 8 * pass;
        if (tid < 256) hist[tid] = 0u;
        __syncthreads();
        // Distances that share their leading bits (all of them, in the
        // first pass over a row of similar distances) fall into a few bins:
        // lanes of a wave that share the first two bins add with one atomic
        // each, the rest one by one.
#pragma unroll
        for (int i = 0; i < kRadPer; ++i) {
            if (i >= nper) break;
            const unsigned bin = (key[i] >> shift) & 255u;
            bool pend = tid + i * kRadBlock < N && (key[i] & pmask) == prefix;
#pragma unroll
            for (int peel = 0; peel < 2; ++peel) {
                const uint64_t act = __ballot(pend);
                if (act == 0) break;
                const unsigned b0 = __builtin_amdgcn_readlane(bin, __builtin_ctzll(act));
                const uint64_t same = __ballot(pend && bin == b0);
                if (pend && bin == b0) {
                    if (lane == __builtin_ctzll(same))
                        atomicAdd(&hist[b0], (unsigned)__builtin_popcountll(same));
                    pend = false;
                }
            }
            if (pend) atomicAdd(&hist[bin], 1u);
        }
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
        if (i >= nper) break;
        if (key[i] < T) {
            const int pos = atomicAdd(&s_nsel, 1);
            const int c = tid + i * kRadBlock;
            sd[pos] = row[c]; si[pos] = c;
        }
    }
    __syncthreads();
    const int nless = s_nsel;           // == E - need
    // ties at T in index order (c = tid + i*kRadBlock: i-major, then tid)
    for (int i = 0; i < nper; ++i) {
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
    if (E <= 64) {
        // one wave, in registers: a bitonic network over 64 lanes (lanes
        // past E hold the padding entry and sort last), no barriers
        __syncthreads();
        if (wave != 0) return;
        float d = lane < E ? sd[lane] : pad_d();
        int id = lane < E ? si[lane] : INT32_MAX;
#pragma unroll
        for (int size = 2; size <= 64; size <<= 1) {
#pragma unroll
            for (int stride = size >> 1; stride > 0; stride >>= 1) {
                const float d2 = __shfl_xor(d, stride, 64);
                const int id2 = __shfl_xor(id, stride, 64);
                // both lanes of a pair decide the same swap, from the lower
                // lane's element (so a pair the order cannot rank, NaN
                // against NaN, is swapped or kept whole, never duplicated)
                const bool up = (lane & size) == 0;
                const bool sw = (lane & stride) == 0 ? up != lt(d, id, d2, id2)
                                                     : up != lt(d2, id2, d, id);
                if (sw) { d = d2; id = id2; }
            }
        }
        if (lane < E) {
            oi[r * E + lane] = id;
            if (od) od[r * E + lane] = d;
        }
        return;
    }
    int n = 1;
    while (n < E) n <<= 1;
    for (int i = E + tid; i < n; i += kRadBlock) { sd[i] = pad_d(); si[i] = INT32_MAX; }
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
            sd[i] = real ? row[c] : pad_d();
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

// The distance matrix of a small batch: one pass over the catalogue.
static int gemv_run(const float* Q, int64_t nq, int dim, const float* Vp, int64_t P, int metric,
                    const float* qn, float* Dm, hipStream_t st) {
    const dim3 g((unsigned)((P + kGvRows * kGvWaves - 1) / (kGvRows * kGvWaves)));
    const dim3 b(kGvWaves * 64);
    const int q = (int)nq;
    if (nq == 1) hipLaunchKernelGGL(dist_gemv<1>, g, b, 0, st, Q, Vp, q, P, dim, metric, qn, Dm);
    else if (nq == 2) hipLaunchKernelGGL(dist_gemv<2>, g, b, 0, st, Q, Vp, q, P, dim, metric, qn, Dm);
    else if (nq <= 4) hipLaunchKernelGGL(dist_gemv<4>, g, b, 0, st, Q, Vp, q, P, dim, metric, qn, Dm);
    else hipLaunchKernelGGL(dist_gemv<8>, g, b, 0, st, Q, Vp, q, P, dim, metric, qn, Dm);
    return launch_status("select gemv");
}

// The distance matrix of a larger batch: 64 x 64 tiles, K split when the
// tiles alone would not fill the chip.
static int gemm_run(const float* Q, int64_t nq, int dim, const float* Vp, int64_t P, int metric,
                    const float* qn, float* vn, float* Dm, hipStream_t st) {
    if (metric == SWANN_METRIC_L2)
        hipLaunchKernelGGL(row_norms, dim3((unsigned)((P + 3) / 4)), dim3(256), 0, st, Vp, P, dim,
                           vn);
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
    return launch_status("select gemm");
}

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
    if (metric == SWANN_METRIC_L2)
        hipLaunchKernelGGL(row_norms, dim3((unsigned)((nq + 3) / 4)), dim3(256), 0, st, Q, nq, dim,
                           qn);
    const int rc = nq <= kGvMaxQ ? gemv_run(Q, nq, dim, Vp, P, metric, qn, Dm, st)
                                 : gemm_run(Q, nq, dim, Vp, P, metric, qn, vn, Dm, st);
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
