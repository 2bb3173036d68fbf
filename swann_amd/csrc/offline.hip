// The offline builder's extras (offline/build_graph.py): candidates taken from
// an existing graph, mutual-rank protection, degree fill and the in-degree
// floor.  All graph-shaped integer work; each kernel is bandwidth or latency
// bound and none needs MFMA.
//
//   * candidates_from_graph (:63-91): one workgroup per row; 16-lane teams
//     score the row's first C graph entries exactly (1 - <a,v>, or the direct
//     sum of squares), -1 and self at 3.4e38; a bitonic sort in LDS orders them
//     by (distance, column).
//   * mutual_rank (:93-131): one thread per (node, rank < M) entry.
//   * fill_degree (:132-200): one workgroup per node, in chunks launched in
//     order, each chunk reading the graph as the earlier chunks left it and
//     writing its rows to a side buffer that is copied back after the chunk;
//     the bridge rule's two-hop set lives in an LDS hash table.
//   * enforce_min_in (:203-294): per round and candidate column a fixed
//     sequence of small kernels (offer -> decide -> move counts -> write), so
//     no step waits on the host; a column with nothing to place is a no-op,
//     as the reference's early exit.
#include <float.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "common.h"

namespace swann {
namespace {

constexpr float kFar = 3.4e38f;
constexpr int kCgMax = 256;        // candidates per row for candidates_from_graph
constexpr int kFillMaxW = 128;     // fill: row width
constexpr int kFillMaxC = 256;     // fill: candidates per row

__device__ __forceinline__ bool lt_dp(float da, int pa, float db, int pb) {
    return (da < db) || (da == db && pa < pb);
}

template <typename XT> __device__ __forceinline__ float ldf(const XT* p) { return (float)*p; }

// ---------------------------------------------------------------------------
template <typename XT>
__global__ __launch_bounds__(256) void cand_graph_kernel(const XT* __restrict__ X, int64_t n,
                                                         int dim, int metric,
                                                         const int32_t* __restrict__ Gc, int gw,
                                                         int C, int32_t* __restrict__ oi,
                                                         float* __restrict__ od) {
    __shared__ float sd[kCgMax];
    __shared__ int sp[kCgMax];
    const int64_t u = blockIdx.x;
    const int tid = threadIdx.x, team = tid >> 4, tl = tid & 15;
    const XT* a = X + u * dim;
    for (int j = team; j < C; j += 16) {
        const int v = Gc[u * gw + j];
        float acc = 0.f;
        const bool real = v >= 0 && v < n && v != u;
        if (real) {
            const XT* x = X + (int64_t)v * dim;
            for (int t = tl; t < dim; t += 16) {
                const float p = ldf(a + t), q = ldf(x + t);
                if (metric == SWANN_METRIC_IP) acc = __builtin_fmaf(p, q, acc);
                else { const float df = p - q; acc = __builtin_fmaf(df, df, acc); }
            }
        }
#pragma unroll
        for (int off = 8; off > 0; off >>= 1) acc += __shfl_down(acc, off, 16);
        if (tl == 0) {
            sd[j] = real ? (metric == SWANN_METRIC_IP ? 1.0f - acc : acc) : kFar;
            sp[j] = j;
        }
    }
    int np = 1;
    while (np < C) np <<= 1;
    for (int j = C + tid; j < np; j += 256) { sd[j] = INFINITY; sp[j] = INT32_MAX; }
    __syncthreads();
    for (int size = 2; size <= np; size <<= 1)
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int i = tid; i < np; i += 256) {
                const int j = i ^ stride;
                if (j > i) {
                    const bool up = (i & size) == 0;
                    if (up != lt_dp(sd[i], sp[i], sd[j], sp[j])) {
                        const float td = sd[i]; sd[i] = sd[j]; sd[j] = td;
                        const int tp = sp[i]; sp[i] = sp[j]; sp[j] = tp;
                    }
                }
            }
            __syncthreads();
        }
    for (int j = tid; j < C; j += 256) {
        oi[u * C + j] = Gc[u * gw + sp[j]];
        od[u * C + j] = sd[j];
    }
}

// ---------------------------------------------------------------------------
__global__ void mutual_kernel(const int32_t* __restrict__ cand, int64_t n, int C, int M,
                              uint8_t* __restrict__ out) {
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= n * C) return;
    const int64_t u = e / C;
    const int j = (int)(e - u * C);
    uint8_t m = 0;
    const int v = cand[e];
    if (j < M && v >= 0 && v < n) {
        const int32_t* h = cand + (int64_t)v * C;
        for (int t = 0; t < M; ++t)
            if (h[t] == (int32_t)u) { m = 1; break; }
    }
    out[e] = m;
}

// ---------------------------------------------------------------------------
// fill: rule 0 near, 1 far, 2 bridge.  Node u = s + blockIdx.x.
__global__ __launch_bounds__(256) void fill_kernel(const int32_t* __restrict__ G, int64_t n,
                                                   int W, const int32_t* __restrict__ cand, int C,
                                                   int rule, int64_t s, int hbits,
                                                   int32_t* __restrict__ next) {
    extern __shared__ int32_t hs[];                    // hash of the two-hop set (bridge)
    __shared__ int32_t kept[kFillMaxW];
    __shared__ int32_t cd[kFillMaxC];
    __shared__ int freeflag[kFillMaxC];
    __shared__ int empty[kFillMaxW];
    __shared__ int s_nempty;
    const int64_t u = s + blockIdx.x;
    const int tid = threadIdx.x;
    for (int k = tid; k < W; k += 256) kept[k] = G[u * W + k];
    for (int j = tid; j < C; j += 256) cd[j] = cand[u * C + j];
    const int hsize = rule == 2 ? (1 << hbits) : 0;
    for (int i = tid; i < hsize; i += 256) hs[i] = -1;
    __syncthreads();
    if (rule == 2) {
        const unsigned mask = (unsigned)hsize - 1u;
        for (int e = tid; e < W * W; e += 256) {
            const int k = e / W, t = e - k * W;
            const int h = kept[k];
            if (h < 0 || h >= n) continue;
            const int32_t v = G[(int64_t)h * W + t];
            if (v < 0) continue;
            unsigned pos = (2654435761u * (unsigned)v) & mask;
            for (int probe = 0; probe < hsize; ++probe) {
                const int32_t old = atomicCAS(&hs[pos], -1, v);
                if (old == -1 || old == v) break;
                pos = (pos + 1) & mask;
            }
        }
        __syncthreads();
    }
    for (int j = tid; j < C; j += 256) {
        const int32_t c = cd[j];
        bool taken = c < 0 || c == (int32_t)u;
        for (int k = 0; k < W && !taken; ++k) taken = kept[k] == c;
        if (!taken && rule == 2) {
            const unsigned mask = (unsigned)hsize - 1u;
            unsigned pos = (2654435761u * (unsigned)c) & mask;
            for (int probe = 0; probe < hsize; ++probe) {
                const int32_t v = hs[pos];
                if (v == c) { taken = true; break; }
                if (v == -1) break;
                pos = (pos + 1) & mask;
            }
        }
        freeflag[j] = taken ? 0 : 1;
    }
    if (tid == 0) {
        int ne = 0;
        for (int k = 0; k < W; ++k) if (kept[k] < 0) empty[ne++] = k;
        s_nempty = ne;
    }
    __syncthreads();
    if (tid == 0) {
        // free candidates in column order (far: reverse) into the empty slots
        int t = 0;
        const int ne = s_nempty;
        if (rule == 1) {
            for (int j = C - 1; j >= 0 && t < ne; --j)
                if (freeflag[j]) kept[empty[t++]] = cd[j];
        } else {
            for (int j = 0; j < C && t < ne; ++j)
                if (freeflag[j]) kept[empty[t++]] = cd[j];
        }
    }
    __syncthreads();
    for (int k = tid; k < W; k += 256) next[(int64_t)blockIdx.x * W + k] = kept[k];
}

__global__ void copy_rows(const int32_t* __restrict__ src, int64_t count,
                          int32_t* __restrict__ dst) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < count) dst[i] = src[i];
}

// ---------------------------------------------------------------------------
// in-degree floor
__global__ void fill_i32v(int32_t* p, int64_t n, int32_t v) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

__global__ void indeg_count(const int32_t* __restrict__ G, int64_t n, int W,
                            int32_t* __restrict__ indeg) {
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= n * W) return;
    const int v = G[e];
    if (v >= 0 && v < n) atomicAdd(&indeg[v], 1);
}

__global__ void weak_init(const int32_t* __restrict__ indeg, int64_t n, int min_in, int C,
                          int32_t* __restrict__ remaining) {
    const int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (u >= n) return;
    const int need = min_in - indeg[u];
    remaining[u] = need > 0 ? (need < C ? need : C) : 0;
}

// offers of column i: the lowest offering node per target wins
__global__ void mi_offer(const int32_t* __restrict__ G, int64_t n, int W,
                         const int32_t* __restrict__ cand, int C, int i,
                         const int32_t* __restrict__ remaining, int32_t* __restrict__ winner) {
    const int64_t sn = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (sn >= n || remaining[sn] <= 0) return;
    const int32_t t = cand[sn * C + i];
    if (t < 0 || t >= n || t == (int32_t)sn) return;
    const int32_t* row = G + (int64_t)t * W;
    for (int k = 0; k < W; ++k)
        if (row[k] == (int32_t)sn) return;              // already linked
    atomicMin(&winner[t], (int32_t)sn);
}

// a target with a winner gives up its farthest edge whose head stays above
// the floor (never slot 0); decided against the column's starting counts
__global__ void mi_decide(const int32_t* __restrict__ G, int64_t n, int W, int min_in,
                          const int32_t* __restrict__ indeg, int32_t* __restrict__ winner,
                          int32_t* __restrict__ slot_of, int32_t* __restrict__ vflag) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= n || winner[t] == INT32_MAX) return;
    const int32_t* row = G + t * W;
    int slot = -1;
    for (int k = 0; k < W; ++k) {
        const int32_t h = row[k];
        if (h >= 0 && h < n && indeg[h] > min_in) slot = k;
    }
    if (slot < 1) { winner[t] = INT32_MAX; return; }
    slot_of[t] = slot;
    vflag[row[slot]] = 1;                               // several losses count once
}

__global__ void mi_victims(int64_t n, int32_t* __restrict__ indeg, int32_t* __restrict__ vflag) {
    const int64_t v = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (v >= n) return;
    if (vflag[v]) { indeg[v] -= 1; vflag[v] = 0; }
}

__global__ void mi_apply(int32_t* __restrict__ G, int64_t n, int W,
                         int32_t* __restrict__ winner, const int32_t* __restrict__ slot_of,
                         int32_t* __restrict__ indeg, int32_t* __restrict__ remaining) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= n) return;
    const int32_t s = winner[t];
    winner[t] = INT32_MAX;
    if (s == INT32_MAX) return;
    G[t * W + slot_of[t]] = s;
    indeg[s] += 1;                                      // one target per offering node
    remaining[s] -= 1;
}

inline int64_t a256(int64_t b) { return ((b + 255) / 256) * 256; }
inline unsigned blocks_for(int64_t n, int b) { return (unsigned)((n + b - 1) / b); }

}  // namespace
}  // namespace swann

using namespace swann;

extern "C" {

int swann_candidates_from_graph(const void* X, int x_dtype, int64_t n, int dim, int metric,
                                const int32_t* Gc, int gw, int C, int32_t* out_idx,
                                float* out_dist, void* stream) {
    clear_error();
    SWANN_REQUIRE(metric == SWANN_METRIC_IP || metric == SWANN_METRIC_L2,
                  "metric must be 0 (ip) or 1 (l2)");
    SWANN_REQUIRE(x_dtype == SWANN_DTYPE_F32 || x_dtype == SWANN_DTYPE_F16,
                  "X: float32 or float16");
    SWANN_REQUIRE(n >= 1 && n <= INT32_MAX && dim >= 1, "candidates_from_graph: bad shape");
    SWANN_REQUIRE(C >= 1 && C <= gw && C <= kCgMax,
                  "candidates_from_graph: C must be in 1..min(graph width, %d)", kCgMax);
    SWANN_REQUIRE(X && Gc && out_idx && out_dist, "candidates_from_graph: NULL pointer");
    hipStream_t st = (hipStream_t)stream;
    if (x_dtype == SWANN_DTYPE_F32)
        hipLaunchKernelGGL(cand_graph_kernel<float>, dim3((unsigned)n), dim3(256), 0, st,
                           (const float*)X, n, dim, metric, Gc, gw, C, out_idx, out_dist);
    else
        hipLaunchKernelGGL(cand_graph_kernel<_Float16>, dim3((unsigned)n), dim3(256), 0, st,
                           (const _Float16*)X, n, dim, metric, Gc, gw, C, out_idx, out_dist);
    return launch_status("candidates_from_graph");
}

int swann_mutual_rank(const int32_t* cand, int64_t n, int C, int M, uint8_t* out,
                      void* stream) {
    clear_error();
    SWANN_REQUIRE(n >= 1 && C >= 1 && M >= 0, "mutual_rank: bad shape");
    SWANN_REQUIRE(cand && out, "mutual_rank: NULL pointer");
    if (M > C) M = C;
    hipLaunchKernelGGL(mutual_kernel, dim3(blocks_for(n * C, 256)), dim3(256), 0,
                       (hipStream_t)stream, cand, n, C, M, out);
    return launch_status("mutual_rank");
}

int64_t swann_fill_workspace_size(int64_t n, int W, int chunk) {
    const int64_t rows = chunk < n ? chunk : n;
    return a256(rows * (int64_t)W * 4);
}

int swann_fill_degree(const int32_t* G, int64_t n, int W, const int32_t* cand, int C, int rule,
                      int chunk, int32_t* out, void* workspace, void* stream) {
    clear_error();
    SWANN_REQUIRE(rule >= 0 && rule <= 2, "fill: rule must be 0 (near), 1 (far) or 2 (bridge)");
    SWANN_REQUIRE(n >= 1 && n <= INT32_MAX, "fill: n out of range");
    SWANN_REQUIRE(W >= 1 && W <= kFillMaxW, "fill: row width must be in 1..%d", kFillMaxW);
    SWANN_REQUIRE(C >= 1 && C <= kFillMaxC, "fill: candidates per row must be in 1..%d",
                  kFillMaxC);
    SWANN_REQUIRE(chunk >= 1, "fill: chunk must be >= 1");
    SWANN_REQUIRE(G && cand && out && workspace, "fill: NULL pointer");
    hipStream_t st = (hipStream_t)stream;
    int hbits = 1;
    while ((1 << hbits) < 2 * W * W) ++hbits;
    const size_t lds = rule == 2 ? ((size_t)1 << hbits) * 4 : 0;
    SWANN_REQUIRE(lds <= 128 * 1024, "fill: two-hop table does not fit in LDS");
    int32_t* next = (int32_t*)workspace;
    if (out != G)
        hipLaunchKernelGGL(copy_rows, dim3(blocks_for(n * W, 256)), dim3(256), 0, st, G, n * W,
                           out);
    for (int64_t s = 0; s < n; s += chunk) {
        const int64_t e = s + chunk < n ? s + chunk : n;
        hipLaunchKernelGGL(fill_kernel, dim3((unsigned)(e - s)), dim3(256), lds, st, out, n, W,
                           cand, C, rule, s, hbits, next);
        hipLaunchKernelGGL(copy_rows, dim3(blocks_for((e - s) * W, 256)), dim3(256), 0, st, next,
                           (e - s) * W, out + s * W);
    }
    return launch_status("fill_degree");
}

int64_t swann_min_in_workspace_size(int64_t n) { return a256(n * 4) * 5; }

int swann_enforce_min_in(int32_t* G, int64_t n, int W, const int32_t* cand, int C, int min_in,
                         int rounds, void* workspace, void* stream) {
    clear_error();
    SWANN_REQUIRE(n >= 1 && n <= INT32_MAX && W >= 1 && C >= 1, "min_in: bad shape");
    SWANN_REQUIRE(min_in >= 0 && rounds >= 0, "min_in: min_in and rounds must be >= 0");
    SWANN_REQUIRE(G && cand && workspace, "min_in: NULL pointer");
    hipStream_t st = (hipStream_t)stream;
    char* ws = (char*)workspace;
    int32_t* indeg = (int32_t*)ws; ws += a256(n * 4);
    int32_t* remaining = (int32_t*)ws; ws += a256(n * 4);
    int32_t* winner = (int32_t*)ws; ws += a256(n * 4);
    int32_t* slot_of = (int32_t*)ws; ws += a256(n * 4);
    int32_t* vflag = (int32_t*)ws;
    const unsigned nb = blocks_for(n, 256), eb = blocks_for(n * W, 256);
    hipLaunchKernelGGL(fill_i32v, dim3(nb), dim3(256), 0, st, winner, n, INT32_MAX);
    hipLaunchKernelGGL(fill_i32v, dim3(nb), dim3(256), 0, st, vflag, n, 0);
    for (int r = 0; r < rounds; ++r) {
        hipLaunchKernelGGL(fill_i32v, dim3(nb), dim3(256), 0, st, indeg, n, 0);
        hipLaunchKernelGGL(indeg_count, dim3(eb), dim3(256), 0, st, G, n, W, indeg);
        hipLaunchKernelGGL(weak_init, dim3(nb), dim3(256), 0, st, indeg, n, min_in, C, remaining);
        for (int i = 0; i < C; ++i) {
            hipLaunchKernelGGL(mi_offer, dim3(nb), dim3(256), 0, st, G, n, W, cand, C, i,
                               remaining, winner);
            hipLaunchKernelGGL(mi_decide, dim3(nb), dim3(256), 0, st, G, n, W, min_in, indeg,
                               winner, slot_of, vflag);
            hipLaunchKernelGGL(mi_victims, dim3(nb), dim3(256), 0, st, n, indeg, vflag);
            hipLaunchKernelGGL(mi_apply, dim3(nb), dim3(256), 0, st, G, n, W, winner, slot_of,
                               indeg, remaining);
        }
    }
    return launch_status("enforce_min_in");
}

}  // extern "C"
