// Candidate sweep on MFMA: exact top-C neighbours of every row (swann/build.py:28-43)
// as a dense contraction on gfx950 matrix cores with the top-C selection fused
// into the tile epilogue, so the n^2 scores never reach HBM.
//
// Operands are 16-bit rows of X, read K-contiguous for both sides of
// S = X_rows . X_cols^T:
//   * an fp16 corpus is used as is: fp16 x fp16 products are exact in fp32 and
//     accumulate in fp32, so the scores are as good as an fp32 GEMM's;
//   * an fp32 corpus is screened: rows are scaled by a power of two s and
//     rounded once to fp16, s_a s_b (h_a . h_b) ranks the candidates to within
//     ~1e-4 relative, the sweep keeps C + 32 per row, and the caller re-ranks
//     those in fp32 (one gather of C + 32 rows per row, not a second sweep).
// Epilogue per tile: score -> distance by the reference formula, test against
// the row's running threshold (LDS), append survivors to the row's buffer;
// rows near capacity are compacted to their C best (wave-level exact select).
#include <float.h>
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdlib.h>

#include <vector>

#include "common.h"
#include "lanes.h"
#include "panel_order.h"

namespace swann {
namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kBK = 32;
constexpr int kPad = 8;                       // fp16 elements of padding per LDS row
constexpr int kLdsRow = kBK + kPad;           // 40 halves = 80 bytes
constexpr int kBM2 = 256, kBN2 = 256, kT2 = 512;   // workgroup tile rows, columns; threads

// Widest band of the symmetric sweep.  Wider bands mean fewer launches and
// merges but staler column thresholds (more foreign appends); with the
// balanced panel order (sym_panel) the candidate stage at n = 1M took 1.506 s
// (1M x 1024 fp32, l2) and 1.959 s (1M x 1536 fp16, ip) with bands of 256,
// 1.452 s and 1.901 s with 512, and within 1% of that with 640 to 1,024.
constexpr int64_t kBandMax = 512;

__device__ __forceinline__ uint32_t fkey(float f) {
    const uint32_t b = __float_as_uint(f);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float funkey(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

template <int METRIC>
__device__ __forceinline__ float dist_formula(float dot, float na, float nb) {
    if (METRIC == SWANN_METRIC_IP) return 1.0f - dot;
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
        if (lo) lo[r * dim + t] = (_Float16)((v - (float)h) * 2048.0f);
    }
    if (lane == 0) { scale[r] = s; norm[r] = s2; }
}

// The spread of an fp32 corpus's row maxima: rng[0] the largest and rng[1] the
// smallest max |x| of a row, as float bits.  Compared as integers: |x|'s bits
// order as |x| does, and a NaN's bits lie above infinity's, so a row holding
// a NaN reads as NaN, the largest, and fails the caller's range test.  rng
// starts at {0, INT_MAX}.  Each wave takes rows in a grid stride, reading a
// row as 16-byte vectors when vec4 (four in flight a lane, dim % 4 == 0 and
// X 16-byte aligned) and keeping its own extremes: one pair of atomics a
// wave, not a row.
constexpr int kRangeBlocks = 4096;

__global__ __launch_bounds__(256) void row_range(const float* __restrict__ X, int64_t n, int dim,
                                                 int vec4, int* __restrict__ rng) {
    const int lane = threadIdx.x & 63;
    const int64_t w0 = (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t stride = (int64_t)gridDim.x * 4;
    uint32_t hi = 0, lo = 0x7fffffffu;
    for (int64_t r = w0; r < n; r += stride) {
        const float* x = X + r * dim;
        uint32_t m = 0;
        auto take = [&](float v) {
            const uint32_t b = __float_as_uint(v) & 0x7fffffffu;
            m = b > m ? b : m;
        };
        if (vec4) {
            const float4* x4 = reinterpret_cast<const float4*>(x);
            const int d4 = dim >> 2;
            for (int t = lane; t < d4; t += 256) {
                float4 v[4];
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    v[j] = t + 64 * j < d4 ? x4[t + 64 * j] : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
                for (int j = 0; j < 4; ++j) { take(v[j].x); take(v[j].y); take(v[j].z); take(v[j].w); }
            }
        } else {
            for (int t = lane; t < dim; t += 64) take(x[t]);
        }
        m = ~wave_min_u32(~m);
        hi = m > hi ? m : hi;
        lo = m < lo ? m : lo;
    }
    if (lane == 0 && w0 < n) {
        atomicMax(&rng[0], (int)hi);
        atomicMin(&rng[1], (int)lo);
    }
}

__global__ void range_init(int* rng) {
    if (threadIdx.x == 0) { rng[0] = 0; rng[1] = 0x7fffffff; }
}

// An fp32 corpus whose row maxima all lie in [2^-4, 2^14] goes to fp16 as it
// is: fp16 keeps 11 significant bits of every element in its normal range at
// any scale, as the row-scaled plane does, and the sweep then runs its
// unscaled kernel (no per-score scale products).  Norms as split_rows
// computes them (the same order), so the re-rank's are unchanged.
__global__ __launch_bounds__(256) void rows_to_f16(const float* __restrict__ X, int64_t n, int dim,
                                                   _Float16* __restrict__ hi,
                                                   float* __restrict__ norm) {
    const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (r >= n) return;
    const float* x = X + r * dim;
    float s2 = 0.f;
    for (int t = lane; t < dim; t += 64) {
        const float v = x[t];
        s2 = __builtin_fmaf(v, v, s2);
        hi[r * dim + t] = (_Float16)v;
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) s2 += __shfl_xor(s2, off, 64);
    if (lane == 0) norm[r] = s2;
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
    int scaled;                  // rows carry a power-of-two scale (fp32 corpus)
    int splits;                  // column splits G: row r's buffer s is (r * G + s) * cap
    // symmetric (banded) sweep: tiles (I, I + b) for b in [b0, b1), each
    // scored once for both of its panels' rows; splits = 2 lists a row, list 0
    // the row's own (row panel) candidates, list 1 those another workgroup
    // found for it (column panel), with bcnt[2r + 1] a global slot counter
    int sym;
    int64_t b0, b1;
    const float* gthr;           // [n] a row's threshold when the launch began
    int* ovf;                    // foreign appends that found no room
    int fcap;                    // room in list 1 (<= cap; smaller only as a test hook)
    // one-sided sweep of listed row panels only (the repair of rows whose
    // second list overflowed): workgroup g takes panel plist[g / G]
    const int* plist;
    int npl;
    // the pruned ordered sweep: workgroup (panel) I scores only the column
    // tiles tlist[I * kBandMax + k], k < tcnt[I] (ascending, inside its band);
    // a one-sided launch over listed panels (the bounded repair): panel
    // plist[p] scores only tlist[p * tstride + k], k < tcnt[p], ascending,
    // which its G workgroups share out in order
    const int* tlist;
    const int* tcnt;
    // symmetric sweep: each row's list-0 count as the last merge left it; a
    // launch that compacts a row's list sets it to -1, so that the next merge
    // cannot take the row for unchanged (sym_merge)
    int* mcnt;
    int tstride;                 // the bounded repair's list stride (tiles a panel)
};

// Wave-cooperative compaction of one row's buffer to its C best (exact:
// threshold by bitwise search, ties kept in index order).  Every key and id is
// loaded before any is used (lanes past cnt read the last entry and are
// masked; cnt >= 1 here), so a row costs one memory round trip; the search counts with
// ballots and scalar popcounts, no cross-lane shuffles; the kept entries are
// written back from registers (funkey inverts fkey bit for bit).
struct Compacted { uint32_t T; int kept; };     // wave-uniform: the C-th key, entries kept

__device__ __forceinline__ Compacted compact_row_core(float* key, int32_t* id, int cnt, int C) {
    const int lane = threadIdx.x & 63;
    constexpr int R = 16;                      // cap <= 1024
    cnt = __builtin_amdgcn_readfirstlane(cnt);
    // lanes of word t that hold an entry: l < cnt - 64 t
    auto valid = [&](int t) -> uint64_t {
        const int rem = cnt - t * 64;
        return rem >= 64 ? ~0ull : rem <= 0 ? 0ull : ((1ull << rem) - 1);
    };
    uint32_t u[R];
    int32_t v[R];
    float kf[R];
#pragma unroll
    for (int t = 0; t < R; ++t) {           // no branch between the loads
        const int i = min(t * 64 + lane, cnt - 1);
        kf[t] = key[i];
        v[t] = id[i];
    }
#pragma unroll
    for (int t = 0; t < R; ++t) u[t] = fkey(kf[t]);
    // search over the list's own key range; the words past cnt count
    // nothing (their valid mask is 0), so the counting runs without branches
    uint32_t mn = 0xffffffffu, mx = 0;
#pragma unroll
    for (int t = 0; t < R; ++t) {
        const bool in = (valid(t) >> lane) & 1ull;
        mn = in && u[t] < mn ? u[t] : mn;
        mx = in && u[t] > mx ? u[t] : mx;
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const uint32_t x = __shfl_xor(mn, off, 64), y = __shfl_xor(mx, off, 64);
        mn = x < mn ? x : mn;
        mx = y > mx ? y : mx;
    }
    uint32_t lo = __builtin_amdgcn_readfirstlane(mn), hi = __builtin_amdgcn_readfirstlane(mx);
    if (cnt < C) lo = hi = 0xffffffffu;
    while (lo < hi) {
        const uint32_t mid = lo + ((hi - lo) >> 1);
        int c = 0;
#pragma unroll
        for (int t = 0; t < R; ++t) c += __popcll(__ballot(u[t] <= mid) & valid(t));
        if (c >= C) hi = mid; else lo = mid + 1;
    }
    const uint32_t T = lo;
    int nlt = 0;
#pragma unroll
    for (int t = 0; t < R; ++t) nlt += __popcll(__ballot(u[t] < T) & valid(t));
    int eq_left = C - nlt;
    int w = 0;
    const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
#pragma unroll
    for (int t = 0; t < R; ++t) {
        if (t * 64 >= cnt) break;
        const bool in = (valid(t) >> lane) & 1ull;
        const bool is_lt = in && u[t] < T;
        const bool is_eq = in && u[t] == T;
        const uint64_t meq = __ballot(is_eq);
        const int eq_rank = __popcll(meq & below);
        const bool keep = is_lt || (is_eq && eq_rank < eq_left);
        const uint64_t mk = __ballot(keep);
        if (keep) {
            const int dst = w + __popcll(mk & below);
            key[dst] = funkey(u[t]);
            id[dst] = v[t];
        }
        w += __popcll(mk);
        const int used = __popcll(meq);
        eq_left -= used < eq_left ? used : eq_left;
    }
    return Compacted{T, w};
}

__device__ __forceinline__ void compact_row_w(float* key, int32_t* id, int cnt, int C,
                                              float* thr_out, int* cnt_out) {
    const Compacted r = compact_row_core(key, id, cnt, C);
    if ((threadIdx.x & 63) == 0) { *thr_out = funkey(r.T); *cnt_out = r.kept; }
}


// A row's threshold in score space, for the epilogue's first test.  ip keeps
// a score s when 1 - s < thr, so s > (1 - thr) - slack lets every such s
// through (and a few more); l2 keeps when (nb - 2s) + na < thr, so
// s > ((na - thr) - slack) / 2 + (nb - slack') / 2 does.  The slacks are 1e-5
// relative to the magnitudes, far above the rounding of either form, and the
// survivors are then tested exactly.  thr = +inf gives -inf (every finite
// score passes); a row past n (thr = -inf) gives +inf or NaN (none passes).
template <int METRIC>
__device__ __forceinline__ float screen_thr(float thr, float na) {
    if (METRIC == SWANN_METRIC_IP) return (1.0f - thr) - 1e-5f * (1.0f + fabsf(thr));
    return 0.5f * ((na - thr) - 1e-5f * (fabsf(na) + fabsf(thr)));
}

// Epilogue for one 32 x 32 accumulator block: lane holds column c and the 16
// rows rbase + (e/4)*8 + (e%4).  The common case -- no score of the block
// beats its row's threshold -- costs the distance formula and one compare per
// score, the "any" kept as a lane mask, one row group (4 rows: threshold,
// norms, scales) live at a time; only a block with a survivor recomputes its
// distances from fresh LDS reads and appends.  Rows past n carry a -inf
// threshold, so they never pass.  Self scores were set to -inf in the
// accumulator (self_out), so their distance is +inf and never passes; the
// merge adds self back at 3.4e38 where a row has fewer than C others.
// The survivors of one block for their rows' own buffers: each distance
// recomputed exactly from fresh LDS reads and appended to its row's buffer.
// Called by the lanes whose screen passed, once the wave's ballot has shown
// that some did.
template <int METRIC>
__device__ __forceinline__ void append_own(const f32x16& v, int rbase, int64_t r0, int64_t c,
                                           float cn, float sc, const float* rs, const float* thr,
                                           const float* rnorm, int* cnt, const MfmaSweepArgs& a,
                                           int split, int nterm_scale, const f32x16* vx,
                                           int* needf, bool cok = true) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        const float4 t4 = *reinterpret_cast<const float4*>(thr + rbase + g * 8);
        const float4 r4 = METRIC == SWANN_METRIC_L2
                              ? *reinterpret_cast<const float4*>(rnorm + rbase + g * 8)
                              : make_float4(0.f, 0.f, 0.f, 0.f);
        const float4 s4 = nterm_scale ? *reinterpret_cast<const float4*>(rs + rbase + g * 8)
                                      : make_float4(1.f, 1.f, 1.f, 1.f);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int e = g * 4 + q;
            float dot;
            if (nterm_scale == 1)
                dot = s4[q] * sc * (v[e] + (*vx)[e] * (1.0f / 2048.0f));
            else if (nterm_scale == 2)
                dot = s4[q] * sc * v[e];
            else
                dot = v[e];
            if (!cok) continue;
            const float d = dist_formula<METRIC>(dot, METRIC == SWANN_METRIC_L2 ? r4[q] : 0.f, cn);
            if (!(d < t4[q])) continue;
            const int rl = rbase + g * 8 + q;
            const int p = atomicAdd(&cnt[rl], 1);
            // the append that leaves less than a tile of room flags a compaction
            if (needf && p == a.cap - kBN2) *needf = 1;
            const int64_t o = ((r0 + rl) * a.splits + split) * (int64_t)a.cap + p;
            a.bkey[o] = d;
            a.bid[o] = (int32_t)c;
        }
    }
}

template <int METRIC>
__device__ __forceinline__ void epilogue_block(const f32x16& v, int rbase, int64_t r0, int64_t c,
                                               bool cok, float cn, float sc, const float* rs,
                                               const float* thr, const float* rnorm, int* cnt,
                                               const MfmaSweepArgs& a, int split, int nterm_scale,
                                               const f32x16* vx, int* needf = nullptr,
                                               const float* sthr = nullptr) {
    auto dist = [&](int e, const float4& r4, const float4& s4) {
        const int q = e & 3;
        float dot;
        if (nterm_scale == 1)
            dot = s4[q] * sc * (v[e] + (*vx)[e] * (1.0f / 2048.0f));
        else if (nterm_scale == 2)
            dot = s4[q] * sc * v[e];
        else
            dot = v[e];
        return dist_formula<METRIC>(dot, METRIC == SWANN_METRIC_L2 ? r4[q] : 0.f, cn);
    };
    auto group = [&](int g, float4& t4, float4& r4, float4& s4) {
        t4 = *reinterpret_cast<const float4*>(thr + rbase + g * 8);
        r4 = METRIC == SWANN_METRIC_L2 ? *reinterpret_cast<const float4*>(rnorm + rbase + g * 8)
                                       : make_float4(0.f, 0.f, 0.f, 0.f);
        s4 = nterm_scale ? *reinterpret_cast<const float4*>(rs + rbase + g * 8)
                         : make_float4(1.f, 1.f, 1.f, 1.f);
    };
    bool any = false;
    if (sthr && nterm_scale != 1) {
        // one compare per score against the row's screen threshold
        const float ch = METRIC == SWANN_METRIC_L2 ? 0.5f * (cn - 1e-5f * fabsf(cn)) : 0.f;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const float4 h4 = *reinterpret_cast<const float4*>(sthr + rbase + g * 8);
            const float4 s4 = nterm_scale ? *reinterpret_cast<const float4*>(rs + rbase + g * 8)
                                          : make_float4(1.f, 1.f, 1.f, 1.f);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float dot = nterm_scale ? s4[q] * sc * v[g * 4 + q] : v[g * 4 + q];
                any = any || (METRIC == SWANN_METRIC_IP ? dot > h4[q] : dot > ch + h4[q]);
            }
        }
    } else {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            float4 t4, r4, s4;
            group(g, t4, r4, s4);
#pragma unroll
            for (int q = 0; q < 4; ++q) any = any || (dist(g * 4 + q, r4, s4) < t4[q]);
        }
    }
    any = any && cok;
    if (__ballot(any) == 0ull) return;
    asm volatile("" ::: "memory");           // rare path: reload rather than keep live
    if (!any) return;
    append_own<METRIC>(v, rbase, r0, c, cn, sc, rs, thr, rnorm, cnt, a, split, nterm_scale, vx,
                       needf);
}

// The foreign half of a tile's epilogue in the symmetric sweep: the same 32 x
// 32 block scored for the column panel's rows.  Lane holds column c -- a row
// of the column panel, whose threshold `thc` came from the last merge -- and
// its 16 candidates rbase + (e/4)*8 + (e%4) of the row panel.  Row c's
// distance to candidate r is the reference formula with the roles swapped
// (na = |c|^2, nb = |r|^2), from the same score.  Survivors of the screen
// (screen_pair) take a slot of row c's second list from its global counter.
// Candidates past n are copies of row n - 1 (the panel loads clamp) and are
// skipped.
template <int METRIC>
__device__ __forceinline__ void append_foreign(const f32x16& v, int rbase, int64_t r0,
                                               int64_t c, float cn, float sc, float thc,
                                               const float* rs, const float* rnorm,
                                               const MfmaSweepArgs& a, int scaled, bool cok) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        const float4 s4 = scaled ? *reinterpret_cast<const float4*>(rs + rbase + g * 8)
                                 : make_float4(1.f, 1.f, 1.f, 1.f);
        const float4 r4 = METRIC == SWANN_METRIC_L2
                              ? *reinterpret_cast<const float4*>(rnorm + rbase + g * 8)
                              : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float dot = scaled ? s4[q] * sc * v[g * 4 + q] : v[g * 4 + q];
            if (!cok) continue;
            const float d = dist_formula<METRIC>(dot, cn, r4[q]);
            const int64_t r = r0 + rbase + g * 8 + q;
            if (!(d < thc) || r >= a.n) continue;
            const int p = atomicAdd(&a.bcnt[c * 2 + 1], 1);
            if (p < a.fcap) {
                const int64_t o = (c * 2 + 1) * (int64_t)a.cap + p;
                a.bkey[o] = d;
                a.bid[o] = (int32_t)r;
            } else {
                atomicAdd(a.ovf, 1);
            }
        }
    }
}

// Foreign survivors queued in LDS instead of taking their global slots at
// once: a slot is a returning atomic on row c's counter, and a wave that
// waits for it (vmcnt) stalls for a memory round trip per survivor.  The
// queue (column and row within the tile, distance) is drained at the next
// column tile's first stage, where each thread takes one entry's slot with
// an atomic whose return is waited for by that stage's own barrier, and the
// entries are stored at the second stage.  A full queue takes the direct
// path.
constexpr int kFQueue = 1024;

template <int METRIC>
__device__ __forceinline__ void queue_foreign(const f32x16& v, int rbase, int64_t r0, int64_t c,
                                              int cl, float cn, float sc, float thc,
                                              const float* rs, const float* rnorm,
                                              const MfmaSweepArgs& a, int scaled, int* qn,
                                              int2* qe, bool cok) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        const float4 s4 = scaled ? *reinterpret_cast<const float4*>(rs + rbase + g * 8)
                                 : make_float4(1.f, 1.f, 1.f, 1.f);
        const float4 r4 = METRIC == SWANN_METRIC_L2
                              ? *reinterpret_cast<const float4*>(rnorm + rbase + g * 8)
                              : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float dot = scaled ? s4[q] * sc * v[g * 4 + q] : v[g * 4 + q];
            if (!cok) continue;
            const float d = dist_formula<METRIC>(dot, cn, r4[q]);
            const int rl = rbase + g * 8 + q;
            if (!(d < thc) || r0 + rl >= a.n) continue;
            const int k = atomicAdd(qn, 1);
            if (k < kFQueue) {
                qe[k] = make_int2((cl << 16) | rl, __float_as_int(d));
            } else {
                const int p = atomicAdd(&a.bcnt[c * 2 + 1], 1);
                if (p < a.fcap) {
                    const int64_t o = (c * 2 + 1) * (int64_t)a.cap + p;
                    a.bkey[o] = d;
                    a.bid[o] = (int32_t)(r0 + rl);
                } else {
                    atomicAdd(a.ovf, 1);
                }
            }
        }
    }
}

// Both screens of a block of the DMA sweep in one pass, as wave masks: each
// score is scaled once, then tested for its row's own buffer and, when `fon`
// (the symmetric sweep off the diagonal), for its column's foreign list.
// The tests are in score space, one compare each after at most one add: the
// row's own threshold sthr (screen_thr) plus, for l2, the column's half-norm
// term ch; the column's threshold h (screen_thr of thc) plus, for l2, the
// row's half-norm term fr = (|r|^2 - 1e-5 ||r|^2|) / 2.  Each compare goes
// straight into a 64-bit lane mask (a ballot), so the "any" costs no VALU.
// Both keep at least what the exact tests of the append paths keep.
template <int METRIC, int SCALED>
__device__ __forceinline__ void screen_pair(const f32x16& v, int rbase, float cn, float sc,
                                            float thc, bool fon, const float* rs,
                                            const float* sthr, const float* fr, uint64_t& own,
                                            uint64_t& frn) {
    const float ch = METRIC == SWANN_METRIC_L2 ? 0.5f * (cn - 1e-5f * fabsf(cn)) : 0.f;
    const float h = screen_thr<METRIC>(thc, cn);
    uint64_t o = 0, f = 0;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        const float4 s4 = SCALED ? *reinterpret_cast<const float4*>(rs + rbase + g * 8)
                                 : make_float4(1.f, 1.f, 1.f, 1.f);
        const float4 t4 = *reinterpret_cast<const float4*>(sthr + rbase + g * 8);
        if (fon) {
            const float4 f4 = METRIC == SWANN_METRIC_L2
                                  ? *reinterpret_cast<const float4*>(fr + rbase + g * 8)
                                  : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float dot = SCALED ? s4[q] * sc * v[g * 4 + q] : v[g * 4 + q];
                o |= __ballot(METRIC == SWANN_METRIC_L2 ? dot > ch + t4[q] : dot > t4[q]);
                f |= __ballot(METRIC == SWANN_METRIC_L2 ? dot > h + f4[q] : dot > h);
            }
        } else {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float dot = SCALED ? s4[q] * sc * v[g * 4 + q] : v[g * 4 + q];
                o |= __ballot(METRIC == SWANN_METRIC_L2 ? dot > ch + t4[q] : dot > t4[q]);
            }
        }
    }
    own = o;
    frn = f;
}

// On the diagonal tile, the score of each row against itself becomes -inf
// (its distance +inf), so the epilogue never takes it.  Lane holds column
// ccol (offset in the tile) and rows rbase + (e/4)*8 + (e%4).
__device__ __forceinline__ void self_out(f32x16& v, int rbase, int ccol) {
#pragma unroll
    for (int e = 0; e < 16; ++e)
        if (ccol == rbase + (e >> 2) * 8 + (e & 3)) v[e] = -INFINITY;
}

// ---------------------------------------------------------------------------
// fp16 operands (NTERM = 1): workgroup tile 256 x 256 with eight waves of
// 128 x 64 (4 x 2 blocks of 32 x 32; 128 accumulators each), so two waves share
// a SIMD and one's epilogue or wait overlaps the other's MFMAs.  K tile 32.  The
// workgroup's work is one stream of (column tile, K tile) steps: global loads
// run two steps ahead in two register stages, LDS is double-buffered with one
// barrier per step, and a column tile's epilogue overlaps the next tile's loads.

struct Stage { f16x8 a[2], b[2]; };

template <int METRIC, int SCALED>
__global__ __launch_bounds__(512, 1) void sweep_mfma256_kernel(MfmaSweepArgs a) {
    __shared__ __align__(16) _Float16 sA[2][kBM2 * kLdsRow];
    __shared__ __align__(16) _Float16 sB[2][kBN2 * kLdsRow];
    __shared__ __align__(16) float thr[kBM2];
    __shared__ int cnt[kBM2];
    __shared__ __align__(16) float rnorm[kBM2];
    __shared__ __align__(16) float rscale[kBM2];
    __shared__ int need;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 2, wn = wave & 3;           // rows wm*128.., cols wn*64..
    const int64_t n = a.n;
    const int dim = a.dim;
    const int64_t ntile = (n + kBM2 - 1) / kBM2;
    const int64_t r0 = xcd_remap(blockIdx.x, ntile) * kBM2;

    if (tid < kBM2) {
        thr[tid] = r0 + tid < n ? INFINITY : -INFINITY;
        cnt[tid] = 0;
        rnorm[tid] = (r0 + tid < n) ? a.xn[r0 + tid] : 0.f;
        if (SCALED) rscale[tid] = (r0 + tid < n) ? a.scale[r0 + tid] : 1.f;
    }
    if (tid == 0) need = 0;

    // loader: 256 rows x 4 chunks of 16 B per operand = 2 chunks per thread each
    int lrow[2], lpart[2];
    int64_t aoff[2];
    bool av[2];
#pragma unroll
    for (int m = 0; m < 2; ++m) {
        const int c = tid + kT2 * m;
        lrow[m] = c >> 2;
        lpart[m] = (c & 3) * 8;
        av[m] = r0 + lrow[m] < n;
        aoff[m] = (av[m] ? r0 + lrow[m] : n - 1) * (int64_t)dim + lpart[m];
    }
    const int nk = (dim + kBK - 1) / kBK;
    const int64_t nct = (n + kBN2 - 1) / kBN2;
    const int64_t nsteps = nct * nk;

    auto gload = [&](Stage& S, int64_t t, int kt, int64_t cb) {
        const f16x8 z = {};
        if (t >= nsteps) return;
        const int k0 = kt * kBK;
        const bool kfull = k0 + kBK <= dim;
#pragma unroll
        for (int m = 0; m < 2; ++m) {
            const int64_t rb = cb + lrow[m];
            const bool bv = rb < n;
            const bool kin = kfull || (k0 + lpart[m] < dim);
            const int64_t boff = (bv ? rb : n - 1) * (int64_t)dim + lpart[m];
            const int kk = kin ? k0 : 0;                // never read past a row
            const f16x8 va = *reinterpret_cast<const f16x8*>(a.hi + aoff[m] + kk);
            const f16x8 vb = *reinterpret_cast<const f16x8*>(a.hi + boff + kk);
            S.a[m] = (av[m] && kin) ? va : z;
            S.b[m] = (bv && kin) ? vb : z;
        }
    };
    auto lstore = [&](const Stage& S, int buf) {
#pragma unroll
        for (int m = 0; m < 2; ++m) {
            *reinterpret_cast<f16x8*>(&sA[buf][lrow[m] * kLdsRow + lpart[m]]) = S.a[m];
            *reinterpret_cast<f16x8*>(&sB[buf][lrow[m] * kLdsRow + lpart[m]]) = S.b[m];
        }
    };

    // (kt, cb) of the current step and of the step three ahead, kept by
    // increments: no 64-bit division per step
    int kt_c = 0, kt_f = 0;
    int64_t cb_c = 0, cb_f = 0;
    auto adv = [&](int& kt, int64_t& cb) {
        if (++kt == nk) { kt = 0; cb += kBN2; }
    };
    f32x16 acc[4][2];
    Stage S0, S1;
    gload(S0, 0, kt_f, cb_f); adv(kt_f, cb_f);
    gload(S1, 1, kt_f, cb_f); adv(kt_f, cb_f);
    lstore(S0, 0);
    gload(S0, 2, kt_f, cb_f); adv(kt_f, cb_f);
    __syncthreads();

    auto step = [&](int64_t t, Stage& Snext) {
        const int kt = kt_c;
        const int64_t cbt = cb_c;
        adv(kt_c, cb_c);
        const int buf = (int)(t & 1);
        if (kt == 0) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) acc[i][j] = (f32x16){};
        }
        // column norms of this tile, loaded before the next steps' prefetch so
        // the epilogue never waits on it
        float cn[2] = {0.f, 0.f}, cs[2] = {1.f, 1.f};
        if (kt == nk - 1) {
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int64_t c = cbt + wn * 64 + j * 32 + (lane & 31);
                if (METRIC == SWANN_METRIC_L2) cn[j] = c < n ? a.xn[c] : 0.f;
                if (SCALED) cs[j] = c < n ? a.scale[c] : 1.f;
            }
        }
#pragma unroll
        for (int ks = 0; ks < kBK; ks += 16) {
            const int kof = ks + (lane >> 5) * 8;
            f16x8 fa[4], fb[2];
#pragma unroll
            for (int i = 0; i < 4; ++i)
                fa[i] = *reinterpret_cast<const f16x8*>(
                    &sA[buf][(wm * 128 + i * 32 + (lane & 31)) * kLdsRow + kof]);
#pragma unroll
            for (int j = 0; j < 2; ++j)
                fb[j] = *reinterpret_cast<const f16x8*>(
                    &sB[buf][(wn * 64 + j * 32 + (lane & 31)) * kLdsRow + kof]);
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[i], fb[j], acc[i][j],
                                                                      0, 0, 0);
        }
        if (t + 1 < nsteps) lstore(Snext, buf ^ 1);
        gload(Snext, t + 3, kt_f, cb_f);
        adv(kt_f, cb_f);
        if (kt == nk - 1) {
            // ---- epilogue of this column tile: distance, threshold, append ----
            const int64_t cb = cbt;
            const bool diag = (cb == r0);
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int64_t c = cb + wn * 64 + j * 32 + (lane & 31);
                const bool cok = c < n;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    int rbase = wm * 128 + i * 32 + (lane >> 5) * 4;
                    asm volatile("" : "+v"(rbase));
                    if (diag) self_out(acc[i][j], rbase, wn * 64 + j * 32 + (lane & 31));
                    epilogue_block<METRIC>(acc[i][j], rbase, r0, c, cok, cn[j], cs[j], rscale,
                                           thr, rnorm, cnt, a, 0, SCALED ? 2 : 0, nullptr);
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
            __syncthreads();
            if (tid < kBM2 && cnt[tid] > a.cap - kBN2) atomicOr(&need, 1);
            __syncthreads();
            if (need) {
                for (int rl = wave; rl < kBM2; rl += kT2 / 64) {
                    const int64_t r = r0 + rl;
                    if (r < n && cnt[rl] > a.cap - kBN2)
                        compact_row_w(a.bkey + r * a.splits * a.cap, a.bid + r * a.splits * a.cap, cnt[rl], a.C,
                                      &thr[rl], &cnt[rl]);
                }
                __syncthreads();
                if (tid == 0) need = 0;
            }
        }
        __syncthreads();
    };
    for (int64_t t = 0; t < nsteps; t += 2) {
        step(t, S1);
        if (t + 1 < nsteps) step(t + 1, S0);
    }
    if (tid < kBM2 && r0 + tid < n) a.bcnt[(r0 + tid) * a.splits] = cnt[tid];
}

// ---------------------------------------------------------------------------
// dim % 64 == 0: the same 256 x 256 workgroup tile and 128 x 64 wave tiles,
// with the operands moved global -> LDS by the gfx950 direct load
// (global_load_lds_dwordx4: lane i's 16 bytes land at the wave-uniform base
// + 16 i), so no registers stage them.  K stage 64 (128 bytes of a row), two
// LDS buffers of 64 KB: the load of stage t + 1 is issued right after the
// barrier that opens stage t and lands while stage t computes.  Inside a
// stage the four 16-wide substeps double-buffer their fragments in
// registers, so LDS reads overlap MFMAs; one barrier per 32 MFMAs per wave.
//
// LDS layout: row-major, 128 bytes per row per stage, with the eight 16-byte
// chunks of row r stored at chunk (c ^ swz(r)), swz(r) = (r & 7) ^ ((r >> 3) & 1):
// a fragment read (32 consecutive rows, one logical chunk) touches eight
// distinct chunk positions in every group of 8 rows and in every group of 16
// rows of either parity, so it is free of bank conflicts.  Each direct-load
// instruction fills 1 KB = 8 rows; lane i fetches row 8q + i/8, logical chunk
// (i % 8) ^ swz(row), which lands at physical chunk i % 8.
constexpr int kBK3 = 64;
constexpr int kRowBytes = kBK3 * 2;
constexpr int kStage = kBM2 * kRowBytes;           // 32 KB per operand per stage

typedef __attribute__((address_space(3))) void* lds_vptr;

__device__ __forceinline__ int swz(int r) { return (r & 7) ^ ((r >> 3) & 1); }

// One wave-wide direct load global -> LDS of 16 bytes a lane: lane i's 16
// bytes at base + voff (a wave-uniform base, a 32-bit byte offset per lane)
// land at lds + 16 i.  Written as assembly so that the compiler does not
// track it: it cannot tell the stage being read from the stage being filled
// (they alternate at run time), and would make every fragment read wait for
// the loads in flight.  The kernel waits for them itself: vmcnt(0) and a
// barrier before a stage is read.  m0 carries the LDS address: an input
// operand, so the compiler writes m0 and knows it holds this value.
// The compiler does not see into the assembly, so it does not pad the
// hazards of its operands: a VMEM instruction that reads an SGPR a VALU
// instruction wrote (v_readlane restoring a spilled base) needs 5 wait
// states, and one that reads m0 after an SALU write 1.  The s_nop 4 gives
// both: with one wait state only, a base restored by v_readlane the
// instruction before was read stale, and the load went to a wild address.
__device__ __forceinline__ void dma16(const void* base, uint32_t voff, unsigned char* lds) {
    const unsigned m = (unsigned)(uintptr_t)(lds_vptr)lds;
    asm volatile("s_nop 4\n\tglobal_load_lds_dwordx4 %0, %1"
                 :: "v"(voff), "s"(base), "{m0}"(m) : "memory");
}

// The same for 4 bytes a lane: lane i's word lands at lds + 4 i.
__device__ __forceinline__ void dma4(const void* base, uint32_t voff, unsigned char* lds) {
    const unsigned m = (unsigned)(uintptr_t)(lds_vptr)lds;
    asm volatile("s_nop 4\n\tglobal_load_lds_dword %0, %1"
                 :: "v"(voff), "s"(base), "{m0}"(m) : "memory");
}

// WAVES = 8: two waves per SIMD with 128 x 64 wave tiles (128 accumulators);
// WAVES = 16: four waves per SIMD with 64 x 64 wave tiles (64 accumulators),
// which leaves the registers to keep fragment reads ahead of their MFMAs and
// twice the waves to cover one another's LDS and barrier waits.
template <int METRIC, int SCALED, int WAVES>
__global__ __launch_bounds__(WAVES * 64, 1) void sweep_dma_kernel(MfmaSweepArgs a) {
    constexpr int WR = WAVES == 16 ? 4 : 2;    // waves down the 256 rows
    constexpr int WN = WAVES / WR;             // waves across the 256 columns
    constexpr int RW = kBM2 / WR, CW = kBN2 / WN;   // wave tile
    constexpr int BI = RW / 32, BJ = CW / 32;  // 32 x 32 blocks per wave
    constexpr int NQ = 32 / WAVES;             // 1 KB direct loads per wave per operand
    __shared__ __align__(16) unsigned char sA[2][kStage];
    __shared__ __align__(16) unsigned char sB[2][kStage];
    __shared__ __align__(16) float thr[kBM2];
    // thr in score space (screen_thr), kept beside thr: the screens compare
    // scores with it, and only survivors evaluate the distance formula
    __shared__ __align__(16) float sthr[kBM2];
    __shared__ __align__(16) float frow[kBM2];   // l2: the foreign screen's row term
    __shared__ int cnt[kBM2];
    __shared__ __align__(16) float rnorm[kBM2];
    __shared__ __align__(16) float rscale[kBM2];
    __shared__ int need[2];      // set by the appends of column tiles of that parity
    // symmetric sweep: the current column tile's rows' thresholds (from the
    // last merge, fixed for the launch), for the foreign half of its epilogue
    __shared__ __align__(16) float thrc[kBN2];
    // symmetric sweep: foreign survivors waiting for their slots (queue_foreign)
    __shared__ int fqn;
    __shared__ int2 fq[kFQueue];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WN, wn = wave % WN;          // rows wm*RW.., cols wn*CW..
    // Row and tile indices are 32-bit (the entry point bounds n by
    // INT32_MAX / 2); only addresses are formed in 64 bits.  Held in 64-bit
    // scalar pairs they overflowed the SGPRs into VGPR lanes.
    const int n = (int)a.n;
    const int dim = a.dim;
    const int ntile = (n + kBM2 - 1) / kBM2;
    // G workgroups share a row panel, each taking 1/G of the column tiles;
    // xcd_remap gives consecutive logical ids to one XCD, so the G readers of
    // a panel run together on one L2
    const int G = a.splits;
    // symmetric sweep: one workgroup per row panel, which keeps list 0 of
    // its rows and starts from the thresholds and lists the last merge left;
    // sym_panel spreads the band's short panels over the XCDs
    const int lid = a.sym ? sym_panel((int)blockIdx.x, (int)gridDim.x, (int)(a.b1 - a.b0))
                          : (int)xcd_remap(blockIdx.x, (int64_t)(a.plist ? a.npl : ntile) * G);
    const int r0 = (a.sym ? lid : a.plist ? a.plist[lid / G] : lid / G) * kBM2;
    const int split = a.sym ? 0 : lid % G;

    if (tid < kBM2) {
        thr[tid] = r0 + tid >= n ? -INFINITY : a.sym ? a.gthr[r0 + tid] : INFINITY;
        cnt[tid] = (a.sym && r0 + tid < n) ? a.bcnt[(int64_t)(r0 + tid) * 2] : 0;
        rnorm[tid] = (r0 + tid < n) ? a.xn[r0 + tid] : 0.f;
        if (SCALED) rscale[tid] = (r0 + tid < n) ? a.scale[r0 + tid] : 1.f;
        sthr[tid] = screen_thr<METRIC>(thr[tid], rnorm[tid]);
        if (METRIC == SWANN_METRIC_L2) frow[tid] = 0.5f * (rnorm[tid] - 1e-5f * fabsf(rnorm[tid]));
    }
    if (tid < 2) need[tid] = 0;
    if (tid == 0) fqn = 0;

    // direct-load assignment: instruction j of this wave fills rows
    // 8 (NQ wave + j) .. + 7 of the stage; this lane fetches one 16-byte
    // chunk, at byte offset lrow * rowb + chunk from the stage's first row
    // (rows past n read row n - 1: the panel and the last column tile clamp)
    const uint32_t rowb = (uint32_t)dim * 2;
    const int nk = dim / kBK3;
    const int nct = (n + kBN2 - 1) / kBN2;
    int ct0 = (int)((int64_t)nct * split / G), ct1 = (int)((int64_t)nct * (split + 1) / G);
    if (a.sym) {
        ct0 = lid + (int)a.b0;
        ct1 = lid + a.b1 < nct ? lid + (int)a.b1 : nct;
    }
    // with a tile list the column tiles are a listed subset, in order: in a
    // symmetric launch (the pruned ordered sweep) panel lid's, inside its
    // band; in a one-sided launch over listed panels (the bounded repair)
    // this workgroup's share of panel plist[lid / G]'s list
    const int* tls = nullptr;
    int ntl = ct1 - ct0;
    if (a.tlist && a.sym) {
        tls = a.tlist + (int64_t)lid * kBandMax;
        ntl = a.tcnt[lid];
    } else if (a.tlist && a.plist) {
        const int p = lid / G, m = a.tcnt[p];
        const int k0 = (int)((int64_t)m * split / G), k1 = (int)((int64_t)m * (split + 1) / G);
        tls = a.tlist + (int64_t)p * a.tstride + k0;
        ntl = k1 - k0;
    }
    const int nsteps = ntl * nk;
    const _Float16* X = a.hi;

    auto issue = [&](int t, int kt, int cb) {
        if (t >= nsteps) return;
        const int buf = t & 1;
        const int k0 = kt * kBK3;
        const _Float16* ba = X + (int64_t)r0 * dim + k0;
        const _Float16* bb = X + (int64_t)cb * dim + k0;
        // The lane offsets are recomputed at every issue (a few VALU) rather
        // than held across the loop: held, they are the first registers the
        // allocator spills, and each reload's wait (vmcnt counts scratch
        // loads and direct loads alike) then waited for the direct load
        // issued just before it, a memory latency per instruction.
        int ln = lane;
        asm volatile("" : "+v"(ln));
#pragma unroll
        for (int j = 0; j < NQ; ++j) {
            const int q = wave * NQ + j;
            const int lrow = q * 8 + (ln >> 3);
            const uint32_t lb = (uint32_t)(((ln & 7) ^ swz(lrow)) * 16);
            const uint32_t ra = r0 + lrow < n ? (uint32_t)lrow : (uint32_t)(n - 1 - r0);
            const uint32_t rb = cb + lrow < n ? (uint32_t)lrow : (uint32_t)(n - 1 - cb);
            dma16(ba, ra * rowb + lb, &sA[buf][q * 1024]);
            dma16(bb, rb * rowb + lb, &sB[buf][q * 1024]);
        }
    };

    // fragment addresses: row r's logical chunk c sits at r*128 + ((c ^ swz(r)) * 16);
    // the fragment rows are (multiple of 32) + lane % 32, so swz is per lane
    const int fsw = swz(lane & 31);
    int aro[BI], bro[BJ];
#pragma unroll
    for (int i = 0; i < BI; ++i) aro[i] = (wm * RW + i * 32 + (lane & 31)) * kRowBytes;
#pragma unroll
    for (int j = 0; j < BJ; ++j) bro[j] = (wn * CW + j * 32 + (lane & 31)) * kRowBytes;

    // wave-uniform (the list entry is the same for every lane): the direct
    // loads take the tile's base address in scalar registers.
    // A full band of a symmetric launch (column tiles ct0 .. ct0 + bw - 1,
    // one of each residue mod bw) is taken in residue order: step k scores
    // the tile J == k (mod bw).  The workgroups an XCD runs together hold
    // consecutive panels (sym_panel), so at every step they read one column
    // panel, or two where the residue wraps, and all but the first find its
    // lines in L2; in the order ct0 + k, neighbours read the same panel one
    // tile apart, long after L2 has dropped it.  The lists do not depend on
    // the order.
    const int bw = a.sym ? (int)(a.b1 - a.b0) : 0;
    const bool rot = a.sym && !tls && bw > 1 && ntl == bw;
    const int cmod = rot ? ct0 % bw : 0;
    auto tile_at = [&](int k) {
        if (tls) return __builtin_amdgcn_readfirstlane(tls[k]);
        if (rot) return ct0 + (k >= cmod ? k - cmod : k - cmod + bw);
        return ct0 + k;
    };
    int kt_c = 0, kt_f = 0, ki_c = 0, ki_f = 0;
    int cb_c = ntl > 0 ? tile_at(0) * kBN2 : 0, cb_f = cb_c;
    auto adv = [&](int& kt, int& ki, int& cb) {
        if (++kt == nk) {
            kt = 0;
            if (++ki < ntl) cb = tile_at(ki) * kBN2;
        }
    };
    f32x16 acc[BI][BJ];
    // the foreign queue: staged when a tile has at least three stages, so
    // that its drain (first stage) and stores (second) come before the next
    // epilogue (last stage) refills it
    const bool fstage = a.sym && nk >= 3;
    int fslot = 0, fqd = 0;          // this thread's drained entry: its slot; entries drained
    int cb_prev = 0;                 // column base of the tile whose entries are queued
    int tpar = 0;                    // parity of the current column tile (its need flag)
    issue(0, kt_f, cb_f);
    adv(kt_f, ki_f, cb_f);

    for (int t = 0; t < nsteps; ++t) {
        const int kt = kt_c;
        const int cbt = cb_c;
        adv(kt_c, ki_c, cb_c);
        const int buf = t & 1;
        // column norms/scales of a finishing tile, issued before the next
        // stage's loads so the epilogue's wait does not include them
        float cn[BJ], cs[BJ];
#pragma unroll
        for (int j = 0; j < BJ; ++j) { cn[j] = 0.f; cs[j] = 1.f; }
        if (kt == nk - 1) {
#pragma unroll
            for (int j = 0; j < BJ; ++j) {
                const int c = cbt + wn * CW + j * 32 + (lane & 31);
                if (METRIC == SWANN_METRIC_L2) cn[j] = c < n ? a.xn[c] : 0.f;
                if (SCALED) cs[j] = c < n ? a.scale[c] : 1.f;
            }
        }
        __builtin_amdgcn_s_waitcnt(0x0F70);             // vmcnt(0): this wave's stage-t loads
        __syncthreads();                                // every wave's stage-t loads have landed
        // Everything a stage does before its MFMAs that may wait on memory
        // (the queue's slot atomics, the compaction, the column thresholds)
        // comes before the next stage's direct loads are issued, so that no
        // wait of its own -- the compiler's vmcnt for a spill or a load --
        // also waits for those.
        if (fstage && kt == 0) {
            // take the slots of the last tile's queued foreign survivors; the
            // returns are waited for by the next stage's barrier
            fqd = fqn < kFQueue ? fqn : kFQueue;
            if (tid < fqd) {
                const int2 e = fq[tid];
                fslot = atomicAdd(&a.bcnt[(int64_t)(cb_prev + (e.x >> 16)) * 2 + 1], 1);
            }
        }
        if (fstage && kt == 1) {
            if (tid < fqd) {
                const int2 e = fq[tid];
                const int64_t c = cb_prev + (e.x >> 16);
                if (fslot < a.fcap) {
                    const int64_t o = (c * 2 + 1) * (int64_t)a.cap + fslot;
                    a.bkey[o] = __int_as_float(e.y);
                    a.bid[o] = (int32_t)(r0 + (e.x & 0xffff));
                } else {
                    atomicAdd(a.ovf, 1);
                }
            }
            if (tid == 0) fqn = 0;      // the next refill is after the next barrier
            fqd = 0;
        }
        if (kt == 0) {
          if (t > 0) {
            // compaction flagged by the previous column tile's appends; the
            // flag was set before the barrier above, so every wave reads the
            // same value, and it is cleared only after every wave has read it.
            // The accumulators are dead here (the tile's epilogue used them,
            // and they are zeroed at the end of this branch, where the
            // compiler can see it), so the compaction may use their registers.
            const int par = tpar ^ 1;    // the tile that just ended
            if (need[par]) {
                for (int rl = wave; rl < kBM2; rl += WAVES) {
                    const int64_t r = r0 + rl;
                    if (r < n && cnt[rl] > a.cap - kBN2) {
                        compact_row_w(a.bkey + (r * G + split) * a.cap,
                                      a.bid + (r * G + split) * a.cap, cnt[rl], a.C, &thr[rl],
                                      &cnt[rl]);
                        if (lane == 0) sthr[rl] = screen_thr<METRIC>(thr[rl], rnorm[rl]);
                        if (lane == 0 && a.sym && a.mcnt) a.mcnt[r] = -1;
                    }
                }
                // let the compaction's stores finish here: left pending, the
                // compiler's count of them reaches the join below and makes
                // every stage's first fragment read wait for all loads in
                // flight, the next stage's direct loads included
                __builtin_amdgcn_s_waitcnt(0x0F70);
                __syncthreads();
                if (tid == 0) need[par] = 0;
            }
          }
#pragma unroll
            for (int i = 0; i < BI; ++i)
#pragma unroll
                for (int j = 0; j < BJ; ++j) acc[i][j] = (f32x16){};
            // the new tile's column thresholds, straight into LDS by a
            // direct load (no register held, no wait here): the next stage's
            // barrier waits for it, and the tile's epilogue, at its last
            // stage, reads it; every wave finished the last tile's epilogue
            // before this stage's barrier.  Columns past n read row n - 1's
            // (their scores are never appended).  A one-stage tile waits at
            // once.
            if (a.sym && cbt != r0) {
                if (tid < kBN2) {
                    const int ci = cbt + tid < n ? cbt + tid : n - 1;
                    dma4(a.gthr, (uint32_t)ci * 4u,
                         reinterpret_cast<unsigned char*>(thrc) + wave * 256);
                }
                if (nk == 1) {
                    __builtin_amdgcn_s_waitcnt(0x0F70);
                    __syncthreads();
                }
            }
        }
        issue(t + 1, kt_f, cb_f);
        adv(kt_f, ki_f, cb_f);
        const unsigned char* pA = sA[buf];
        const unsigned char* pB = sB[buf];
        f16x8 fa[2][BI], fb[2][BJ];
        auto fload = [&](int sub, int slot) {
            const int co = ((2 * sub + (lane >> 5)) ^ fsw) * 16;
#pragma unroll
            for (int i = 0; i < BI; ++i)
                fa[slot][i] = *reinterpret_cast<const f16x8*>(pA + aro[i] + co);
#pragma unroll
            for (int j = 0; j < BJ; ++j)
                fb[slot][j] = *reinterpret_cast<const f16x8*>(pB + bro[j] + co);
        };
        fload(0, 0);
#pragma unroll
        for (int sub = 0; sub < 4; ++sub) {
            if (sub < 3) fload(sub + 1, (sub + 1) & 1);
#pragma unroll
            for (int i = 0; i < BI; ++i)
#pragma unroll
                for (int j = 0; j < BJ; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[sub & 1][i],
                                                                      fb[sub & 1][j], acc[i][j],
                                                                      0, 0, 0);
        }
        // interleave the next substep's fragment reads with this one's MFMAs
        // (the scheduler otherwise reads each fragment just before its use)
        __builtin_amdgcn_iglp_opt(1);
        if (kt == nk - 1) {
            // ---- epilogue of this column tile: distance, threshold, append ----
            const int cb = cbt;
            const bool diag = (cb == r0);
#pragma unroll
            for (int j = 0; j < BJ; ++j) {
                const int c = cb + wn * CW + j * 32 + (lane & 31);
                const bool cok = c < n;
#pragma unroll
                for (int i = 0; i < BI; ++i) {
                    int rbase = wm * RW + i * 32 + (lane >> 5) * 4;
                    asm volatile("" : "+v"(rbase));
                    if (diag) self_out(acc[i][j], rbase, wn * CW + j * 32 + (lane & 31));
                    const bool fon = a.sym && !diag;
                    const float thc = fon ? thrc[wn * CW + j * 32 + (lane & 31)] : 0.f;
                    uint64_t own, frn;
                    screen_pair<METRIC, SCALED>(acc[i][j], rbase, cn[j], cs[j], thc, fon, rscale,
                                                sthr, frow, own, frn);
                    // the append paths test every score exactly, so once any
                    // lane passed a screen the whole wave runs them
                    const uint64_t valid = __ballot(cok);
                    if (own & valid) {
                        asm volatile("" ::: "memory");   // rare path: reload, do not keep live
                        append_own<METRIC>(acc[i][j], rbase, r0, c, cn[j], cs[j], rscale, thr,
                                           rnorm, cnt, a, split, SCALED ? 2 : 0, nullptr,
                                           &need[tpar], cok);
                    }
                    if (frn & valid) {
                        asm volatile("" ::: "memory");
                        if (fstage)
                            queue_foreign<METRIC>(acc[i][j], rbase, r0, c, c - cb, cn[j], cs[j],
                                                  thc, rscale, rnorm, a, SCALED, &fqn, fq, cok);
                        else
                            append_foreign<METRIC>(acc[i][j], rbase, r0, c, cn[j], cs[j], thc,
                                                   rscale, rnorm, a, SCALED, cok);
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
            tpar ^= 1;
            cb_prev = cb;
        }
    }
    __builtin_amdgcn_s_waitcnt(0x0F70);
    __syncthreads();
    if (fstage) {
        // the last tile's queue: slots, then stores
        const int nq = fqn < kFQueue ? fqn : kFQueue;
        for (int k = tid; k < nq; k += WAVES * 64) {
            const int2 e = fq[k];
            const int64_t c = cb_prev + (e.x >> 16);
            const int p = atomicAdd(&a.bcnt[c * 2 + 1], 1);
            if (p < a.fcap) {
                const int64_t o = (c * 2 + 1) * (int64_t)a.cap + p;
                a.bkey[o] = __int_as_float(e.y);
                a.bid[o] = (int32_t)(r0 + (e.x & 0xffff));
            } else {
                atomicAdd(a.ovf, 1);
            }
        }
    }
    if (G > 1 && !a.sym) {
        // each split leaves at most C per row, so the merge of the G lists
        // sorts at most G * C
        for (int rl = wave; rl < kBM2; rl += WAVES) {
            const int64_t r = r0 + rl;
            if (r < n && cnt[rl] > a.C)
                compact_row_w(a.bkey + (r * G + split) * a.cap, a.bid + (r * G + split) * a.cap,
                              cnt[rl], a.C, &thr[rl], &cnt[rl]);
        }
        __syncthreads();
    }
    if (tid < kBM2 && r0 + tid < n) a.bcnt[(int64_t)(r0 + tid) * G + split] = cnt[tid];
}

// ---------------------------------------------------------------------------
// Between two launches of the symmetric sweep: each row's two lists become its
// C best so far (list 0), list 1 is emptied, and the row's threshold -- the
// C-th best distance, +inf while it has fewer -- is published for the next
// launch's screens in both directions.  One wave a row, one pass: every entry
// of list 0 and then list 1 is loaded into registers, the C smallest of that
// concatenation are found by the same exact search compact_row_core runs
// (ties kept in concatenation order), and the kept entries are written to the
// front of list 0 in that order.  This keeps exactly what compacting list 0,
// appending list 1 and compacting again would keep, in the same order: an
// entry among the C smallest of the whole is among the C smallest of its own
// list, and whatever a first compaction drops has C entries ahead of it.
// With seeds (below), a row under C entries keeps its seed as threshold.
// A row the launch left as the last merge did (list 1 empty, list 0 of the
// count that merge wrote and not compacted since: mcnt) is a fixed point of
// the merge and is skipped; in the pruned bands that is most rows.
__global__ __launch_bounds__(256) void sym_merge(float* __restrict__ bkey,
                                                 int32_t* __restrict__ bid,
                                                 int32_t* __restrict__ bcnt,
                                                 float* __restrict__ gthr, int* ovf, int64_t n,
                                                 int cap, int fcap, int C,
                                                 const float* __restrict__ seed,
                                                 int* __restrict__ flag,
                                                 int* __restrict__ mcnt) {
    const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= n) return;
    const int lane = threadIdx.x & 63;
    float* k0 = bkey + r * 2 * (int64_t)cap;
    int32_t* i0 = bid + r * 2 * (int64_t)cap;
    const float* k1 = k0 + cap;
    const int32_t* i1 = i0 + cap;
    const int c0 = __builtin_amdgcn_readfirstlane(bcnt[r * 2]);
    int c1 = __builtin_amdgcn_readfirstlane(bcnt[r * 2 + 1]);
    if (c1 == 0 && c0 == __builtin_amdgcn_readfirstlane(mcnt[r])) return;
    if (c1 > fcap) {                     // appends were dropped: the caller redoes the row
        if (lane == 0) {
            atomicAdd(ovf, 1);
            if (flag) flag[r] = 1;
        }
        c1 = fcap;
    }
    const int cnt = c0 + c1;
    constexpr int R = 32;                // c0 <= cap, c1 <= fcap <= cap, cap <= 1024
    // lanes of word t that hold an entry: l < cnt - 64 t
    auto valid = [&](int t) -> uint64_t {
        const int rem = cnt - t * 64;
        return rem >= 64 ? ~0ull : rem <= 0 ? 0ull : ((1ull << rem) - 1);
    };
    uint32_t u[R];
    int32_t v[R];
#pragma unroll
    for (int t = 0; t < R; ++t) {        // words past cnt are neither loaded nor used
        u[t] = 0xffffffffu;
        v[t] = 0;
        if (t * 64 < cnt) {
            const int i = min(t * 64 + lane, cnt - 1);
            const bool first = i < c0;
            const float* kp = first ? k0 + i : k1 + (i - c0);
            const int32_t* ip = first ? i0 + i : i1 + (i - c0);
            const float kf = *kp;
            v[t] = *ip;
            u[t] = fkey(kf);
        }
    }
    uint32_t mn = 0xffffffffu, mx = 0;
#pragma unroll
    for (int t = 0; t < R; ++t) {
        if (t * 64 >= cnt) break;
        const bool in = (valid(t) >> lane) & 1ull;
        mn = in && u[t] < mn ? u[t] : mn;
        mx = in && u[t] > mx ? u[t] : mx;
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const uint32_t x = __shfl_xor(mn, off, 64), y = __shfl_xor(mx, off, 64);
        mn = x < mn ? x : mn;
        mx = y > mx ? y : mx;
    }
    uint32_t lo = __builtin_amdgcn_readfirstlane(mn), hi = __builtin_amdgcn_readfirstlane(mx);
    if (cnt < C) lo = hi = 0xffffffffu;
    while (lo < hi) {
        const uint32_t mid = lo + ((hi - lo) >> 1);
        int c = 0;
#pragma unroll
        for (int t = 0; t < R; ++t) {
            if (t * 64 >= cnt) break;
            c += __popcll(__ballot(u[t] <= mid) & valid(t));
        }
        if (c >= C) hi = mid; else lo = mid + 1;
    }
    const uint32_t T = lo;
    int nlt = 0;
#pragma unroll
    for (int t = 0; t < R; ++t) {
        if (t * 64 >= cnt) break;
        nlt += __popcll(__ballot(u[t] < T) & valid(t));
    }
    int eq_left = C - nlt;
    int w = 0;
    const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
#pragma unroll
    for (int t = 0; t < R; ++t) {
        if (t * 64 >= cnt) break;
        const bool in = (valid(t) >> lane) & 1ull;
        const bool is_lt = in && u[t] < T;
        const bool is_eq = in && u[t] == T;
        const uint64_t meq = __ballot(is_eq);
        const int eq_rank = __popcll(meq & below);
        const bool keep = is_lt || (is_eq && eq_rank < eq_left);
        const uint64_t mk = __ballot(keep);
        if (keep) {
            const int dst = w + __popcll(mk & below);
            k0[dst] = funkey(u[t]);
            i0[dst] = v[t];
        }
        w += __popcll(mk);
        const int used = __popcll(meq);
        eq_left -= used < eq_left ? used : eq_left;
    }
    if (lane == 0) {
        gthr[r] = cnt >= C ? funkey(T) : seed ? seed[r] : INFINITY;
        bcnt[r * 2] = w;
        bcnt[r * 2 + 1] = 0;
        mcnt[r] = w;
    }
}

// ---------------------------------------------------------------------------
// Pruning the locality-ordered sweep's tiles.  A tile (I, J) can append a pair
// (r in panel I, c in panel J) only if the screened distance d^(r, c) falls
// below r's threshold (own list) or c's (foreign list); thresholds only fall
// during a launch, so the panels' largest thresholds when it starts bound
// both tests.  Each panel of the ordered plane, per group of its rows
// (panel_stats), gets a centre c_I (the mean of the rows as the screen sees
// them, v = scale * fp16 row), a radius R_I (largest |v - c_I|), its largest
// |v| (N_I) and the largest gap between a row's fp32 norm, which the screen's
// l2 formula takes, and |v|^2 (D_I).  Then for every pair of groups:
//   l2: d^ >= (|c_I - c_J| - R_I - R_J)^2 - D_I - D_J - 2 g N_I N_J - rounding
//   ip: d^ >= 1 - (c_I.c_J + R_I |c_J| + R_J |c_I| + R_I R_J) - g N_I N_J - rounding
// (the triangle inequality; Cauchy-Schwarz on the rows' offsets from the
// centres; g = (dim + 64) 2^-23 covers the screen's fp32 accumulation and
// scale products), with the centre terms in double.  A tile whose bound
// exceeds both panels' largest thresholds is left out of the launch: no pair
// in it could have been appended, so the lists are the unpruned sweep's.
// On clustered rows in locality order most tiles pair different clusters.

// A panel's rows are split into up to kSegs groups, each bounded on its own,
// so that a panel holding two clusters is two tight groups, not one wide one.
// The groups are the rows nearest to farthest-point seeds: the first seed is
// the panel's first row, and while some row lies farther than kSplit times
// the panel's largest threshold (in squared l2 of v; a threshold in ip is
// half that) from every seed so far, the farthest such row becomes the next
// seed.  Rows of one cluster lie within about its threshold of each other,
// so a panel of one cluster stays one group, and a panel whose rows came
// under one pivot from two clusters (the k-means leaves some clusters
// without a pivot of their own) splits along them.  Any grouping gives a
// valid bound; this one only decides how tight.  One workgroup per panel:
// nseg[I] groups; for group a, centre cen[(I kSegs + a) dim ..] and
// pst[4 (I kSegs + a) ..] = R, N, D, |c|, each rounded up.
constexpr int kSegs = 8;
constexpr float kSplit = 2.0f;

__global__ __launch_bounds__(256) void panel_stats(const _Float16* __restrict__ hp,
                                                   const float* __restrict__ scp,
                                                   const float* __restrict__ xnp,
                                                   const float* __restrict__ pthr, int metric,
                                                   int64_t n, int dim, int scaled,
                                                   float* __restrict__ cen,
                                                   float* __restrict__ pst,
                                                   int* __restrict__ nseg) {
    const int I = blockIdx.x, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int64_t r0 = (int64_t)I * kBM2;
    const int rows = (int)(n - r0 < kBM2 ? n - r0 : kBM2);
    __shared__ unsigned char seg[kBM2];
    __shared__ float mind[kBM2];
    __shared__ float rmax[4];
    __shared__ int rarg[4];
    __shared__ int cnt[kSegs];
    __shared__ int s_ns;
    __shared__ int s_seed;
    if (tid < kSegs) cnt[tid] = 0;
    if (tid == 0) { s_ns = 0; s_seed = 0; }
    const float th = pthr[I];
    const float tau = kSplit * (metric == SWANN_METRIC_IP ? 2.0f * th : th);
    __syncthreads();
    for (int k = 0; k < kSegs; ++k) {
        const int sr = s_seed;
        const float ssc = scaled ? scp[r0 + sr] : 1.f;
        // every row's squared distance to seed sr; a nearer seed takes the row
        for (int r = w; r < rows; r += 4) {
            const float sc = scaled ? scp[r0 + r] : 1.f;
            float d2 = 0.f;
            for (int t = lane; t < dim; t += 64) {
                const float dv = sc * (float)hp[(r0 + r) * dim + t] -
                                 ssc * (float)hp[(r0 + sr) * dim + t];
                d2 = __builtin_fmaf(dv, dv, d2);
            }
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) d2 += __shfl_xor(d2, off, 64);
            if (lane == 0 && (k == 0 || d2 < mind[r])) {
                mind[r] = d2;
                seg[r] = (unsigned char)k;
            }
        }
        __syncthreads();
        if (k + 1 == kSegs) break;
        // the farthest row from every seed so far (lowest index on ties)
        float v = tid < rows ? mind[tid] : -1.f;
        int at = tid;
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
            const float ov = __shfl_xor(v, off, 64);
            const int oa = __shfl_xor(at, off, 64);
            if (ov > v || (ov == v && oa < at)) { v = ov; at = oa; }
        }
        if (lane == 0) { rmax[w] = v; rarg[w] = at; }
        __syncthreads();
        if (tid == 0) {
            float bv = rmax[0];
            int ba = rarg[0];
            for (int q = 1; q < 4; ++q)
                if (rmax[q] > bv || (rmax[q] == bv && rarg[q] < ba)) { bv = rmax[q]; ba = rarg[q]; }
            // a NaN or infinite threshold never splits (every tile is kept)
            s_seed = (bv > tau && tau < INFINITY) ? ba : -1;
        }
        __syncthreads();
        if (s_seed < 0) break;
    }
    if (tid == 0) {
        int ns = 0;
        for (int r = 0; r < rows; ++r) {
            cnt[seg[r]] += 1;
            ns = seg[r] + 1 > ns ? seg[r] + 1 : ns;
        }
        s_ns = ns;
        nseg[I] = ns;
    }
    __syncthreads();
    const int ns = s_ns;
    for (int t = tid; t < dim; t += 256) {
        float sum[kSegs];
#pragma unroll
        for (int q = 0; q < kSegs; ++q) sum[q] = 0.f;
        for (int r = 0; r < rows; ++r) {
            const float v = (scaled ? scp[r0 + r] : 1.f) * (float)hp[(r0 + r) * dim + t];
#pragma unroll
            for (int q = 0; q < kSegs; ++q) sum[q] += seg[r] == q ? v : 0.f;
        }
        for (int q = 0; q < ns; ++q)
            cen[((int64_t)I * kSegs + q) * dim + t] = sum[q] / (float)cnt[q];
    }
    __syncthreads();
    double rad2[kSegs], nrm2[kSegs], dev[kSegs], cn2[kSegs];
#pragma unroll
    for (int q = 0; q < kSegs; ++q) { rad2[q] = 0.0; nrm2[q] = 0.0; dev[q] = 0.0; cn2[q] = 0.0; }
    if (w == 0) {
        for (int q = 0; q < ns; ++q) {
            const float* c = cen + ((int64_t)I * kSegs + q) * dim;
            double acc = 0.0;
            for (int t = lane; t < dim; t += 64) acc += (double)c[t] * (double)c[t];
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
            cn2[q] = acc;
        }
    }
    for (int r = w; r < rows; r += 4) {
        const int q = seg[r];
        const float* c = cen + ((int64_t)I * kSegs + q) * dim;
        const float sc = scaled ? scp[r0 + r] : 1.f;
        double d2 = 0.0, v2 = 0.0;
        for (int t = lane; t < dim; t += 64) {
            const double v = (double)(sc * (float)hp[(r0 + r) * dim + t]);
            const double dv = v - (double)c[t];
            d2 += dv * dv;
            v2 += v * v;
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
            d2 += __shfl_xor(d2, off, 64);
            v2 += __shfl_xor(v2, off, 64);
        }
        const double g = fabs((double)xnp[r0 + r] - v2);
#pragma unroll
        for (int s2 = 0; s2 < kSegs; ++s2)
            if (s2 == q) {
                rad2[s2] = d2 > rad2[s2] ? d2 : rad2[s2];
                nrm2[s2] = v2 > nrm2[s2] ? v2 : nrm2[s2];
                dev[s2] = g > dev[s2] ? g : dev[s2];
            }
    }
    __shared__ double red[4][kSegs][3];
    if (lane == 0)
#pragma unroll
        for (int q = 0; q < kSegs; ++q) { red[w][q][0] = rad2[q]; red[w][q][1] = nrm2[q]; red[w][q][2] = dev[q]; }
    __syncthreads();
    if (tid < ns) {
        const int q = tid;
        double a0 = 0.0, a1 = 0.0, a2 = 0.0;
        for (int ww = 0; ww < 4; ++ww) {
            a0 = red[ww][q][0] > a0 ? red[ww][q][0] : a0;
            a1 = red[ww][q][1] > a1 ? red[ww][q][1] : a1;
            a2 = red[ww][q][2] > a2 ? red[ww][q][2] : a2;
        }
        // double sums of dim terms are exact to ~1e-13 relative: 1e-6 up
        // covers them and the rounding to float
        const double up = 1.0 + 1e-6;
        float* o = pst + 4 * ((int64_t)I * kSegs + q);
        o[0] = (float)(sqrt(a0) * up);
        o[1] = (float)(sqrt(a1) * up);
        o[2] = (float)(a2 * up + 1e-30);
        o[3] = 0.f;
    }
    __syncthreads();
    if (w == 0 && lane < ns)
        for (int q = 0; q < ns; ++q)
            if (lane == q) pst[4 * ((int64_t)I * kSegs + q) + 3] = (float)(sqrt(cn2[q]) * (1.0 + 1e-6));
}

// The largest threshold of each panel's rows as the last merge published
// them (+inf for a row with fewer than C so far, or a NaN).
__global__ __launch_bounds__(256) void panel_thr(const float* __restrict__ gthr, int64_t n,
                                                 const int* __restrict__ dense,
                                                 float* __restrict__ pthr) {
    const int64_t r = (int64_t)blockIdx.x * kBM2 + threadIdx.x;
    float v = r < n ? gthr[r] : -INFINITY;
    if (v != v) v = INFINITY;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    __shared__ float red[4];
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    if (threadIdx.x == 0)
        pthr[blockIdx.x] = (dense && dense[blockIdx.x])
                               ? -INFINITY
                               : fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// The groups of every panel in panel order, as slots I * kSegs + a (a <
// nseg[I]), and their number.  One workgroup.
__global__ __launch_bounds__(1024) void group_list(const int* __restrict__ nseg, int ntile,
                                                   int* __restrict__ glist,
                                                   int* __restrict__ gcount) {
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    __shared__ int wsum[16];
    __shared__ int base;
    if (tid == 0) base = 0;
    __syncthreads();
    for (int c0 = 0; c0 < ntile; c0 += 1024) {
        const int I = c0 + tid;
        const int v = I < ntile ? nseg[I] : 0;
        int x = v;                                   // inclusive scan within the wave
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const int y = __shfl_up(x, off, 64);
            if (lane >= off) x += y;
        }
        if (lane == 63) wsum[w] = x;
        __syncthreads();
        int pre = base;
        for (int q = 0; q < w; ++q) pre += wsum[q];
        pre += x - v;
        for (int q = 0; q < v; ++q) glist[pre + q] = I * kSegs + q;
        __syncthreads();
        if (tid == 0)
            for (int q = 0; q < 16; ++q) base += wsum[q];
        __syncthreads();
    }
    if (tid == 0) *gcount = base;
}

// Every pair of groups (ga in panel I, gb in panel J > I) at once: the centres'
// squared distance (l2) or dot product (ip) in double, as a 64 x 64 block of
// the groups' Gram per workgroup (LDS tiles of 16 coordinates, 4 x 4 pairs a
// thread), then the pair's bound (above), rounded down to float, and the
// tile's bound tlb[I ntile + J] (fkey order) as the least over its pairs.  A
// NaN bound stores -inf, which keeps the tile.
constexpr int kGB = 64, kGK = 16;

__global__ __launch_bounds__(256) void group_bounds(const float* __restrict__ cen,
                                                    const float* __restrict__ pst,
                                                    const int* __restrict__ glist, int G,
                                                    int ntile, int dim, int metric,
                                                    unsigned* __restrict__ tlb) {
    const int bi = blockIdx.y, bj = blockIdx.x;
    if (bj < bi) return;
    const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
    __shared__ double sa[kGK][kGB + 1];
    __shared__ double sb[kGK][kGB + 1];
    __shared__ int slot_a[kGB], slot_b[kGB];
    if (tid < kGB) {
        const int ga = bi * kGB + tid, gb = bj * kGB + tid;
        slot_a[tid] = ga < G ? glist[ga] : -1;
        slot_b[tid] = gb < G ? glist[gb] : -1;
    }
    __syncthreads();
    const bool l2 = metric == SWANN_METRIC_L2;
    double acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = 0.0;
    for (int k0 = 0; k0 < dim; k0 += kGK) {
        // 64 groups x 16 coordinates a side: 4 elements a thread each
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int idx = e * 256 + tid;
            const int gr = idx >> 4, kk = idx & 15;
            const int k = k0 + kk;
            const int sa_ = slot_a[gr], sb_ = slot_b[gr];
            sa[kk][gr] = (sa_ >= 0 && k < dim) ? (double)cen[(int64_t)sa_ * dim + k] : 0.0;
            sb[kk][gr] = (sb_ >= 0 && k < dim) ? (double)cen[(int64_t)sb_ * dim + k] : 0.0;
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < kGK; ++kk) {
            double x[4], y[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) x[i] = sa[kk][ty * 4 + i];
#pragma unroll
            for (int j = 0; j < 4; ++j) y[j] = sb[kk][tx * 4 + j];
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    if (l2) {
                        const double d = x[i] - y[j];
                        acc[i][j] = __builtin_fma(d, d, acc[i][j]);
                    } else {
                        acc[i][j] = __builtin_fma(x[i], y[j], acc[i][j]);
                    }
                }
        }
        __syncthreads();
    }
    const double g = ((double)dim + 64.0) * 0x1p-23;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int ia = slot_a[ty * 4 + i];
        if (ia < 0) continue;
        const int I = ia / kSegs;
        const double RI = pst[4 * ia], NI = pst[4 * ia + 1], DI = pst[4 * ia + 2],
                     CI = pst[4 * ia + 3];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int jb = slot_b[tx * 4 + j];
            if (jb < 0) continue;
            const int J = jb / kSegs;
            if (J <= I) continue;
            const double RJ = pst[4 * jb], NJ = pst[4 * jb + 1], DJ = pst[4 * jb + 2],
                         CJ = pst[4 * jb + 3];
            double lb;
            if (l2) {
                const double gap = sqrt(acc[i][j]) * (1.0 - 1e-9) - RI - RJ;
                lb = (gap > 0.0 ? gap * gap : 0.0) - DI - DJ - 2.0 * g * NI * NJ -
                     0x1p-21 * 1.1 * (NI + NJ) * (NI + NJ);
            } else {
                lb = 1.0 - (acc[i][j] + 1e-9 * CI * CJ + RI * CJ + RJ * CI + RI * RJ) -
                     g * NI * NJ - 0x1p-22 * (1.0 + NI * NJ);
            }
            float f;
            if (lb != lb) {
                f = -INFINITY;
            } else {
                f = (float)lb;
                if ((double)f > lb) f = nextafterf(f, -INFINITY);
            }
            atomicMin(&tlb[(int64_t)I * ntile + J], fkey(f));
        }
    }
}

__global__ void fill_u32(unsigned* p, int64_t n, unsigned v) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) p[i] = v;
}

// One wave per panel I of a band launch [b0, b1): the column tiles J it must
// still score, ascending, into tlist[I * kBandMax ..], their count into
// tcnt[I], and the launch's total into *tsum.  A tile is kept unless its
// bound exceeds both panels' largest thresholds (a NaN threshold keeps it); a
// dense panel's tiles wait for the dense launch (dense_keep).
__global__ __launch_bounds__(64) void tile_keep(const unsigned* __restrict__ tlb,
                                                const int* __restrict__ dense,
                                                const float* __restrict__ pthr, int ntile,
                                                int b0, int b1, int* __restrict__ tlist,
                                                int* __restrict__ tcnt,
                                                unsigned long long* __restrict__ tsum) {
    const int I = blockIdx.x, lane = threadIdx.x;
    const int j0 = I + b0, j1 = I + b1 < ntile ? I + b1 : ntile;
    const int nj = (dense && dense[I]) ? 0 : j1 - j0;
    const float thI = pthr[I];
    int base = 0;
    for (int jc = 0; jc < nj; jc += 64) {
        const int j = jc + lane;
        bool k = false;
        if (j < nj) {
            const int J = j0 + j;
            const float th = fmaxf(thI, pthr[J]);
            k = J == I || !(funkey(tlb[(int64_t)I * ntile + J]) > th);
        }
        const uint64_t m = __ballot(k);
        const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
        if (k) tlist[(int64_t)I * kBandMax + base + __popcll(m & below)] = j0 + j;
        base += __popcll(m);
    }
    if (lane == 0) {
        tcnt[I] = base;
        atomicAdd(tsum, (unsigned long long)base);
    }
}

// Dense panels.  A panel whose own rows still need more than kDenseTiles tiles
// beyond the seed window after the seed bands -- its rows have neighbours in
// few of them, but its groups bound nothing: rows of many clusters that the
// order's pivots gathered into one run -- would score that many tiles alone
// in its workgroup, band after band.  Its rows are instead swept again
// one-sided after the bands (the ordered sweep's repair, which writes their
// lists from scratch); in the bands it scores none of its tiles and keeps none
// for its own rows (its panel threshold counts as -inf), and the tiles other
// panels' rows need from it are scored after the bands by those panels'
// workgroups (dense_keep), in parallel.  dense_mark lists them (dense[I] = 1,
// dlist / *nd); dense_flag flags their rows for the repair and raises the
// overflow count so that the repair runs.
constexpr int kDenseTiles = 64;

__global__ __launch_bounds__(256) void dense_mark(const unsigned* __restrict__ tlb,
                                                  const float* __restrict__ pthr, int ntile,
                                                  int win, int* __restrict__ dense,
                                                  int* __restrict__ dlist, int* nd) {
    const int I = blockIdx.x, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const float th = pthr[I];
    int c = 0;
    for (int J = tid; J < ntile; J += 256) {
        if ((J > I ? J - I : I - J) < win) continue;
        const int a0 = J < I ? J : I, b0 = J < I ? I : J;
        c += !(funkey(tlb[(int64_t)a0 * ntile + b0]) > th) ? 1 : 0;
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) c += __shfl_xor(c, off, 64);
    __shared__ int red[4];
    if (lane == 0) red[w] = c;
    __syncthreads();
    if (tid == 0 && red[0] + red[1] + red[2] + red[3] > kDenseTiles) {
        dense[I] = 1;
        dlist[atomicAdd(nd, 1)] = I;
    }
}

__global__ __launch_bounds__(256) void dense_flag(const int* __restrict__ dlist, int64_t n,
                                                  int* __restrict__ flag, int* ovf) {
    const int64_t r = (int64_t)dlist[blockIdx.x] * kBM2 + threadIdx.x;
    if (threadIdx.x == 0) atomicAdd(ovf, 1);
    if (r < n) flag[r] = 1;
}

// The dense launch's lists: one wave per panel J (not dense), the dense
// panels D <= J - win whose tile (D, J) J's rows still need at the thresholds
// the bands left.  (A tile (I, D) with I < D was scored in I's band list.)
__global__ __launch_bounds__(64) void dense_keep(const unsigned* __restrict__ tlb,
                                                 const int* __restrict__ dense,
                                                 const int* __restrict__ dlist, int nd,
                                                 const float* __restrict__ pthr, int ntile,
                                                 int win, int* __restrict__ tlist,
                                                 int* __restrict__ tcnt,
                                                 unsigned long long* __restrict__ tsum) {
    const int J = blockIdx.x, lane = threadIdx.x;
    const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
    const float th = pthr[J];
    int base = 0;
    for (int qc = 0; qc < (dense[J] ? 0 : nd); qc += 64) {
        const int q = qc + lane;
        bool k = false;
        int D = 0;
        if (q < nd) {
            D = dlist[q];
            k = D <= J - win && !(funkey(tlb[(int64_t)D * ntile + J]) > th);
        }
        const uint64_t m = __ballot(k);
        if (k) tlist[(int64_t)J * kBandMax + base + __popcll(m & below)] = D;
        base += __popcll(m);
    }
    if (lane == 0) {
        tcnt[J] = base;
        atomicAdd(tsum, (unsigned long long)base);
    }
}

// The bounded repair of a repaired panel D = plist[p]: each of its rows
// against every panel group, the bound of group_bounds with the row as a
// group of one (radius 0; its norm, centre norm and norm deviation its own),
// so that a tile J is swept again only when some row r of D may have a pair
// there no farther than its threshold gthr[r] as the last merge left it (an
// upper bound of r's C-th listed distance, +inf while r holds fewer).  A
// tile left out holds no pair closer than its row's C-th, so the one-sided
// sweep over the rest rebuilds D's lists exactly.
//
// Row stats as panel_stats takes them for a group: the row's plane values
// v = scale * plane in double, N = |v| (1 + 1e-6), Dv = |xn - |v|^2| (1 +
// 1e-6) + 1e-30.  rst[2 (p * 256 + i) + {0, 1}].
__global__ __launch_bounds__(256) void repair_row_stats(const _Float16* __restrict__ hp,
                                                        const float* __restrict__ scp,
                                                        const float* __restrict__ xnp,
                                                        const int* __restrict__ plist, int64_t n,
                                                        int dim, int scaled,
                                                        double* __restrict__ rst) {
    const int p = blockIdx.x, lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int64_t r0 = (int64_t)plist[p] * kBM2;
    for (int i = w; i < kBM2; i += 4) {
        const int64_t r = r0 + i;
        if (r >= n) {
            if (lane == 0) { rst[2 * ((int64_t)p * kBM2 + i)] = 0.0; rst[2 * ((int64_t)p * kBM2 + i) + 1] = 0.0; }
            continue;
        }
        const float sc = scaled ? scp[r] : 1.f;
        double v2 = 0.0;
        for (int t = lane; t < dim; t += 64) {
            const double v = (double)(sc * (float)hp[r * dim + t]);
            v2 += v * v;
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) v2 += __shfl_xor(v2, off, 64);
        if (lane == 0) {
            const double up = 1.0 + 1e-6;
            rst[2 * ((int64_t)p * kBM2 + i)] = sqrt(v2) * up;
            rst[2 * ((int64_t)p * kBM2 + i) + 1] = fabs((double)xnp[r] - v2) * up + 1e-30;
        }
    }
}

// need[p * ntile + J] = 1 when some row of D = plist[p] may need tile J.
// Grid (groups / 64, 4 row quarters of D, np): 64 rows x 64 groups a
// workgroup, their distances (l2) or products (ip) in double as in
// group_bounds.
__global__ __launch_bounds__(256) void repair_need(const _Float16* __restrict__ hp,
                                                   const float* __restrict__ scp,
                                                   const float* __restrict__ cen,
                                                   const float* __restrict__ pst,
                                                   const int* __restrict__ glist, int G,
                                                   const float* __restrict__ gthr,
                                                   const int* __restrict__ plist,
                                                   const double* __restrict__ rst, int64_t n,
                                                   int ntile, int dim, int metric, int scaled,
                                                   int* __restrict__ need) {
    const int bj = blockIdx.x, rq = blockIdx.y, p = blockIdx.z;
    const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
    const int64_t r0 = (int64_t)plist[p] * kBM2 + rq * kGB;
    __shared__ double sa[kGK][kGB + 1];
    __shared__ double sb[kGK][kGB + 1];
    __shared__ int slot_b[kGB];
    __shared__ float rsc[kGB];
    if (tid < kGB) {
        const int gb = bj * kGB + tid;
        slot_b[tid] = gb < G ? glist[gb] : -1;
        const int64_t r = r0 + tid;
        rsc[tid] = r < n ? (scaled ? scp[r] : 1.f) : 0.f;
    }
    __syncthreads();
    const bool l2 = metric == SWANN_METRIC_L2;
    double acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = 0.0;
    for (int k0 = 0; k0 < dim; k0 += kGK) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int idx = e * 256 + tid;
            const int gr = idx >> 4, kk = idx & 15;
            const int k = k0 + kk;
            const int64_t r = r0 + gr;
            const int sb_ = slot_b[gr];
            sa[kk][gr] = (r < n && k < dim) ? (double)(rsc[gr] * (float)hp[r * dim + k]) : 0.0;
            sb[kk][gr] = (sb_ >= 0 && k < dim) ? (double)cen[(int64_t)sb_ * dim + k] : 0.0;
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < kGK; ++kk) {
            double x[4], y[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) x[i] = sa[kk][ty * 4 + i];
#pragma unroll
            for (int j = 0; j < 4; ++j) y[j] = sb[kk][tx * 4 + j];
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    if (l2) {
                        const double d = x[i] - y[j];
                        acc[i][j] = __builtin_fma(d, d, acc[i][j]);
                    } else {
                        acc[i][j] = __builtin_fma(x[i], y[j], acc[i][j]);
                    }
                }
        }
        __syncthreads();
    }
    const double g = ((double)dim + 64.0) * 0x1p-23;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int rl = rq * kGB + ty * 4 + i;
        const int64_t r = (int64_t)plist[p] * kBM2 + rl;
        if (r >= n) continue;
        const double NI = rst[2 * ((int64_t)p * kBM2 + rl)];
        const double DI = rst[2 * ((int64_t)p * kBM2 + rl) + 1];
        const double th = (double)gthr[r];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int jb = slot_b[tx * 4 + j];
            if (jb < 0) continue;
            const double RJ = pst[4 * jb], NJ = pst[4 * jb + 1], DJ = pst[4 * jb + 2],
                         CJ = pst[4 * jb + 3];
            double lb;
            if (l2) {
                const double gap = sqrt(acc[i][j]) * (1.0 - 1e-9) - RJ;
                lb = (gap > 0.0 ? gap * gap : 0.0) - DI - DJ - 2.0 * g * NI * NJ -
                     0x1p-21 * 1.1 * (NI + NJ) * (NI + NJ);
            } else {
                lb = 1.0 - (acc[i][j] + 1e-9 * NI * CJ + RJ * NI) - g * NI * NJ -
                     0x1p-22 * (1.0 + NI * NJ);
            }
            // a NaN bound or threshold keeps the tile
            if (!(lb > th)) need[(int64_t)p * ntile + jb / kSegs] = 1;
        }
    }
}

// The bounded repair's lists: for repaired panel D = plist[p], D itself and
// the tiles need marks, ascending, in tlist[p * ntile ..]; their number in
// tcnt[p], the total added to *tsum.  One wave a panel.
__global__ __launch_bounds__(64) void repair_list(const int* __restrict__ need,
                                                  const int* __restrict__ plist, int ntile,
                                                  int* __restrict__ tlist,
                                                  int* __restrict__ tcnt,
                                                  unsigned long long* __restrict__ tsum) {
    const int p = blockIdx.x, lane = threadIdx.x;
    const int D = plist[p];
    const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
    int base = 0;
    for (int J0 = 0; J0 < ntile; J0 += 64) {
        const int J = J0 + lane;
        const bool k = J < ntile && (J == D || need[(int64_t)p * ntile + J] != 0);
        const uint64_t m = __ballot(k);
        if (k) tlist[(int64_t)p * ntile + base + __popcll(m & below)] = J;
        base += __popcll(m);
    }
    if (lane == 0) {
        tcnt[p] = base;
        atomicAdd(tsum, (unsigned long long)base);
    }
}

__global__ __launch_bounds__(256) void sym_init(float* __restrict__ gthr,
                                                int32_t* __restrict__ bcnt, int* ovf,
                                                int64_t n, const float* __restrict__ seed,
                                                int* __restrict__ mcnt) {
    const int64_t r = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (r < n) {
        gthr[r] = seed ? seed[r] : INFINITY;
        bcnt[r * 2] = 0;
        bcnt[r * 2 + 1] = 0;
        mcnt[r] = 0;
    }
    if (r == 0) *ovf = 0;
}

// ---------------------------------------------------------------------------
// Locality order for the symmetric sweep.  A row's threshold only falls as
// the bands reach its neighbours; until then it appends much of what it
// sees, and in row order its survivors spread over many tiles, sending many
// 32 x 32 blocks down the epilogue's slow path.  So rows are first grouped by
// the nearest of P evenly spaced pivot rows, measured on a 64-coordinate
// sketch.  The first assignment (on every kSampleStride-th row) also tells
// whether the rows cluster at all: if their mean distance to the nearest
// pivot is not under kClusterRatio of that to an arbitrary pivot, an order
// would not help and the sweep runs plain.  Otherwise kKmeanSteps k-means
// steps refine the pivots, the pivots are chained nearest to nearest, and
// the rows, sorted by their pivot's place in the chain, are gathered into an
// ordered copy that the whole sweep runs on: a row's neighbours then sit in
// few tiles near the diagonal, its threshold falls within the first
// launches, and most blocks have no survivor.  The lists come out as in row
// order (the sweep is exact in any order), in ordered ids that sweep_final
// maps back.  A row whose threshold stayed loose can still meet its
// neighbours in one burst that overflows its second list; the merge flags
// it and its row panel is swept again one-sided (repair_merge).
// option sweep_order = 0 keeps the rows' own order and uses the first
// kSeedBand bands of the ordered copy as a pre-pass instead: each row's
// resulting threshold -- the C-th best of real distances, an upper bound of
// its true C-th -- seeds its threshold in the sweep in row order.  A seed
// holds back (in both directions) only candidates that could not be among
// the row's C best; the margin added to it (2^-16 of |t| + |x|^2) lies far
// above any difference in how the accumulators round the same pair in
// another tile position.
constexpr int kSketch = 64;          // sketch coordinates a row
constexpr int kMaxPivots = 2048;
constexpr int kPivChunk = 256;       // pivots staged in LDS at a time (64 KB)
constexpr int64_t kSeedBand = 4;     // first bands: tiles (I, I + b), b < kSeedBand
constexpr int kKmeanSteps = 2;       // refinements of the pivots' sketches
constexpr int64_t kSampleStride = 8; // rows of the k-means steps: every 8th
constexpr float kClusterRatio = 0.3f;  // nearest-pivot / arbitrary-pivot distance for an order

// Coordinates l * dim / 64 of each row, as float (zeros past dim).
template <typename XT>
__global__ __launch_bounds__(256) void row_sketch(const XT* __restrict__ X, int64_t n, int dim,
                                                  float* __restrict__ sk) {
    const int64_t r = (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (r >= n) return;
    const int l = threadIdx.x & 63;
    const int k = dim >= kSketch ? (int)(((int64_t)l * dim) / kSketch) : l;
    sk[r * kSketch + l] = k < dim ? (float)X[r * (int64_t)dim + k] : 0.f;
}

// Each row's nearest pivot on the sketch (pivot p is row p * n / P; ties to
// the lower p), and the rows per pivot.  One thread a row; the pivots'
// sketches are staged in LDS, kPivChunk at a time, read by every lane at
// once (broadcast).
// With acc, also adds up (over all rows) the distance to the nearest pivot
// and to pivot r % P, a stand-in for an arbitrary one: their ratio says how
// clustered the rows are.
// Rows r = i * stride for i < m (every row, or a sample for the k-means
// steps); lab and the counts are by i.
__global__ __launch_bounds__(256) void nearest_pivot(const float* __restrict__ sk, int64_t m,
                                                     int64_t stride, int P,
                                                     const float* __restrict__ psk,
                                                     int* __restrict__ lab,
                                                     int* __restrict__ pcnt,
                                                     float* __restrict__ acc) {
    __shared__ __align__(16) float sp[kPivChunk * kSketch];
    __shared__ float red[2][4];
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const bool ok = i < m;
    const int64_t r = i * stride;
    const int pr = (int)(r % P);
    float drand = 0.f;
    float x[kSketch];
#pragma unroll
    for (int k = 0; k < kSketch; k += 4) {
        const float4 v = ok ? *reinterpret_cast<const float4*>(sk + r * kSketch + k)
                            : make_float4(0.f, 0.f, 0.f, 0.f);
        x[k] = v.x; x[k + 1] = v.y; x[k + 2] = v.z; x[k + 3] = v.w;
    }
    float best = INFINITY;
    int bi = 0;
    for (int p0 = 0; p0 < P; p0 += kPivChunk) {
        const int pc = P - p0 < kPivChunk ? P - p0 : kPivChunk;
        __syncthreads();
        for (int t = threadIdx.x; t < pc * kSketch; t += 256) sp[t] = psk[(int64_t)p0 * kSketch + t];
        __syncthreads();
        for (int p = 0; p < pc; ++p) {
            const float4* s4 = reinterpret_cast<const float4*>(sp + p * kSketch);
            float d = 0.f;
#pragma unroll
            for (int k = 0; k < kSketch / 4; ++k) {
                const float4 v = s4[k];
                float t;
                t = x[4 * k] - v.x; d = __builtin_fmaf(t, t, d);
                t = x[4 * k + 1] - v.y; d = __builtin_fmaf(t, t, d);
                t = x[4 * k + 2] - v.z; d = __builtin_fmaf(t, t, d);
                t = x[4 * k + 3] - v.w; d = __builtin_fmaf(t, t, d);
            }
            if (d < best) { best = d; bi = p0 + p; }
            if (p0 + p == pr) drand = d;
        }
    }
    if (ok) {
        lab[i] = bi;
        atomicAdd(&pcnt[bi], 1);
    }
    if (acc) {
        float b0 = ok ? best : 0.f, b1 = ok ? drand : 0.f;
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
            b0 += __shfl_xor(b0, off, 64);
            b1 += __shfl_xor(b1, off, 64);
        }
        const int wv = threadIdx.x >> 6;
        if ((threadIdx.x & 63) == 0) { red[0][wv] = b0; red[1][wv] = b1; }
        __syncthreads();
        if (threadIdx.x == 0) {
            atomicAdd(&acc[0], red[0][0] + red[0][1] + red[0][2] + red[0][3]);
            atomicAdd(&acc[1], red[1][0] + red[1][1] + red[1][2] + red[1][3]);
        }
    }
}

__global__ void fill_zero(int* p, int n) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) p[i] = 0;
}

// Exclusive scan of the P <= 2048 counts: each pivot's first slot, into
// pstart (P + 1 entries, the last n) and into pcnt (the cursor pivot_place
// advances).
__global__ __launch_bounds__(1024) void pivot_scan(int* pcnt, int* pstart, int P) {
    __shared__ int s[kMaxPivots];
    const int t = threadIdx.x;
    const int v0 = 2 * t < P ? pcnt[2 * t] : 0, v1 = 2 * t + 1 < P ? pcnt[2 * t + 1] : 0;
    s[t] = v0 + v1;
    __syncthreads();
    for (int off = 1; off < 1024; off <<= 1) {
        const int u = t >= off ? s[t - off] : 0;
        __syncthreads();
        s[t] += u;
        __syncthreads();
    }
    const int e = s[t] - v0 - v1;                  // exclusive start of the pair
    if (2 * t < P) { pcnt[2 * t] = e; if (pstart) pstart[2 * t] = e; }
    if (2 * t + 1 < P) { pcnt[2 * t + 1] = e + v0; if (pstart) pstart[2 * t + 1] = e + v0; }
    if (pstart && t == 1023) pstart[P] = s[t];
}

// The mean sketch of each pivot's rows (rows perm[pstart[p] .. pstart[p+1])):
// one workgroup a pivot, one thread a coordinate; a pivot with no rows keeps
// its sketch.
__global__ __launch_bounds__(kSketch) void group_mean(const float* __restrict__ sk,
                                                      const int* __restrict__ perm,
                                                      const int* __restrict__ pstart,
                                                      int64_t stride, float* __restrict__ psk) {
    const int p = blockIdx.x, k = threadIdx.x;
    const int b = pstart[p], e = pstart[p + 1];
    if (e <= b) return;
    float acc = 0.f;
    for (int i = b; i < e; ++i) acc += sk[(int64_t)perm[i] * stride * kSketch + k];
    psk[(int64_t)p * kSketch + k] = acc / (float)(e - b);
}

// The pivots' initial sketches: rows p * n / P.
__global__ void pivot_init(const float* __restrict__ sk, int64_t n, int P, float* __restrict__ psk) {
    const int p = blockIdx.x, k = threadIdx.x;
    psk[(int64_t)p * kSketch + k] = sk[((int64_t)p * n / P) * kSketch + k];
}

// Squared sketch distances between pivots: D[p][q].
__global__ void pivot_dist(const float* __restrict__ psk, int P, float* __restrict__ D) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)P * P) return;
    const int p = (int)(i / P), q = (int)(i % P);
    float d = 0.f;
    for (int k = 0; k < kSketch; ++k) {
        const float t = psk[(int64_t)p * kSketch + k] - psk[(int64_t)q * kSketch + k];
        d = __builtin_fmaf(t, t, d);
    }
    D[i] = d;
}

// Rows' sort key: their pivot's place in the chain.
__global__ void relabel(int* __restrict__ lab, int64_t n, const int* __restrict__ rank,
                        int* __restrict__ pcnt) {
    const int64_t r = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (r >= n) return;
    const int v = rank[lab[r]];
    lab[r] = v;
    atomicAdd(&pcnt[v], 1);
}

// perm[i]: the row at position i of the locality order (rows of one pivot
// together, in no particular order among themselves).
__global__ void pivot_place(const int* __restrict__ lab, int64_t n, int* pcur,
                            int* __restrict__ perm) {
    const int64_t r = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (r < n) perm[atomicAdd(&pcur[lab[r]], 1)] = (int)r;
}

// The ordered copy: row perm[i] of the plane, its norm and scale at i.
__global__ __launch_bounds__(256) void gather_rows(const _Float16* __restrict__ h, int64_t n,
                                                   int dim, const int* __restrict__ perm,
                                                   const float* __restrict__ xn,
                                                   const float* __restrict__ sc,
                                                   _Float16* __restrict__ hp,
                                                   float* __restrict__ xnp,
                                                   float* __restrict__ scp) {
    const int64_t i = (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (i >= n) return;
    const int lane = threadIdx.x & 63;
    const int64_t r = perm[i];
    const uint4* src = reinterpret_cast<const uint4*>(h + r * dim);
    uint4* dst = reinterpret_cast<uint4*>(hp + i * dim);
    for (int t = lane; t < dim / 8; t += 64) dst[t] = src[t];
    if (lane == 0) {
        xnp[i] = xn[r];
        if (sc) scp[i] = sc[r];
    }
}

// seed[perm[i]]: ordered row i's pre-pass threshold plus the margin, or +inf
// where the pre-pass left it under C entries.
__global__ void seed_map(const float* __restrict__ gthr, const int* __restrict__ perm,
                         const float* __restrict__ xn, int64_t n, float* __restrict__ seed) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const float t = gthr[i];
    const int r = perm[i];
    seed[r] = t < INFINITY ? t + (fabsf(t) + fabsf(xn[r])) * (1.f / 65536.f) + 1e-30f : INFINITY;
}

// The row panels holding a flagged row (one thread a panel), listed in plist
// with their count in *npl.
__global__ void flag_panels(const int* __restrict__ flag, int64_t n, int ntile,
                            int* __restrict__ plist, int* npl) {
    const int p = blockIdx.x * 256 + threadIdx.x;
    if (p >= ntile) return;
    int any = 0;
    for (int64_t r = (int64_t)p * kBM2; r < n && r < (int64_t)(p + 1) * kBM2; ++r) any |= flag[r];
    if (any) plist[atomicAdd(npl, 1)] = p;
}

// The repair of one row panel in kRepairSplits column ranges (its rows' lists
// in a scratch area, row-panel relative), then per row: the entries of those
// lists sorted by (d, the rows' own ids) and the first C written as the row's
// list 0 (list 1 emptied).  One workgroup a row.
constexpr int kRepairSplits = 16;
constexpr int kRepairSort = 4096;    // >= kRepairSplits * C for C <= 256

__global__ __launch_bounds__(256) void repair_merge(const float* __restrict__ rkey,
                                                    const int32_t* __restrict__ rid,
                                                    const int32_t* __restrict__ rcnt, int r0,
                                                    int64_t n, int cap, int C,
                                                    const int32_t* __restrict__ perm,
                                                    float* __restrict__ bkey,
                                                    int32_t* __restrict__ bid,
                                                    int32_t* __restrict__ bcnt) {
    __shared__ float sd[kRepairSort];
    __shared__ int si[kRepairSort];
    __shared__ int so[kRepairSort];
    const int rl = blockIdx.x;
    const int64_t r = (int64_t)r0 + rl;
    if (r >= n) return;
    int segc[kRepairSplits], cnt = 0;
    for (int sg = 0; sg < kRepairSplits; ++sg) {
        segc[sg] = rcnt[rl * kRepairSplits + sg];
        cnt += segc[sg];
    }
    int np = 2;
    while (np < cnt) np <<= 1;
    for (int i = threadIdx.x; i < np; i += 256) {
        int sg = 0, off = i;
        while (sg < kRepairSplits - 1 && off >= segc[sg]) { off -= segc[sg]; ++sg; }
        const bool real = i < cnt;
        const int64_t at = ((int64_t)rl * kRepairSplits + sg) * cap + off;
        sd[i] = real ? rkey[at] : INFINITY;
        si[i] = real ? rid[at] : INT32_MAX;
        so[i] = real ? perm[rid[at]] : INT32_MAX;    // the order of ties
    }
    __syncthreads();
    for (int size = 2; size <= np; size <<= 1)
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int i = threadIdx.x; i < np; i += 256) {
                const int j = i ^ stride;
                if (j > i) {
                    const bool up = (i & size) == 0;
                    const bool lt = sd[j] < sd[i] || (sd[j] == sd[i] && so[j] < so[i]);
                    if (up == lt) {
                        const float td = sd[i]; sd[i] = sd[j]; sd[j] = td;
                        const int ti = si[i]; si[i] = si[j]; si[j] = ti;
                        const int to = so[i]; so[i] = so[j]; so[j] = to;
                    }
                }
            }
            __syncthreads();
        }
    const int kept = cnt < C ? cnt : C;
    for (int t = threadIdx.x; t < kept; t += 256) {
        bkey[r * 2 * (int64_t)cap + t] = sd[t];
        bid[r * 2 * (int64_t)cap + t] = si[t];
    }
    if (threadIdx.x == 0) {
        bcnt[r * 2] = kept;
        bcnt[r * 2 + 1] = 0;
    }
}

inline int64_t al256(int64_t b) { return ((b + 255) / 256) * 256; }

inline int64_t prune_bytes(int64_t n, int dim);

inline int64_t seed_bytes(int64_t n, int dim) {
    const int64_t ntile = (n + kBM2 - 1) / kBM2;
    return al256(n * kSketch * 4) + al256(n * 4) * 7 + al256(kMaxPivots * 4) +
           al256(n * (int64_t)dim * 2) + al256(ntile * 4) + 256 +
           al256((int64_t)kMaxPivots * kSketch * 4) + al256((kMaxPivots + 1) * 4) +
           al256((int64_t)kMaxPivots * kMaxPivots * 4) + al256(kMaxPivots * 4) +
           prune_bytes(n, dim);
}

// The few-panel repair's scratch: lists of one panel in kRepairSplits ranges.
inline int64_t repair_bytes(int cap) {
    return al256((int64_t)kBM2 * kRepairSplits * cap * 4) * 2 + al256(kBM2 * kRepairSplits * 4);
}


// The pruned ordered sweep's scratch: panel centres and statistics, the
// panels' largest thresholds, the launch's tile lists and counts, a counter,
// the list of groups, every tile's bound (ntile^2 floats: 61 MB at 1M rows)
// and the dense panels.
inline int64_t prune_bytes(int64_t n, int dim) {
    const int64_t ntile = (n + kBM2 - 1) / kBM2;
    return al256(ntile * kSegs * (int64_t)dim * 4) + al256(ntile * kSegs * 16) +
           al256(ntile * 4) * 2 + al256(ntile * kBandMax * 4) + al256(ntile * 4) + 256 +
           al256(ntile * kSegs * 4) + 256 + al256(ntile * ntile * 4) + al256((ntile + 1) * 4) +
           al256(ntile * 4);
}

// 256 x 256 tiles the last sweep on this thread scored (the bands' tiles, less
// those the pruned ordered sweep proved empty, plus any repair), -1 before.
thread_local int64_t g_tiles_scored = -1;

// Row panels the last sweep on this thread handled as dense (tiles scored by
// the other panels' workgroups after the bands, rows repaired one-sided), -1
// before any sweep.
thread_local int64_t g_dense_panels = -1;

// Tiles of one band launch [b0, b1) over ntile panels: panel I has
// min(b1, ntile - I) - b0 of them while that is positive.
inline int64_t band_tiles(int64_t ntile, int64_t b0, int64_t b1) {
    const int64_t M = ntile - b0, B = b1 - b0;
    if (M <= 0) return 0;
    return M <= B ? M * (M + 1) / 2 : B * (B + 1) / 2 + (M - B) * B;
}

// Whether the direct-load sweep runs symmetric: by default when there are at
// least 1,024 row panels (n > 261,888), where every band launch still fills
// the GPU; option sweep_sym = 0|1 forces it.
inline bool sweep_sym(int64_t ntile) {
    const int f = option(kOptSweepSym);
    if (f >= 0) return f == 1 && ntile >= 2;
    return ntile >= 1024;
}

// Waves per direct-load workgroup: 16 (64 x 64 wave tiles, the default) or
// 8 (128 x 64; option sweep_waves).
inline int sweep_waves() { return option(kOptSweepWaves) == 8 ? 8 : 16; }

}  // namespace

// Runs the MFMA sweep into the row buffers (bkey/bid/bcnt); the caller sorts.
// fp16 rows: exact products, one term.  fp32 rows: one fp16 term of the
// power-of-two-scaled rows (a screen; the caller re-ranks the survivors in fp32).
// The buffers hold `splits` lists of `cap` per row (sweep_mfma_splits); *used
// returns how many the launched kernel filled (the register-staged kernel
// fills one), which is what the merge must read.
int sweep_mfma_run(const void* X, int x_dtype, int64_t n, int dim, int metric, int C, int cap,
                   int splits, float* bkey, int32_t* bid, int32_t* bcnt, char* extra,
                   hipStream_t st, int* used, const int32_t** perm_out) {
    *perm_out = nullptr;
    g_tiles_scored = 0;
    g_dense_panels = 0;
    const int64_t ntile_all = (n + kBM2 - 1) / kBM2;
    float* xn = (float*)extra; extra += al256(n * 4);
    float* scale = (float*)extra; extra += al256(n * 4);
    const _Float16* hi;
    int scaled = x_dtype == SWANN_DTYPE_F16 ? 0 : 1;
    const unsigned nrb = (unsigned)((n + 3) / 4);
    if (!scaled) {
        hi = (const _Float16*)X;
        hipLaunchKernelGGL(norms_f16, dim3(nrb), dim3(256), 0, st, hi, n, dim, xn, scale);
    } else {
        _Float16* h = (_Float16*)extra;
        extra += al256(n * (int64_t)dim * 2);
        // the row maxima's range (in `scale`, unused until split_rows writes it)
        int* rng = (int*)scale;
        hipLaunchKernelGGL(range_init, dim3(1), dim3(64), 0, st, rng);
        const int vec4 = dim % 4 == 0 && (uintptr_t)X % 16 == 0;
        const unsigned nrr = (unsigned)(nrb < (unsigned)kRangeBlocks ? nrb : kRangeBlocks);
        hipLaunchKernelGGL(row_range, dim3(nrr), dim3(256), 0, st, (const float*)X, n, dim, vec4,
                           rng);
        int hr[2] = {0, 0};
        if (hipMemcpyAsync(hr, rng, sizeof(hr), hipMemcpyDeviceToHost, st) != hipSuccess ||
            hipStreamSynchronize(st) != hipSuccess) {
            set_error("sweep (mfma): reading the rows' range failed");
            return SWANN_E_LAUNCH;
        }
        const float gmax = __builtin_bit_cast(float, hr[0]), gmin = __builtin_bit_cast(float, hr[1]);
        if (gmax <= 16384.f && gmin >= 0.0625f && !option_on(kOptSweepRowscale)) {
            hipLaunchKernelGGL(rows_to_f16, dim3(nrb), dim3(256), 0, st, (const float*)X, n, dim,
                               h, xn);
            scaled = 0;
        } else {
            hipLaunchKernelGGL(split_rows, dim3(nrb), dim3(256), 0, st, (const float*)X, n, dim,
                               h, (_Float16*)nullptr, scale, xn);
        }
        hi = h;
    }
    MfmaSweepArgs a{hi, nullptr, scale, xn, n, dim, metric, C, cap, bkey, bid, bcnt, scaled, 1,
                    0, 0, 0, nullptr, nullptr, cap};
    const unsigned grid = (unsigned)((n + kBM2 - 1) / kBM2);
    const bool ip = metric == SWANN_METRIC_IP;
    *used = 1;
    // the direct loads address a stage's 256 rows with 32-bit byte offsets
    const bool off32 = (int64_t)dim * 2 * kBM2 < (int64_t(1) << 32);
    if (dim % kBK3 == 0 && (uintptr_t)hi % 16 == 0 && off32 && !option_on(kOptSweepRegstage)) {
        const int64_t ntile = (n + kBM2 - 1) / kBM2;
        if (splits >= 2 && sweep_sym(ntile) && sweep_waves() == 16) {
            // symmetric sweep: tile (I, J), J >= I, scored once for the rows of
            // both panels; launched in bands of J - I (1, 1, 2, 4, ... 256, then
            // kBandMax at a time) with a merge after each, so every launch
            // starts from thresholds over everything scored so far.  Two lists
            // a row.
            float* gthr = (float*)extra; extra += al256(n * 4);
            int* ovf = (int*)extra; extra += 256;
            int* mcnt = (int*)extra; extra += al256(n * 4);
            MfmaSweepArgs s = a;
            s.splits = 2;
            s.sym = 1;
            s.gthr = gthr;
            s.ovf = ovf;
            s.mcnt = mcnt;
            s.fcap = cap;
            {                                       // option sweep_sym_fcap: force overflow
                const int f = option(kOptSweepSymFcap);
                if (f >= 1 && f < cap) s.fcap = f;
            }
            // the pruned ordered sweep's tile bounds and lists (set when it runs)
            const unsigned* tlb = nullptr;
            int* dns = nullptr;          // dense panels (dense_mark)
            float* pthr = nullptr;
            int* tlist = nullptr;
            int* tcnt = nullptr;
            unsigned long long* tsum = nullptr;
            // the ordered plane and its groups, kept for the bounded repair
            const _Float16* rhp = nullptr;
            const float* rscp = nullptr;
            const float* rcen = nullptr;
            const float* rpst = nullptr;
            const float* rxnp = nullptr;
            const int* rglist = nullptr;
            int rng = 0;
            int64_t host_tiles = 0;      // tiles of the launches not pruned
            // the launches of bands [b0, bend), each followed by a merge;
            // with `prune`, each launch scores only the tiles tile_keep keeps
            auto bands = [&](MfmaSweepArgs& sa, int64_t bstart, int64_t bend, const float* seed,
                             int* flag, bool prune) -> int {
                for (int64_t b0 = bstart; b0 < bend;) {
                    const int64_t B = b0 == 0 ? 1 : (b0 < kBandMax ? b0 : kBandMax);
                    sa.b0 = b0;
                    sa.b1 = b0 + B < bend ? b0 + B : bend;
                    const unsigned grid = (unsigned)(ntile - b0);
                    if (prune) {
                        hipLaunchKernelGGL(panel_thr, dim3((unsigned)ntile), dim3(256), 0, st,
                                           (const float*)gthr, n, (const int*)dns, pthr);
                        hipLaunchKernelGGL(tile_keep, dim3(grid), dim3(64), 0, st, tlb,
                                           (const int*)dns, (const float*)pthr, (int)ntile,
                                           (int)sa.b0, (int)sa.b1, tlist, tcnt, tsum);
                        sa.tlist = tlist;
                        sa.tcnt = tcnt;
                    } else {
                        sa.tlist = nullptr;
                        sa.tcnt = nullptr;
                        host_tiles += band_tiles(ntile, sa.b0, sa.b1);
                    }
                    if (scaled) {
                        if (ip) hipLaunchKernelGGL((sweep_dma_kernel<SWANN_METRIC_IP, 1, 16>), dim3(grid), dim3(1024), 0, st, sa);
                        else hipLaunchKernelGGL((sweep_dma_kernel<SWANN_METRIC_L2, 1, 16>), dim3(grid), dim3(1024), 0, st, sa);
                    } else {
                        if (ip) hipLaunchKernelGGL((sweep_dma_kernel<SWANN_METRIC_IP, 0, 16>), dim3(grid), dim3(1024), 0, st, sa);
                        else hipLaunchKernelGGL((sweep_dma_kernel<SWANN_METRIC_L2, 0, 16>), dim3(grid), dim3(1024), 0, st, sa);
                    }
                    hipLaunchKernelGGL(sym_merge, dim3((unsigned)((n + 3) / 4)), dim3(256), 0, st,
                                       bkey, bid, bcnt, gthr, ovf, n, cap, sa.fcap, C, seed,
                                       flag, mcnt);
                    const int rc = launch_status("sweep (mfma, symmetric)");
                    if (rc) return rc;
                    b0 = sa.b1;
                }
                return SWANN_OK;
            };
            const unsigned nb256 = (unsigned)((n + 255) / 256);
            float* seed = nullptr;
            int* flag = nullptr;         // rows whose second list overflowed (ordered sweep)
            int* plist = nullptr;
            int* npl = nullptr;
            float* rkey = nullptr;       // the few-panel repair's scratch lists
            int32_t* rid = nullptr;
            int32_t* rcnt = nullptr;
            const int32_t* ordered = nullptr;
            if (ntile > 2 * kSeedBand && !option_on(kOptSweepNoseed)) {
                bool clustered = false;
                // the order's workspace (seed_bytes, repair_bytes)
                float* sk = (float*)extra; extra += al256(n * kSketch * 4);
                int* lab = (int*)extra; extra += al256(n * 4);
                int* perm = (int*)extra; extra += al256(n * 4);
                seed = (float*)extra; extra += al256(n * 4);
                float* xnp = (float*)extra; extra += al256(n * 4);
                float* scp = (float*)extra; extra += al256(n * 4) * 2;
                int* pcnt = (int*)extra; extra += al256(kMaxPivots * 4);
                _Float16* hp = (_Float16*)extra; extra += al256(n * (int64_t)dim * 2);
                flag = (int*)extra; extra += al256(n * 4);
                plist = (int*)extra; extra += al256(ntile * 4);
                npl = (int*)extra; extra += 256;
                float* psk = (float*)extra; extra += al256((int64_t)kMaxPivots * kSketch * 4);
                int* pstart = (int*)extra; extra += al256((kMaxPivots + 1) * 4);
                float* pd = (float*)extra; extra += al256((int64_t)kMaxPivots * kMaxPivots * 4);
                int* prank = (int*)extra; extra += al256(kMaxPivots * 4);
                rkey = (float*)extra; extra += al256((int64_t)kBM2 * kRepairSplits * cap * 4);
                rid = (int32_t*)extra; extra += al256((int64_t)kBM2 * kRepairSplits * cap * 4);
                rcnt = (int32_t*)extra; extra += al256(kBM2 * kRepairSplits * 4);
                const int64_t pw = n / 512;
                const int P = (int)(pw < 1 ? 1 : pw > kMaxPivots ? kMaxPivots : pw);
                if (x_dtype == SWANN_DTYPE_F16)
                    hipLaunchKernelGGL(row_sketch<_Float16>, dim3(nrb), dim3(256), 0, st,
                                       (const _Float16*)X, n, dim, sk);
                else
                    hipLaunchKernelGGL(row_sketch<float>, dim3(nrb), dim3(256), 0, st,
                                       (const float*)X, n, dim, sk);
                hipLaunchKernelGGL(pivot_init, dim3(P), dim3(kSketch), 0, st, sk, n, P, psk);
                // two k-means steps on the sketches, then the final grouping;
                // after the first assignment, rows that do not cluster (mean
                // distance to the nearest pivot above kClusterRatio of that to
                // an arbitrary one) gain nothing from an order or seeds: the
                // sweep then runs plain
                // (the check and the k-means steps on every kSampleStride-th
                // row; the final grouping on all of them)
                float* cacc = (float*)npl + 2;
                for (int it = 0; it <= kKmeanSteps; ++it) {
                    const bool fin = it == kKmeanSteps;
                    const int64_t stride = fin ? 1 : kSampleStride;
                    const int64_t m = fin ? n : (n + kSampleStride - 1) / kSampleStride;
                    hipLaunchKernelGGL(fill_zero, dim3(kMaxPivots / 256), dim3(256), 0, st, pcnt,
                                       kMaxPivots);
                    if (it == 0)
                        hipLaunchKernelGGL(fill_zero, dim3(1), dim3(256), 0, st, (int*)cacc, 2);
                    hipLaunchKernelGGL(nearest_pivot, dim3((unsigned)((m + 255) / 256)), dim3(256),
                                       0, st, sk, m, stride, P, (const float*)psk, lab, pcnt,
                                       it == 0 ? cacc : nullptr);
                    if (it == 0) {
                        float ca[2] = {0.f, 0.f};
                        if (hipMemcpyAsync(ca, cacc, sizeof(ca), hipMemcpyDeviceToHost, st) !=
                                hipSuccess ||
                            hipStreamSynchronize(st) != hipSuccess) {
                            set_error("sweep (mfma): reading the clustering ratio failed");
                            return SWANN_E_LAUNCH;
                        }
                        if (!(ca[0] < kClusterRatio * ca[1])) break;
                        clustered = true;
                    }
                    hipLaunchKernelGGL(pivot_scan, dim3(1), dim3(1024), 0, st, pcnt, pstart, P);
                    hipLaunchKernelGGL(pivot_place, dim3((unsigned)((m + 255) / 256)), dim3(256), 0,
                                       st, lab, m, pcnt, perm);
                    if (!fin)
                        hipLaunchKernelGGL(group_mean, dim3(P), dim3(kSketch), 0, st, sk,
                                           (const int*)perm, (const int*)pstart, stride, psk);
                }
                const bool in_order = clustered && option_on(kOptSweepOrder);
                if (in_order) {
                    // pivots chained nearest to nearest (on the host: P^2
                    // distances), rows ordered by their pivot's place in it
                    hipLaunchKernelGGL(pivot_dist, dim3((unsigned)(((int64_t)P * P + 255) / 256)),
                                       dim3(256), 0, st, (const float*)psk, P, pd);
                    std::vector<float> dh((size_t)P * P);
                    std::vector<int> rank(P), seen(P, 0);
                    if (hipMemcpyAsync(dh.data(), pd, dh.size() * 4, hipMemcpyDeviceToHost, st) !=
                            hipSuccess ||
                        hipStreamSynchronize(st) != hipSuccess) {
                        set_error("sweep (mfma): reading the pivot distances failed");
                        return SWANN_E_LAUNCH;
                    }
                    int cur = 0;
                    seen[0] = 1;
                    rank[0] = 0;
                    for (int i = 1; i < P; ++i) {
                        int best = -1;
                        float bd = INFINITY;
                        const float* row = dh.data() + (size_t)cur * P;
                        for (int q = 0; q < P; ++q)
                            if (!seen[q] && (best < 0 || row[q] < bd)) { best = q; bd = row[q]; }
                        seen[best] = 1;
                        rank[best] = i;
                        cur = best;
                    }
                    if (hipMemcpyAsync(prank, rank.data(), (size_t)P * 4, hipMemcpyHostToDevice,
                                       st) != hipSuccess ||
                        hipStreamSynchronize(st) != hipSuccess) {
                        set_error("sweep (mfma): writing the pivot chain failed");
                        return SWANN_E_LAUNCH;
                    }
                    hipLaunchKernelGGL(fill_zero, dim3(kMaxPivots / 256), dim3(256), 0, st, pcnt,
                                       kMaxPivots);
                    hipLaunchKernelGGL(relabel, dim3(nb256), dim3(256), 0, st, lab, n,
                                       (const int*)prank, pcnt);
                    hipLaunchKernelGGL(pivot_scan, dim3(1), dim3(1024), 0, st, pcnt,
                                       (int*)nullptr, P);
                    hipLaunchKernelGGL(pivot_place, dim3(nb256), dim3(256), 0, st, lab, n, pcnt,
                                       perm);
                }
                if (!clustered) {
                    seed = nullptr;
                    flag = nullptr;
                    goto plain;
                }
                hipLaunchKernelGGL(gather_rows, dim3(nrb), dim3(256), 0, st, hi, n, dim, perm, xn,
                                   scaled ? scale : nullptr, hp, xnp, scp);
                hipLaunchKernelGGL(sym_init, dim3(nb256), dim3(256), 0, st, gthr, bcnt, ovf, n,
                                   (const float*)nullptr, mcnt);
                if (in_order)
                    hipLaunchKernelGGL(fill_zero, dim3(nb256), dim3(256), 0, st, flag, (int)n);
                MfmaSweepArgs pre = s;
                pre.hi = hp;
                pre.xn = xnp;
                pre.scale = scp;
                int rc = launch_status("sweep (mfma, seed order)");
                if (rc) return rc;
                rc = bands(pre, 0, kSeedBand, nullptr, in_order ? flag : nullptr, false);
                if (rc) return rc;
                if (in_order) {
                    // the main sweep in the locality order too: the pre-pass
                    // was its first bands, so it goes on from there, its lists
                    // and thresholds as the last merge left them (ordered ids),
                    // leaving out the tiles the panels' bounds show empty
                    float* cen = (float*)extra; extra += al256(ntile * kSegs * (int64_t)dim * 4);
                    float* pst = (float*)extra; extra += al256(ntile * kSegs * 16);
                    int* nsg = (int*)extra; extra += al256(ntile * 4);
                    pthr = (float*)extra; extra += al256(ntile * 4);
                    tlist = (int*)extra; extra += al256(ntile * kBandMax * 4);
                    tcnt = (int*)extra; extra += al256(ntile * 4);
                    tsum = (unsigned long long*)extra; extra += 256;
                    int* glist = (int*)extra; extra += al256(ntile * kSegs * 4);
                    int* gcnt = (int*)extra; extra += 256;
                    unsigned* tb = (unsigned*)extra; extra += al256(ntile * ntile * 4);
                    int* dn = (int*)extra; extra += al256((ntile + 1) * 4);   // dense[], count
                    int* dl = (int*)extra; extra += al256(ntile * 4);
                    hipLaunchKernelGGL(fill_zero, dim3(1), dim3(256), 0, st, (int*)tsum, 2);
                    // groups split at the thresholds the seed bands left
                    hipLaunchKernelGGL(panel_thr, dim3((unsigned)ntile), dim3(256), 0, st,
                                       (const float*)gthr, n, (const int*)nullptr, pthr);
                    hipLaunchKernelGGL(panel_stats, dim3((unsigned)ntile), dim3(256), 0, st,
                                       (const _Float16*)hp, (const float*)scp, (const float*)xnp,
                                       (const float*)pthr, metric, n, dim, scaled, cen, pst, nsg);
                    // every tile's bound once, from the Gram of the groups' centres
                    hipLaunchKernelGGL(group_list, dim3(1), dim3(1024), 0, st, (const int*)nsg,
                                       (int)ntile, glist, gcnt);
                    int ng = 0;
                    if (hipMemcpyAsync(&ng, gcnt, sizeof(int), hipMemcpyDeviceToHost, st) !=
                            hipSuccess ||
                        hipStreamSynchronize(st) != hipSuccess) {
                        set_error("sweep (mfma): reading the group count failed");
                        return SWANN_E_LAUNCH;
                    }
                    SWANN_REQUIRE(ng >= ntile && ng <= ntile * kSegs,
                                  "sweep: panel group count out of range");
                    hipLaunchKernelGGL(fill_u32, dim3((unsigned)((ntile * ntile + 255) / 256)),
                                       dim3(256), 0, st, tb, ntile * ntile, 0xffffffffu);
                    const unsigned gb = (unsigned)((ng + kGB - 1) / kGB);
                    SWANN_REQUIRE(gb <= 65535, "sweep: too many panel groups for the bound grid");
                    hipLaunchKernelGGL(group_bounds, dim3(gb, gb), dim3(256), 0, st,
                                       (const float*)cen, (const float*)pst, (const int*)glist, ng,
                                       (int)ntile, dim, metric, tb);
                    tlb = tb;
                    rhp = hp;
                    rscp = scp;
                    rxnp = xnp;
                    rcen = cen;
                    rpst = pst;
                    rglist = glist;
                    rng = ng;
                    hipLaunchKernelGGL(fill_zero, dim3((unsigned)((ntile + 256) / 256)), dim3(256), 0,
                                       st, dn, (int)ntile + 1);
                    hipLaunchKernelGGL(dense_mark, dim3((unsigned)ntile), dim3(256), 0, st, tlb,
                                       (const float*)pthr, (int)ntile, (int)kSeedBand, dn, dl,
                                       dn + ntile);
                    int nd = 0;
                    if (hipMemcpyAsync(&nd, dn + ntile, sizeof(int), hipMemcpyDeviceToHost, st) !=
                            hipSuccess ||
                        hipStreamSynchronize(st) != hipSuccess) {
                        set_error("sweep (mfma): reading the dense panel count failed");
                        return SWANN_E_LAUNCH;
                    }
                    SWANN_REQUIRE(nd >= 0 && nd <= ntile, "sweep: dense panel count out of range");
                    // many dense panels (rows that cluster nowhere, spread over most
                    // panels): repairing them would cost more than the bands scoring their
                    // tiles as they are, which then keep about every tile (the plain
                    // sweep's cost, the same lists); also when a tile list cannot hold them
                    if (nd > 0 && nd <= kBandMax && (int64_t)nd * 8 <= ntile) {
                        hipLaunchKernelGGL(dense_flag, dim3((unsigned)nd), dim3(kBM2), 0, st,
                                           (const int*)dl, n, flag, ovf);
                        dns = dn;
                        g_dense_panels = nd;
                    }
                    rc = bands(pre, kSeedBand, ntile, nullptr, flag, true);
                    if (rc) return rc;
                    if (dns) {
                        // the dense launch: tiles (D, J) scored by J's workgroups
                        hipLaunchKernelGGL(panel_thr, dim3((unsigned)ntile), dim3(256), 0, st,
                                           (const float*)gthr, n, (const int*)dns, pthr);
                        int ndl = 0;
                        if (hipMemcpyAsync(&ndl, dn + ntile, sizeof(int), hipMemcpyDeviceToHost,
                                           st) != hipSuccess ||
                            hipStreamSynchronize(st) != hipSuccess) {
                            set_error("sweep (mfma): reading the dense panel count failed");
                            return SWANN_E_LAUNCH;
                        }
                        hipLaunchKernelGGL(dense_keep, dim3((unsigned)ntile), dim3(64), 0, st, tlb,
                                           (const int*)dns, (const int*)dl, ndl,
                                           (const float*)pthr, (int)ntile, (int)kSeedBand, tlist,
                                           tcnt, tsum);
                        MfmaSweepArgs dd = pre;
                        dd.b0 = 0;
                        dd.b1 = ntile;
                        dd.tlist = tlist;
                        dd.tcnt = tcnt;
                        const unsigned gd = (unsigned)ntile;
                        if (scaled) {
                            if (ip) hipLaunchKernelGGL((sweep_dma_kernel<SWANN_METRIC_IP, 1, 16>), dim3(gd), dim3(1024), 0, st, dd);
                            else hipLaunchKernelGGL((sweep_dma_kernel<SWANN_METRIC_L2, 1, 16>), dim3(gd), dim3(1024), 0, st, dd);
                        } else {
                            if (ip) hipLaunchKernelGGL((sweep_dma_kernel<SWANN_METRIC_IP, 0, 16>), dim3(gd), dim3(1024), 0, st, dd);
                            else hipLaunchKernelGGL((sweep_dma_kernel<SWANN_METRIC_L2, 0, 16>), dim3(gd), dim3(1024), 0, st, dd);
                        }
                        hipLaunchKernelGGL(sym_merge, dim3((unsigned)((n + 3) / 4)), dim3(256), 0, st,
                                           bkey, bid, bcnt, gthr, ovf, n, cap, dd.fcap, C,
                                           (const float*)nullptr, flag, mcnt);
                        rc = launch_status("sweep (mfma, dense panels)");
                        if (rc) return rc;
                    }
                    s = pre;
                    seed = nullptr;
                    ordered = perm;
                    goto swept;
                } else {
                    hipLaunchKernelGGL(seed_map, dim3(nb256), dim3(256), 0, st, gthr, perm, xn, n,
                                       seed);
                    flag = nullptr;
                }
            }
        plain:
            hipLaunchKernelGGL(sym_init, dim3(nb256), dim3(256), 0, st, gthr, bcnt, ovf, n,
                               (const float*)seed, mcnt);
            {
                const int rc = bands(s, 0, ntile, seed, flag, false);
                if (rc) return rc;
            }
        swept:
            // a list that overflowed lost candidates: redo the sweep the
            // one-sided way (one small read-back; the build is not on the
            // search path)
            int dropped = 0;
            unsigned long long pruned_kept = 0;
            if (hipMemcpyAsync(&dropped, ovf, sizeof(int), hipMemcpyDeviceToHost, st) !=
                    hipSuccess ||
                (tsum && hipMemcpyAsync(&pruned_kept, tsum, sizeof(pruned_kept),
                                        hipMemcpyDeviceToHost, st) != hipSuccess) ||
                hipStreamSynchronize(st) != hipSuccess) {
                set_error("sweep (mfma, symmetric): reading the overflow count failed");
                return SWANN_E_LAUNCH;
            }
            g_tiles_scored += host_tiles + (int64_t)pruned_kept;
            if (dropped == 0) {
                *used = 2;
                *perm_out = ordered;
                return SWANN_OK;
            }
            if (ordered) {
                // the ordered sweep's repair: the row panels holding a row
                // whose second list overflowed are swept again one-sided
                // (two column halves, lists 0 and 1 of each row written from
                // scratch), so those rows' lists are exact again
                hipLaunchKernelGGL(fill_zero, dim3(1), dim3(256), 0, st, npl, 1);
                hipLaunchKernelGGL(flag_panels, dim3((unsigned)((ntile + 255) / 256)), dim3(256), 0,
                                   st, flag, n, (int)ntile, plist, npl);
                int np = 0;
                if (hipMemcpyAsync(&np, npl, sizeof(int), hipMemcpyDeviceToHost, st) !=
                        hipSuccess ||
                    hipStreamSynchronize(st) != hipSuccess) {
                    set_error("sweep (mfma, symmetric): reading the repair count failed");
                    return SWANN_E_LAUNCH;
                }
                SWANN_REQUIRE(np >= 1 && np <= ntile, "sweep: repair panel count out of range");
                // With the pruned sweep's groups, a repaired panel sweeps only
                // the tiles some row of it can still need, each row against
                // every group at its own threshold (repair_need).  The marks,
                // the rows' stats and the lists take the bands' list space.
                const int* rlist = nullptr;
                const int* rlcnt = nullptr;
                int64_t rtiles = (int64_t)np * ntile;
                const int64_t rspace = 2 * (int64_t)np * ntile + 4 * (int64_t)np * kBM2;
                if (tlb && rcen && rng > 0 && rspace <= ntile * kBandMax) {
                    int* rneed = tlist + (int64_t)np * ntile;
                    double* rst = (double*)(tlist + 2 * (int64_t)np * ntile);
                    hipLaunchKernelGGL(fill_u32, dim3((unsigned)((np * ntile + 255) / 256)),
                                       dim3(256), 0, st, (unsigned*)rneed, (int64_t)np * ntile, 0u);
                    hipLaunchKernelGGL(repair_row_stats, dim3((unsigned)np), dim3(256), 0, st, rhp,
                                       rscp, rxnp, (const int*)plist, n, dim, scaled, rst);
                    hipLaunchKernelGGL(repair_need,
                                       dim3((unsigned)((rng + kGB - 1) / kGB), kBM2 / kGB,
                                            (unsigned)np),
                                       dim3(256), 0, st, rhp, rscp, rcen, rpst, rglist, rng,
                                       (const float*)gthr, (const int*)plist,
                                       (const double*)rst, n, (int)ntile, dim, metric, scaled,
                                       rneed);
                    hipLaunchKernelGGL(fill_zero, dim3(1), dim3(256), 0, st, (int*)tsum, 2);
                    hipLaunchKernelGGL(repair_list, dim3((unsigned)np), dim3(64), 0, st,
                                       (const int*)rneed, (const int*)plist, (int)ntile, tlist,
                                       tcnt, tsum);
                    unsigned long long rt = 0;
                    if (hipMemcpyAsync(&rt, tsum, sizeof(rt), hipMemcpyDeviceToHost, st) !=
                            hipSuccess ||
                        hipStreamSynchronize(st) != hipSuccess) {
                        set_error("sweep (mfma, symmetric): reading the repair tile count failed");
                        return SWANN_E_LAUNCH;
                    }
                    SWANN_REQUIRE(rt >= (unsigned long long)np &&
                                      rt <= (unsigned long long)np * (unsigned long long)ntile,
                                  "sweep: repair tile count out of range");
                    rtiles = (int64_t)rt;
                    rlist = tlist;
                    rlcnt = tcnt;
                }
                // panels repaired one at a time, 16 ways (option sweep_repair_max)
                const int rmax = option(kOptSweepRepairMax);
                if (np <= rmax && C * kRepairSplits <= kRepairSort) {
                    std::vector<int> ph(np);
                    if (hipMemcpyAsync(ph.data(), plist, (size_t)np * 4, hipMemcpyDeviceToHost,
                                       st) != hipSuccess ||
                        hipStreamSynchronize(st) != hipSuccess) {
                        set_error("sweep (mfma, symmetric): reading the repair panels failed");
                        return SWANN_E_LAUNCH;
                    }
                    g_tiles_scored += rtiles;
                    for (int i = 0; i < np; ++i) {
                        SWANN_REQUIRE(ph[i] >= 0 && ph[i] < ntile, "sweep: repair panel out of range");
                        // the one-sided sweep of panel ph[i] into the scratch:
                        // its list addresses are row-absolute, so the bases
                        // are shifted by the panel's first row (only rows of
                        // this panel are touched)
                        const int64_t rb = (int64_t)ph[i] * kBM2;
                        MfmaSweepArgs rep = s;
                        rep.sym = 0;
                        rep.splits = kRepairSplits;
                        rep.plist = plist + i;
                        rep.npl = 1;
                        rep.tlist = rlist ? rlist + (int64_t)i * ntile : nullptr;
                        rep.tcnt = rlist ? rlcnt + i : nullptr;
                        rep.tstride = (int)ntile;
                        rep.bkey = rkey - rb * kRepairSplits * cap;
                        rep.bid = rid - rb * kRepairSplits * cap;
                        rep.bcnt = rcnt - rb * kRepairSplits;
                        const unsigned rg = (unsigned)kRepairSplits;
                        if (scaled) {
                            if (ip) hipLaunchKernelGGL((sweep_dma_kernel<SWANN_METRIC_IP, 1, 16>), dim3(rg), dim3(1024), 0, st, rep);
                            else hipLaunchKernelGGL((sweep_dma_kernel<SWANN_METRIC_L2, 1, 16>), dim3(rg), dim3(1024), 0, st, rep);
                        } else {
                            if (ip) hipLaunchKernelGGL((sweep_dma_kernel<SWANN_METRIC_IP, 0, 16>), dim3(rg), dim3(1024), 0, st, rep);
                            else hipLaunchKernelGGL((sweep_dma_kernel<SWANN_METRIC_L2, 0, 16>), dim3(rg), dim3(1024), 0, st, rep);
                        }
                        hipLaunchKernelGGL(repair_merge, dim3(kBM2), dim3(256), 0, st,
                                           (const float*)rkey, (const int32_t*)rid,
                                           (const int32_t*)rcnt, (int)rb, n, cap, C, ordered, bkey,
                                           bid, bcnt);
                        const int rc = launch_status("sweep (mfma, ordered repair)");
                        if (rc) return rc;
                    }
                    *used = 2;
                    *perm_out = ordered;
                    return SWANN_OK;
                }
                g_tiles_scored += rtiles;
                MfmaSweepArgs rep = s;
                rep.sym = 0;
                rep.splits = 2;
                rep.plist = plist;
                rep.npl = np;
                rep.tlist = rlist;
                rep.tcnt = rlcnt;
                rep.tstride = (int)ntile;
                const unsigned rg = (unsigned)(np * 2);
                if (scaled) {
                    if (ip) hipLaunchKernelGGL((sweep_dma_kernel<SWANN_METRIC_IP, 1, 16>), dim3(rg), dim3(1024), 0, st, rep);
                    else hipLaunchKernelGGL((sweep_dma_kernel<SWANN_METRIC_L2, 1, 16>), dim3(rg), dim3(1024), 0, st, rep);
                } else {
                    if (ip) hipLaunchKernelGGL((sweep_dma_kernel<SWANN_METRIC_IP, 0, 16>), dim3(rg), dim3(1024), 0, st, rep);
                    else hipLaunchKernelGGL((sweep_dma_kernel<SWANN_METRIC_L2, 0, 16>), dim3(rg), dim3(1024), 0, st, rep);
                }
                const int rc = launch_status("sweep (mfma, ordered repair)");
                if (rc) return rc;
                *used = 2;
                *perm_out = ordered;
                return SWANN_OK;
            }
        }
        a.splits = splits;
        *used = splits;
        g_tiles_scored += ntile_all * ntile_all;          // every tile, one-sided
        const unsigned grid = (unsigned)((n + kBM2 - 1) / kBM2 * splits);
        if (sweep_waves() == 16) {
            if (scaled) {
                if (ip) hipLaunchKernelGGL((sweep_dma_kernel<SWANN_METRIC_IP, 1, 16>), dim3(grid), dim3(1024), 0, st, a);
                else hipLaunchKernelGGL((sweep_dma_kernel<SWANN_METRIC_L2, 1, 16>), dim3(grid), dim3(1024), 0, st, a);
            } else {
                if (ip) hipLaunchKernelGGL((sweep_dma_kernel<SWANN_METRIC_IP, 0, 16>), dim3(grid), dim3(1024), 0, st, a);
                else hipLaunchKernelGGL((sweep_dma_kernel<SWANN_METRIC_L2, 0, 16>), dim3(grid), dim3(1024), 0, st, a);
            }
        } else if (scaled) {
            if (ip) hipLaunchKernelGGL((sweep_dma_kernel<SWANN_METRIC_IP, 1, 8>), dim3(grid), dim3(kT2), 0, st, a);
            else hipLaunchKernelGGL((sweep_dma_kernel<SWANN_METRIC_L2, 1, 8>), dim3(grid), dim3(kT2), 0, st, a);
        } else {
            if (ip) hipLaunchKernelGGL((sweep_dma_kernel<SWANN_METRIC_IP, 0, 8>), dim3(grid), dim3(kT2), 0, st, a);
            else hipLaunchKernelGGL((sweep_dma_kernel<SWANN_METRIC_L2, 0, 8>), dim3(grid), dim3(kT2), 0, st, a);
        }
        return launch_status("sweep (mfma, direct loads)");
    }
    g_tiles_scored += ntile_all * ntile_all;
    if (scaled) {
        if (ip) hipLaunchKernelGGL((sweep_mfma256_kernel<SWANN_METRIC_IP, 1>), dim3(grid), dim3(kT2), 0, st, a);
        else hipLaunchKernelGGL((sweep_mfma256_kernel<SWANN_METRIC_L2, 1>), dim3(grid), dim3(kT2), 0, st, a);
    } else {
        if (ip) hipLaunchKernelGGL((sweep_mfma256_kernel<SWANN_METRIC_IP, 0>), dim3(grid), dim3(kT2), 0, st, a);
        else hipLaunchKernelGGL((sweep_mfma256_kernel<SWANN_METRIC_L2, 0>), dim3(grid), dim3(kT2), 0, st, a);
    }
    return launch_status("sweep (mfma)");
}

// Extra workspace: norms, scales, (fp32 corpus) the fp16 plane, the
// symmetric sweep's thresholds and overflow count, and its seed pre-pass.
int64_t sweep_mfma_extra_bytes(int64_t n, int dim, int x_dtype) {
    const int64_t planes = x_dtype == SWANN_DTYPE_F16 ? 0 : 1;
    const int64_t base = al256(n * 4) * 2 + planes * al256(n * (int64_t)dim * 2) +
                         al256(n * 4) + 256 + al256(n * 4);
    // the locality order, seeds and panel repair run only in the symmetric
    // direct-load sweep past its seed bands; only a sweep that may take that
    // path reserves their scratch (a superset of the run's conditions, so the
    // run never finds less than it needs: a corpus the clustering check
    // declines at run time, or option sweep_noseed, still reserves it)
    const int64_t ntile = (n + kBM2 - 1) / kBM2;
    const bool seeded = dim % kBK3 == 0 && sweep_sym(ntile) && ntile > 2 * kSeedBand;
    return base + (seeded ? seed_bytes(n, dim) + repair_bytes(1024) : 0);   // cap <= 1024
}

// Column splits of the direct-load sweep: enough workgroups to give every
// CU one (small n), and at least kMinSplits so that row panels are read from
// L2 more than once.
#ifndef SWANN_SWEEP_MIN_SPLITS
#define SWANN_SWEEP_MIN_SPLITS 2
#endif
int sweep_mfma_splits(int64_t n, int dim) {
    if (dim % kBK3 != 0) return 1;
    const int64_t ntile = (n + kBM2 - 1) / kBM2;
    int g = SWANN_SWEEP_MIN_SPLITS;
    while (g < 8 && ntile * g < 512) g *= 2;
    return g;
}

int sweep_mfma_cap(int C) {
    // room for one 256-column tile of appends above the C kept
    int cap = C + 768;
    return cap > 1024 ? 1024 : cap;
}

}  // namespace swann

extern "C" int64_t swann_sweep_tiles_scored(void) { return swann::g_tiles_scored; }
extern "C" int64_t swann_sweep_dense_panels(void) { return swann::g_dense_panels; }
