// Graph build: exact candidate sweep, alpha robust prune, reverse edges
// (swann/build.py:14-171).
//
// sweep    a tiled distance GEMM over [row tile] x [all columns] whose tiles
//          never leave the chip: each score is tested against its row's
//          running threshold and only survivors are appended to a per-row
//          buffer in the workspace; a full buffer is compacted in place to
//          its C best (exact radix-style threshold search), so the n^2
//          scores cost no HBM traffic.  A last pass sorts each row.
// prune    one workgroup per node: the C x C Gram of its candidates is built
//          in LDS (upper triangle), then one wave applies the sequential
//          rule  take_i = room && !exists kept w: alpha * d(w, i) <= d(u, i).
// reverse  in-degree count, exclusive scan, scatter; then per node the
//          ascending-source first max_in in-edges are joined to its row,
//          deduped, scored exactly, sorted, cut to 128 and pruned.
#include <float.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "common.h"

namespace swann {

int64_t sweep_mfma_extra_bytes(int64_t n, int dim, int x_dtype);
int sweep_mfma_cap(int C);
int sweep_mfma_splits(int64_t n, int dim);
int sweep_mfma_run(const void* X, int x_dtype, int64_t n, int dim, int metric, int C, int cap,
                   int splits, float* bkey, int32_t* bid, int32_t* bcnt, char* extra,
                   hipStream_t st, int* used, const int32_t** perm_out);

namespace {

template <typename XT> __device__ __forceinline__ float ld(const XT* p) { return (float)*p; }

constexpr float kSelf = 3.4e38f;          // build.py:39
constexpr int kRT = 64, kCT = 64, kKT = 16;
constexpr int kMaxC = 256;                 // candidates per row the sweep may keep
constexpr int kPruneMaxC = 128;
constexpr int kBig = 1 << 30;

__device__ __forceinline__ bool lt(float da, int ia, float db, int ib) {
    return (da < db) || (da == db && ia < ib);
}

// float -> uint32 whose unsigned order is the float order
__device__ __forceinline__ uint32_t fkey(float f) {
    const uint32_t b = __float_as_uint(f);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float funkey(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

__device__ __forceinline__ float pair_formula(float dot, float na, float nb, int metric) {
    if (metric == SWANN_METRIC_IP) return 1.0f - dot;
    const float v = (nb - 2.0f * dot) + na;
    return v < 0.f ? 0.f : v;
}

template <typename XT>
__global__ __launch_bounds__(256) void norms_kernel(const XT* __restrict__ A, int64_t n,
                                                    int dim, float* __restrict__ out) {
    const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (r >= n) return;
    const XT* a = A + r * dim;
    float s = 0.f;
    for (int t = lane; t < dim; t += 64) { const float v = ld(a + t); s = __builtin_fmaf(v, v, s); }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
    if (lane == 0) out[r] = s;
}

// ---------------------------------------------------------------------------
// sweep
struct SweepArgs {
    const void* X; const float* xn; int64_t n; int dim; int metric; int C; int cap;
    float* bkey; int32_t* bid; int32_t* bcnt;
};

// Wave-cooperative compaction of one row's buffer to its C best.
__device__ void compact_row(float* key, int32_t* id, int cnt, int C, float* thr_out,
                            int* cnt_out) {
    const int lane = threadIdx.x & 63;
    constexpr int R = 16;                      // cap <= 1024
    uint32_t u[R];
#pragma unroll
    for (int t = 0; t < R; ++t) {
        const int i = t * 64 + lane;
        u[t] = i < cnt ? fkey(key[i]) : 0xffffffffu;
    }
    // smallest T with #{u <= T} >= C
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
    int eq_left = C - nlt;                     // copies of T still to keep, index order
    int w = 0;
#pragma unroll
    for (int t = 0; t < R; ++t) {
        const int i = t * 64 + lane;
        const bool in = i < cnt;
        const bool is_lt = in && u[t] < T;
        const bool is_eq = in && u[t] == T;
        const uint64_t meq = __ballot(is_eq);
        const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
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

template <typename XT>
__global__ __launch_bounds__(256) void sweep_kernel(SweepArgs a) {
    const XT* X = reinterpret_cast<const XT*>(a.X);
    __shared__ float As[kKT][kRT + 4];
    __shared__ float Bs[kKT][kCT + 4];
    __shared__ float thr[kRT];
    __shared__ int cnt[kRT];
    __shared__ int need;
    const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
    const int wave = tid >> 6;
    const int64_t r0 = (int64_t)blockIdx.x * kRT;
    const int dim = a.dim;
    const int lr = tid >> 2, lk = (tid & 3) * 4;
    if (tid < kRT) { thr[tid] = INFINITY; cnt[tid] = 0; }
    if (tid == 0) need = 0;
    __syncthreads();
    float rn[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int64_t r = r0 + ty * 4 + i;
        rn[i] = (a.metric == SWANN_METRIC_L2 && r < a.n) ? a.xn[r] : 0.f;
    }
    for (int64_t c0 = 0; c0 < a.n; c0 += kCT) {
        float acc[4][4] = {};
        for (int k0 = 0; k0 < dim; k0 += kKT) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int k = k0 + lk + e;
                const int64_t ar = r0 + lr, bc = c0 + lr;
                As[lk + e][lr] = (ar < a.n && k < dim) ? ld(X + ar * dim + k) : 0.f;
                Bs[lk + e][lr] = (bc < a.n && k < dim) ? ld(X + bc * dim + k) : 0.f;
            }
            __syncthreads();
#pragma unroll
            for (int k = 0; k < kKT; ++k) {
                float av[4], bv[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) av[i] = As[k][ty * 4 + i];
#pragma unroll
                for (int j = 0; j < 4; ++j) bv[j] = Bs[k][tx * 4 + j];
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_fmaf(av[i], bv[j], acc[i][j]);
            }
            __syncthreads();
        }
        // screen against each row's threshold; append survivors
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int rl = ty * 4 + i;
            const int64_t r = r0 + rl;
            if (r >= a.n) continue;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int64_t c = c0 + tx * 4 + j;
                if (c >= a.n) continue;
                const float cn = a.metric == SWANN_METRIC_L2 ? a.xn[c] : 0.f;
                const float d = (c == r) ? kSelf : pair_formula(acc[i][j], rn[i], cn, a.metric);
                if (d < thr[rl]) {
                    const int p = atomicAdd(&cnt[rl], 1);
                    a.bkey[r * a.cap + p] = d;
                    a.bid[r * a.cap + p] = (int32_t)c;
                }
            }
        }
        __syncthreads();
        // any row that could overflow on the next tile is compacted now
        if (tid < kRT && cnt[tid] > a.cap - kCT) atomicOr(&need, 1);
        __syncthreads();
        if (need) {
            for (int rl = wave; rl < kRT; rl += 4) {
                const int64_t r = r0 + rl;
                if (r < a.n && cnt[rl] > a.cap - kCT)
                    compact_row(a.bkey + r * a.cap, a.bid + r * a.cap, cnt[rl], a.C, &thr[rl],
                                &cnt[rl]);
            }
            __syncthreads();
            if (tid == 0) need = 0;
            __syncthreads();
        }
    }
    if (tid < kRT && r0 + tid < a.n) a.bcnt[r0 + tid] = cnt[tid];
}

// Sort each row's survivors and emit the first C.  A row has G lists
// (column splits of the sweep) of up to `cap` entries at (r * G + s) * cap;
// they are gathered in split order and sorted together.  With perm (the
// sweep ran on the rows in that order), list r is row perm[r]'s and an id j
// means row perm[j]: ids are mapped before the (d, id) sort, so ties order
// by the rows' own ids, and the row is written at perm[r].
__global__ __launch_bounds__(256) void sweep_final(const float* __restrict__ bkey,
                                                   const int32_t* __restrict__ bid,
                                                   const int32_t* __restrict__ bcnt, int64_t n,
                                                   int cap, int G, int C, int pad_self,
                                                   const int32_t* __restrict__ perm,
                                                   int32_t* __restrict__ cand,
                                                   float* __restrict__ cdist) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int64_t r = blockIdx.x;
    const int64_t ro = perm ? (int64_t)perm[r] : r;       // the row written
    int segc[8], cnt = 0;
    for (int sg = 0; sg < 8; ++sg) {
        segc[sg] = sg < G ? bcnt[r * G + sg] : 0;
        cnt += segc[sg];
    }
    int np = 2;
    while (np < cnt) np <<= 1;
    float* sd = reinterpret_cast<float*>(smem);
    int* si = reinterpret_cast<int*>(sd + np);
    for (int i = threadIdx.x; i < np; i += 256) {
        int sg = 0, off = i;
        while (sg < G - 1 && off >= segc[sg]) { off -= segc[sg]; ++sg; }
        const bool real = i < cnt;
        const int64_t at = (r * G + sg) * (int64_t)cap + off;
        sd[i] = real ? bkey[at] : INFINITY;
        si[i] = real ? (perm ? perm[bid[at]] : bid[at]) : INT32_MAX;
    }
    __syncthreads();
    for (int size = 2; size <= np; size <<= 1)
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int i = threadIdx.x; i < np; i += 256) {
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
    // pad_self: the sweep left self out of the lists; it is the row's
    // candidate at 3.4e38 after every real one (swann/build.py:28-43 sets the
    // self score so), so it takes position cnt when the row has fewer than C
    for (int t = threadIdx.x; t < C; t += 256) {
        const bool ok = t < cnt;
        const bool self = pad_self && t == cnt;
        cand[ro * C + t] = ok ? si[t] : self ? (int32_t)ro : -1;
        cdist[ro * C + t] = ok ? sd[t] : self ? kSelf : INFINITY;
    }
}

// ---------------------------------------------------------------------------
// prune: one workgroup (256 threads) per node
constexpr int kPKC = 16;

__device__ __forceinline__ int tri(int w, int i) { return i * (i - 1) / 2 + w; }   // w < i

typedef _Float16 h16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16v __attribute__((ext_vector_type(16)));

typedef float f32x4v __attribute__((ext_vector_type(4)));

// The Gram with the candidate rows staged through LDS, 128 bytes of each
// row at a time (64 halves or 32 floats), so every row is read from memory
// once per node instead of once per wave that needs it.  Each 16-byte chunk c
// of row r sits at chunk c ^ swz(r) (the 32 rows of a fragment read fall in
// distinct banks).  A K chunk is four steps; in step t lane l reads chunk
// 2t + l/32 of its row: fp16 -- 8 halves, one 32x32x16 MFMA; fp32 -- 4
// floats, four 32x32x2 MFMAs (k = 4*(l/32) + s of the step's 8, a
// permutation of the K order, which a sum over k does not see).  Products
// are exact (fp16) or fp32 (fp32), sums fp32.  dim % 8 (fp16: % 16) == 0.
//
// PLANES (fp32 rows): each staged float y = x / s_r (s_r a power of two with
// |y| < 2^15 for the whole row) is split into hi = fp16(y) and lo =
// fp16(y - hi) (y - hi is exact in fp32), hi in logical chunks 0-3 of the
// row's 128 bytes, lo in 4-7; the Gram entry is s_a s_b (hi.hi + hi.lo +
// lo.hi), three 32x32x16 f16 MFMAs per 16 of K into one fp32 accumulator
// (exact products, fp32 sums) for what the fp32 path does in eight 32x32x2
// f32 MFMAs.  y keeps 22 of its 24 significant bits (the lo.lo term and lo's
// own rounding are below 2^-22 of the element; lo is subnormal only for
// elements below 2^-17 of the row's largest), so the Gram differs from the
// fp32 one by a few of its last bits, like a different summation order.
constexpr int kStgRow = 128;                       // bytes of a row per K chunk
typedef _Float16 h16x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ int pswz(int r) { return (r & 7) ^ ((r >> 3) & 1); }

template <typename XT, bool PLANES = false>
__device__ void gram_mfma_staged(const XT* __restrict__ X, int64_t n, int dim, const int* cid,
                                 int C, float* gram, float* vn, unsigned char* stg,
                                 const float* srow = nullptr) {
    static_assert(!PLANES || sizeof(XT) == 4, "the split planes are for fp32 rows");
    constexpr int EPC = 16 / sizeof(XT);           // elements per 16-byte chunk
    constexpr int KC = kStgRow / sizeof(XT);       // elements of a row per K chunk
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    // the 10 upper-triangle 32 x 32 tiles (i <= j) of the 128 x 128 Gram,
    // three or two per wave (a wave per row block would give wave 0 four
    // and wave 3 one); tiles past C (one past the last valid candidate)
    // are skipped
    constexpr int kTI[4][3] = {{0, 0, 0}, {0, 1, 1}, {1, 2, -1}, {2, 3, -1}};
    constexpr int kTJ[4][3] = {{0, 1, 2}, {3, 1, 2}, {3, 2, -1}, {3, 3, -1}};
    int ti[3], tj[3];
    bool on[3];
#pragma unroll
    for (int x = 0; x < 3; ++x) {
        ti[x] = kTI[w][x];
        tj[x] = kTJ[w][x];
        on[x] = ti[x] >= 0 && ti[x] * 32 < C && tj[x] * 32 < C;
    }
    const bool busy = on[0] || on[1] || on[2];
    f32x16v acc[3];
#pragma unroll
    for (int x = 0; x < 3; ++x)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[x][e] = 0.f;
    const int half = lane >> 5;
    // staging: 128 rows x 8 chunks, 4 per thread; two K chunks' loads are in
    // flight ahead of the chunk being multiplied (the kernel waits on memory
    // latency, not on its MFMAs).  The loads are unconditional -- a lane past
    // the candidates or the row reads element 0 of the corpus and its bit in
    // the chunk's mask zeroes it at staging -- so that the compiler counts
    // them exactly and each staging waits only for its own chunk.
    const int rows = (C + 31) & ~31;               // rows some tile reads
    int sid[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int r = (q * 256 + tid) >> 3;
        const int id = r < C ? cid[r] : -1;
        sid[q] = r < rows && id >= 0 && id < n ? id : -1;
    }
    uint4 nxa[4], nxb[4];
    unsigned oka = 0u, okb = 0u;
    auto fetch = [&](uint4* dst, unsigned& okm, int k0) {
        okm = 0u;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int k = k0 + ((q * 256 + tid) & 7) * EPC;
            const bool ok = sid[q] >= 0 && k < dim;
            const int64_t off = ok ? (int64_t)sid[q] * dim + k : 0;
            dst[q] = *reinterpret_cast<const uint4*>(X + off);
            okm |= (ok ? 1u : 0u) << q;
        }
    };
    // thread t stages rows (q 256 + t) / 8 < 128 of every chunk (all of the
    // buffer; rows past the candidates stage zeros), with its rows' scales
    float inv[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) inv[q] = PLANES ? 1.f / srow[(q * 256 + tid) >> 3] : 1.f;
    auto stage = [&](const uint4* src, unsigned okm) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int e = q * 256 + tid;
            const int r = e >> 3, c = e & 7;
            const uint4 raw = ((okm >> q) & 1u) ? src[q] : make_uint4(0u, 0u, 0u, 0u);
            if constexpr (PLANES) {
                // floats 4c..4c+3 of the chunk: their hi halves to byte 8c of
                // the hi plane (logical chunk c/2), lo to the lo plane
                const f32x4v v = __builtin_bit_cast(f32x4v, raw);
                h16x4 hi, lo;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float y = v[i] * inv[q];
                    const _Float16 h = (_Float16)y;
                    hi[i] = h;
                    lo[i] = (_Float16)(y - (float)h);
                }
                unsigned char* row = stg + r * kStgRow + ((c & 1) << 3);
                *reinterpret_cast<uint2*>(row + (((c >> 1) ^ pswz(r)) << 4)) =
                    __builtin_bit_cast(uint2, hi);
                *reinterpret_cast<uint2*>(row + (((4 + (c >> 1)) ^ pswz(r)) << 4)) =
                    __builtin_bit_cast(uint2, lo);
            } else {
                *reinterpret_cast<uint4*>(stg + r * kStgRow + ((c ^ pswz(r)) << 4)) = raw;
            }
        }
    };
    auto multiply = [&]() {
        if (PLANES && busy) {
            // 32 of K a chunk: two 16-wide steps of hi.hi, hi.lo and lo.hi,
            // all into one accumulator
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                const int chh = 2 * t + half, chl = 4 + 2 * t + half;
#pragma unroll
                for (int x = 0; x < 3; ++x) {
                    if (!on[x]) continue;
                    const int ar = ti[x] * 32 + (lane & 31);
                    const int br = tj[x] * 32 + (lane & 31);
                    const h16x8 ah = __builtin_bit_cast(h16x8, *reinterpret_cast<const uint4*>(
                        stg + ar * kStgRow + ((chh ^ pswz(ar)) << 4)));
                    const h16x8 al = __builtin_bit_cast(h16x8, *reinterpret_cast<const uint4*>(
                        stg + ar * kStgRow + ((chl ^ pswz(ar)) << 4)));
                    const h16x8 bh = __builtin_bit_cast(h16x8, *reinterpret_cast<const uint4*>(
                        stg + br * kStgRow + ((chh ^ pswz(br)) << 4)));
                    const h16x8 bl = __builtin_bit_cast(h16x8, *reinterpret_cast<const uint4*>(
                        stg + br * kStgRow + ((chl ^ pswz(br)) << 4)));
                    acc[x] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, bh, acc[x], 0, 0, 0);
                    acc[x] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, bl, acc[x], 0, 0, 0);
                    acc[x] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al, bh, acc[x], 0, 0, 0);
                }
            }
        } else if (busy) {
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const int ch = 2 * t + half;
#pragma unroll
                for (int x = 0; x < 3; ++x) {
                    if (!on[x]) continue;
                    const int ar = ti[x] * 32 + (lane & 31);
                    const int br = tj[x] * 32 + (lane & 31);
                    const uint4 ra = *reinterpret_cast<const uint4*>(stg + ar * kStgRow +
                                                                     ((ch ^ pswz(ar)) << 4));
                    const uint4 rb = *reinterpret_cast<const uint4*>(stg + br * kStgRow +
                                                                     ((ch ^ pswz(br)) << 4));
                    if constexpr (sizeof(XT) == 2) {
                        acc[x] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
                            __builtin_bit_cast(h16x8, ra), __builtin_bit_cast(h16x8, rb), acc[x],
                            0, 0, 0);
                    } else {
                        const f32x4v fa = __builtin_bit_cast(f32x4v, ra);
                        const f32x4v fb = __builtin_bit_cast(f32x4v, rb);
#pragma unroll
                        for (int s2 = 0; s2 < 4; ++s2)
                            acc[x] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[s2], fb[s2], acc[x],
                                                                          0, 0, 0);
                    }
                }
            }
        }
    };
    // Every fetch is issued, also past the last chunk (then of chunk 0 again,
    // which is never staged): with no fetch under a branch, each staging
    // waits for its own four loads only (vmcnt(4)), not for the next chunk's.
    // Two chunks a trip and no exit inside it, so that at the top of the loop
    // the compiler sees buffer a's loads as the older ones on every path; an
    // odd last chunk runs after the loop.
    const int nch = (dim + KC - 1) / KC;
    fetch(nxa, oka, 0);
    fetch(nxb, okb, nch > 1 ? KC : 0);
    int ch = 0;
    for (; ch + 1 < nch; ch += 2) {
        stage(nxa, oka);
        __syncthreads();
        fetch(nxa, oka, ch + 2 < nch ? (ch + 2) * KC : 0);
        multiply();
        __syncthreads();
        stage(nxb, okb);
        __syncthreads();
        fetch(nxb, okb, ch + 3 < nch ? (ch + 3) * KC : 0);
        multiply();
        __syncthreads();
    }
    if (ch < nch) {
        stage(nxa, oka);
        __syncthreads();
        multiply();
        __syncthreads();
    }
    if (!busy) return;
#pragma unroll
    for (int x = 0; x < 3; ++x) {
        if (!on[x]) continue;
        const int cc = tj[x] * 32 + (lane & 31);
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int r = ti[x] * 32 + (e >> 2) * 8 + (lane >> 5) * 4 + (e & 3);
            if (r < C && cc < C) {
                float g = acc[x][e];
                if constexpr (PLANES) g = (srow[r] * srow[cc]) * acc[x][e];
                if (r < cc) gram[tri(r, cc)] = g;
                else if (r == cc) vn[r] = g;
            }
        }
    }
}

// Per fp32 row, the power of two s with max |x| / s < 2^15 (1 for a zero or
// non-finite row): the scale of its split planes.  One wave a row.
__global__ __launch_bounds__(256) void row_scale(const float* __restrict__ X, int64_t n, int dim,
                                                 float* __restrict__ scale) {
    const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= n) return;
    const int lane = threadIdx.x & 63;
    float m = 0.f;
    for (int k = lane; k < dim; k += 64) m = fmaxf(m, fabsf(X[r * dim + k]));
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
    if (lane == 0) {
        float sc = 1.f;
        if (m > 0.f && m <= FLT_MAX) {
            int e;
            frexpf(m, &e);                       // m < 2^e
            sc = ldexpf(1.f, e - 15 < -126 ? -126 : e - 15);
        }
        scale[r] = sc;
    }
}

// At least two workgroups a CU: the split-plane Gram's fragments and its six
// accumulator tiles otherwise take 300 registers a wave, one workgroup a CU.
template <typename XT, bool MFMA, bool PLANES = false>
__global__ __launch_bounds__(256, 2) void prune_kernel(const XT* __restrict__ X, int64_t n,
                                                    int dim, int metric,
                                                    const int32_t* __restrict__ cand,
                                                    const float* __restrict__ cdist, int C,
                                                    int deg, float alpha,
                                                    const int32_t* __restrict__ dpn,
                                                    const uint8_t* __restrict__ protect,
                                                    int32_t* __restrict__ out,
                                                    const float* __restrict__ rscale = nullptr,
                                                    const int32_t* __restrict__ order = nullptr) {
    __shared__ float gram[kPruneMaxC * (kPruneMaxC - 1) / 2];
    __shared__ float vn[kPruneMaxC];
    __shared__ float Vs[MFMA ? 1 : kPKC][kPruneMaxC + 4];
    __shared__ int cid[kPruneMaxC];
    __shared__ float cdu[kPruneMaxC];
    // with an order, consecutive entries (nodes sharing candidates) on one XCD
    const int64_t u = order ? (int64_t)order[xcd_remap(blockIdx.x, gridDim.x)]
                            : (int64_t)blockIdx.x;
    const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
    for (int i = tid; i < C; i += 256) {
        const int c = cand[u * C + i];
        cid[i] = c;
        cdu[i] = cdist[u * C + i];
    }
    __syncthreads();
    if constexpr (MFMA) {
        // candidates past the last valid one are never read: the Gram stops there
        __shared__ __align__(16) unsigned char stg[kPruneMaxC * kStgRow];
        __shared__ float srow[PLANES ? kPruneMaxC : 1];
        __shared__ int s_nv;
        if (tid == 0) s_nv = 0;
        if constexpr (PLANES) {
            for (int i = tid; i < kPruneMaxC; i += 256) {
                const int c = i < C ? cid[i] : -1;
                srow[i] = (c >= 0 && c < n) ? rscale[c] : 1.f;
            }
        }
        __syncthreads();
        for (int i = tid; i < C; i += 256)
            if (cid[i] >= 0 && cid[i] < n) atomicMax(&s_nv, i + 1);
        __syncthreads();
        gram_mfma_staged<XT, PLANES>(X, n, dim, cid, s_nv, gram, vn, stg, srow);
    } else {
    // thread (ty, tx) accumulates Gram rows ty*8.., columns tx*8.. (C <= 128)
    float acc[8][8] = {};
    const bool active = (ty * 8 < C) && (tx * 8 < C) && (tx >= ty);
    for (int k0 = 0; k0 < dim; k0 += kPKC) {
        for (int e = tid; e < kPKC * C; e += 256) {
            const int i = e / kPKC, kk = e % kPKC;
            const int c = cid[i];
            const int k = k0 + kk;
            Vs[kk][i] = (c >= 0 && c < n && k < dim) ? ld(X + (int64_t)c * dim + k) : 0.f;
        }
        __syncthreads();
        if (active) {
#pragma unroll
            for (int kk = 0; kk < kPKC; ++kk) {
                float av[8], bv[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) av[i] = Vs[kk][ty * 8 + i];
#pragma unroll
                for (int j = 0; j < 8; ++j) bv[j] = Vs[kk][tx * 8 + j];
#pragma unroll
                for (int i = 0; i < 8; ++i)
#pragma unroll
                    for (int j = 0; j < 8; ++j) acc[i][j] = __builtin_fmaf(av[i], bv[j], acc[i][j]);
            }
        }
        __syncthreads();
    }
    if (active) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int w = ty * 8 + i;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int c = tx * 8 + j;
                if (w < C && c < C) {
                    if (w < c) gram[tri(w, c)] = acc[i][j];
                    else if (w == c) vn[w] = acc[i][j];
                }
            }
        }
    }
    }
    __syncthreads();
    // The sequential rule, one wave.  Every decision is wave-uniform, so the
    // kept list lives in registers: lane t holds kept[t] and kept[64 + t].
    // Node u keeps at most min(dpn[u], deg); a protected candidate skips the
    // detour test (build.py:78-81).
    if (tid < 64) {
        const int lane = tid;
        int k0 = -1, k1 = -1;
        int nk = 0;
        int cap = deg;
        if (dpn) { const int c = dpn[u]; cap = c < cap ? c : cap; }
        for (int i = 0; i < C && nk < cap; ++i) {
            if (cid[i] < 0) continue;
            const float du = cdu[i];
            bool v = false;
            const bool prot = protect && protect[u * C + i];
            if (!prot && lane < nk)
                v = alpha * pair_formula(gram[tri(k0, i)], vn[k0], vn[i], metric) <= du;
            if (!prot && 64 + lane < nk)
                v = v || alpha * pair_formula(gram[tri(k1, i)], vn[k1], vn[i], metric) <= du;
            if (__ballot(v) == 0ull) {
                if (nk < 64) { if (lane == nk) k0 = i; }
                else if (lane == nk - 64) k1 = i;
                ++nk;
            }
        }
        if (lane < deg) out[u * deg + lane] = lane < nk ? cid[k0] : -1;
        if (64 + lane < deg) out[u * deg + 64 + lane] = 64 + lane < nk ? cid[k1] : -1;
    }
}

// ---------------------------------------------------------------------------
// reverse
__global__ void fill_i32(int32_t* p, int64_t n, int32_t v) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

__global__ void rev_count(const int32_t* __restrict__ G, int64_t n, int deg,
                          int32_t* __restrict__ cnt) {
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= n * deg) return;
    const int v = G[e];
    if (v >= 0 && v < n) atomicAdd(&cnt[v], 1);
}

// exclusive scan of cnt[n] into start[n], one workgroup, in chunks of 1024
__global__ __launch_bounds__(1024) void scan_kernel(const int32_t* __restrict__ cnt, int64_t n,
                                                    int32_t* __restrict__ start) {
    __shared__ int buf[1024];
    __shared__ int carry;
    if (threadIdx.x == 0) carry = 0;
    __syncthreads();
    for (int64_t b = 0; b < n; b += 1024) {
        const int64_t i = b + threadIdx.x;
        const int v = i < n ? cnt[i] : 0;
        buf[threadIdx.x] = v;
        __syncthreads();
        for (int off = 1; off < 1024; off <<= 1) {
            const int t = threadIdx.x >= off ? buf[threadIdx.x - off] : 0;
            __syncthreads();
            buf[threadIdx.x] += t;
            __syncthreads();
        }
        if (i < n) start[i] = carry + buf[threadIdx.x] - v;
        __syncthreads();
        if (threadIdx.x == 1023) carry += buf[1023];
        __syncthreads();
    }
}

__global__ void rev_scatter(const int32_t* __restrict__ G, int64_t n, int deg,
                            const int32_t* __restrict__ start, int32_t* __restrict__ fill,
                            int32_t* __restrict__ src) {
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= n * deg) return;
    const int v = G[e];
    if (v < 0 || v >= n) return;
    const int p = atomicAdd(&fill[v], 1);
    src[start[v] + p] = (int32_t)(e / deg);
}

__device__ void block_sort_int(int* s, int np) {
    for (int size = 2; size <= np; size <<= 1)
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int i = threadIdx.x; i < np; i += 256) {
                const int j = i ^ stride;
                if (j > i) {
                    const bool up = ((i & size) == 0);
                    if (up != (s[i] < s[j])) { const int t = s[i]; s[i] = s[j]; s[j] = t; }
                }
            }
            __syncthreads();
        }
}

constexpr int kRevBuf = 2048;

// Per node: first max_in in-sources (ascending), union with G_u, minus self,
// dedup, exact distances, ascending (d, id), the first keepn.
template <typename XT>
__global__ __launch_bounds__(256) void rev_assemble(const XT* __restrict__ X, int64_t n,
                                                    int dim, int metric,
                                                    const int32_t* __restrict__ G, int deg,
                                                    int max_in,
                                                    const int32_t* __restrict__ cnt,
                                                    const int32_t* __restrict__ start,
                                                    const int32_t* __restrict__ src, int keepn,
                                                    int32_t* __restrict__ cand2,
                                                    float* __restrict__ cd2,
                                                    const int32_t* __restrict__ order) {
    __shared__ int ib[kRevBuf];
    __shared__ int row[512];
    __shared__ float rd[512];
    __shared__ float xu[4096];
    // with an order, consecutive entries (nodes sharing neighbours) on one XCD
    const int64_t u = order ? (int64_t)order[xcd_remap(blockIdx.x, gridDim.x)]
                            : (int64_t)blockIdx.x;
    const int tid = threadIdx.x;
    const int cu = cnt[u];
    const int64_t s0 = start[u];
    // smallest max_in sources, running over chunks
    int keep = 0;
    for (int c0 = 0; c0 < cu;) {
        const int take = (cu - c0) < (kRevBuf - keep) ? (cu - c0) : (kRevBuf - keep);
        const int fill = keep + take;
        int np = 2;
        while (np < fill) np <<= 1;
        for (int i = keep + tid; i < np; i += 256) ib[i] = i < fill ? src[s0 + c0 + (i - keep)] : INT32_MAX;
        __syncthreads();
        block_sort_int(ib, np);
        c0 += take;
        keep = fill < max_in ? fill : max_in;
    }
    const int W = deg + max_in;
    int np = 2;
    while (np < W) np <<= 1;
    for (int i = tid; i < np; i += 256) {
        int v;
        if (i < deg) v = G[u * deg + i];
        else if (i < W) v = (i - deg) < keep ? ib[i - deg] : -1;
        else v = INT32_MAX;
        if (i < W && (v == (int)u || v < 0 || v >= n)) v = kBig;
        row[i] = v;
    }
    __syncthreads();
    block_sort_int(row, np);
    // later copies of an id go (judged on the sorted values)
    int mark[2] = {0, 0};
    for (int t = 0, i = tid; i < W; i += 256, ++t)
        mark[t] = (i > 0 && row[i] == row[i - 1]) ? 1 : 0;
    __syncthreads();
    for (int t = 0, i = tid; i < W; i += 256, ++t)
        if (mark[t]) row[i] = kBig;
    for (int t = tid; t < dim && t < 4096; t += 256) xu[t] = ld(X + u * dim + t);
    __syncthreads();
    // exact distances, 16 lanes per candidate; with 16-byte aligned rows a
    // lane reads 16-byte chunks (8 halves or 4 floats) c = tl, tl + 16, ...
    constexpr int VEC = 16 / (int)sizeof(XT);
    const bool vec = dim <= 4096 && dim % VEC == 0 &&
                     (reinterpret_cast<uintptr_t>(X) & 15) == 0;
    const int team = tid >> 4, tl = tid & 15;
    for (int i = team; i < W; i += 16) {
        const int v = row[i];
        float s = 0.f;
        if (v < kBig && vec) {
            const uint4* xv = reinterpret_cast<const uint4*>(X + (int64_t)v * dim);
            for (int c = tl; c * VEC < dim; c += 16) {
                const uint4 raw = xv[c];
                const XT* e = reinterpret_cast<const XT*>(&raw);
#pragma unroll
                for (int k = 0; k < VEC; ++k) {
                    const float xt = xu[c * VEC + k], xvt = (float)e[k];
                    if (metric == SWANN_METRIC_IP) s = __builtin_fmaf(xvt, xt, s);
                    else { const float df = xvt - xt; s = __builtin_fmaf(df, df, s); }
                }
            }
        } else if (v < kBig) {
            const XT* xv = X + (int64_t)v * dim;
            for (int t = tl; t < dim; t += 16) {
                const float xt = dim <= 4096 ? xu[t] : ld(X + u * dim + t);
                const float xvt = ld(xv + t);
                if (metric == SWANN_METRIC_IP) s = __builtin_fmaf(xvt, xt, s);
                else { const float df = xvt - xt; s = __builtin_fmaf(df, df, s); }
            }
        }
#pragma unroll
        for (int off = 8; off > 0; off >>= 1) s += __shfl_down(s, off, 16);
        if (tl == 0) {
            if (v < kBig) { rd[i] = metric == SWANN_METRIC_IP ? 1.0f - s : s; }
            else { rd[i] = INFINITY; row[i] = 0; }     // build.py: invalid -> id 0, +inf
        }
    }
    for (int i = W + tid; i < np; i += 256) { rd[i] = INFINITY; row[i] = INT32_MAX; }
    __syncthreads();
    for (int size = 2; size <= np; size <<= 1)
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int i = tid; i < np; i += 256) {
                const int j = i ^ stride;
                if (j > i) {
                    const bool up = ((i & size) == 0);
                    if (up != lt(rd[i], row[i], rd[j], row[j])) {
                        const float td = rd[i]; rd[i] = rd[j]; rd[j] = td;
                        const int ti = row[i]; row[i] = row[j]; row[j] = ti;
                    }
                }
            }
            __syncthreads();
        }
    for (int t = tid; t < keepn; t += 256) {
        cand2[u * keepn + t] = row[t];
        cd2[u * keepn + t] = rd[t];
    }
}

// ---------------------------------------------------------------------------
// Row order for the exact re-rank.  Re-ranking row u reads the fp32 rows of its
// Cs screened candidates (Cs x 4 KB at d = 1024), so rows whose candidates
// overlap should run together: then most of those reads come from L2 and the
// memory-side cache instead of HBM.  Each row takes the smallest id reachable
// through its kOrderK nearest screened candidates (min-label propagation, with
// a pointer jump per round), and a counting sort by label groups the rows; on
// a clustered corpus a group is a cluster.  Only the order of the workgroups
// changes: each row's re-rank is the same computation in any order.
constexpr int kOrderK = 8, kOrderRounds = 8;

__global__ void order_init(const int32_t* __restrict__ scand, int Cs, int64_t n,
                           int32_t* __restrict__ lab) {
    const int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (u >= n) return;
    int32_t m = (int32_t)u;
    for (int j = 0; j < kOrderK && j < Cs; ++j) {
        const int32_t c = scand[u * Cs + j];
        if (c >= 0 && c < n && c < m) m = c;
    }
    lab[u] = m;
}

// One round, from lin to lout (labels are row ids, so lin[m] is in range).
__global__ void order_round(const int32_t* __restrict__ scand, int Cs, int64_t n,
                            const int32_t* __restrict__ lin, int32_t* __restrict__ lout) {
    const int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (u >= n) return;
    int32_t m = lin[u];
    const int32_t jump = lin[m];
    m = jump < m ? jump : m;
    for (int j = 0; j < kOrderK && j < Cs; ++j) {
        const int32_t c = scand[u * Cs + j];
        if (c >= 0 && c < n) {
            const int32_t l = lin[c];
            m = l < m ? l : m;
        }
    }
    lout[u] = m;
}

// A wave's rows take their labels' slots one distinct label at a time: one
// atomic per label and wave, so a corpus whose rows share a label (an
// unclustered one ends with one label) does not serialize on one counter.
// Returns this lane's slot: the counter's value before its wave's add, plus
// its rank among the wave's lanes of that label.
__device__ __forceinline__ int wave_label_add(int32_t* ctr, int label, bool on) {
    const int lane = threadIdx.x & 63;
    const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
    uint64_t left = __ballot(on);
    int mine = 0;
    while (left) {
        const int first = __builtin_ctzll(left);
        const int l0 = __shfl(label, first, 64);
        const uint64_t same = __ballot(on && label == l0) & left;
        int base = 0;
        if (lane == first) base = atomicAdd(&ctr[l0], __popcll(same));
        base = __shfl(base, first, 64);
        if ((same >> lane) & 1ull) mine = base + __popcll(same & below);
        left &= ~same;
    }
    return mine;
}

__global__ __launch_bounds__(256) void order_count(const int32_t* __restrict__ lab, int64_t n,
                                                   int32_t* __restrict__ cnt) {
    const int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const bool on = u < n;
    wave_label_add(cnt, on ? lab[u] : 0, on);
}

// start[l] is the first slot of label l (an exclusive scan of the counts); each
// row takes the next one, so order is a permutation of [0, n).
__global__ __launch_bounds__(256) void order_place(const int32_t* __restrict__ lab, int64_t n,
                                                   int32_t* __restrict__ start,
                                                   int32_t* __restrict__ order) {
    const int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const bool on = u < n;
    const int slot = wave_label_add(start, on ? lab[u] : 0, on);
    if (on) order[slot] = (int32_t)u;
}

// Exclusive scan of n counts across the GPU: each 1,024-block scans its own
// (scan_blocks, totals to tmp[b]), one workgroup scans the nb totals
// (scan_kernel, into tmp + nb), each block adds its offset (scan_add).
// tmp holds 2 nb words.
__global__ __launch_bounds__(1024) void scan_blocks(const int32_t* __restrict__ in, int64_t n,
                                                    int32_t* __restrict__ out,
                                                    int32_t* __restrict__ total) {
    __shared__ int buf[1024];
    const int64_t i = (int64_t)blockIdx.x * 1024 + threadIdx.x;
    const int v = i < n ? in[i] : 0;
    buf[threadIdx.x] = v;
    __syncthreads();
    for (int off = 1; off < 1024; off <<= 1) {
        const int t = threadIdx.x >= off ? buf[threadIdx.x - off] : 0;
        __syncthreads();
        buf[threadIdx.x] += t;
        __syncthreads();
    }
    if (i < n) out[i] = buf[threadIdx.x] - v;
    if (threadIdx.x == 1023) total[blockIdx.x] = buf[1023];
}

__global__ __launch_bounds__(1024) void scan_add(int32_t* __restrict__ out, int64_t n,
                                                 const int32_t* __restrict__ offset) {
    const int64_t i = (int64_t)blockIdx.x * 1024 + threadIdx.x;
    if (i < n) out[i] += offset[blockIdx.x];
}

void scan_exclusive(const int32_t* in, int64_t n, int32_t* out, int32_t* tmp, hipStream_t st) {
    const int64_t nb = (n + 1023) / 1024;
    hipLaunchKernelGGL(scan_blocks, dim3((unsigned)nb), dim3(1024), 0, st, in, n, out, tmp);
    hipLaunchKernelGGL(scan_kernel, dim3(1), dim3(1024), 0, st, tmp, nb, tmp + nb);
    hipLaunchKernelGGL(scan_add, dim3((unsigned)nb), dim3(1024), 0, st, out, n, tmp + nb);
}

// The order over `scratch` (4 n words: two label arrays, counts, the order),
// from the first kOrderK of each row's C candidates; returns the order.
int32_t* neighbourhood_order(const int32_t* cand, int C, int64_t n, int32_t* scratch,
                             hipStream_t st) {
    int32_t* lab = scratch;
    int32_t* lab2 = scratch + n;
    int32_t* cntl = scratch + 2 * n;
    int32_t* order = scratch + 3 * n;
    const unsigned nb = (unsigned)((n + 255) / 256);
    hipLaunchKernelGGL(order_init, dim3(nb), dim3(256), 0, st, cand, C, n, lab);
    for (int round = 0; round < kOrderRounds; ++round) {
        hipLaunchKernelGGL(order_round, dim3(nb), dim3(256), 0, st, cand, C, n, lab, lab2);
        int32_t* t = lab; lab = lab2; lab2 = t;
    }
    hipLaunchKernelGGL(fill_i32, dim3(nb), dim3(256), 0, st, cntl, n, 0);
    hipLaunchKernelGGL(order_count, dim3(nb), dim3(256), 0, st, lab, n, cntl);
    // the scan's 2 * ceil(n / 1024) words of block totals sit in `order`,
    // which order_place fills only afterwards
    scan_exclusive(cntl, n, lab2, order, st);
    hipLaunchKernelGGL(order_place, dim3(nb), dim3(256), 0, st, lab, n, lab2, order);
    return order;
}

// Exact re-rank of screened candidates (fp32 corpus): per row, the reference
// formula on fp32 dot products with each of its Cs screened candidates, sorted
// by (d, id), the first C kept.  One workgroup per row, 16 lanes per candidate;
// with an order, the workgroups take its entries in XCD-contiguous runs.
template <int METRIC>
__global__ __launch_bounds__(256) void rerank_kernel(const float* __restrict__ X, int64_t n, int dim,
                                                     const float* __restrict__ xn,
                                                     const int32_t* __restrict__ scand, int Cs,
                                                     int C, const int32_t* __restrict__ order,
                                                     int32_t* __restrict__ cand,
                                                     float* __restrict__ cdist) {
    extern __shared__ __align__(16) unsigned char smem[];
    float* xu = reinterpret_cast<float*>(smem);
    __shared__ float sd[512];
    __shared__ int si[512];
    // consecutive entries of the order run on one XCD (one L2), a group's
    // rows together
    const int64_t u = order ? (int64_t)order[xcd_remap(blockIdx.x, gridDim.x)]
                            : (int64_t)blockIdx.x;
    const int tid = threadIdx.x, team = tid >> 4, tl = tid & 15;
    for (int t = tid; t < dim; t += 256) xu[t] = X[u * dim + t];
    int np = 2;
    while (np < Cs) np <<= 1;
    for (int i = Cs + tid; i < np; i += 256) { sd[i] = INFINITY; si[i] = INT32_MAX; }
    __syncthreads();
    const float nu = METRIC == SWANN_METRIC_L2 ? xn[u] : 0.f;
    const bool v4 = (dim & 3) == 0;
    for (int i = team; i < Cs; i += 16) {
        const int c = scand[u * Cs + i];
        float s = 0.f;
        if (c >= 0 && c < n) {
            const float* xc = X + (int64_t)c * dim;
            if (v4) {
                // unrolled so that four loads are in flight ahead of their
                // FMAs; the FMAs keep their order, so s is the same to the bit
#pragma unroll 4
                for (int t = tl * 4; t < dim; t += 64) {
                    const float4 a = *reinterpret_cast<const float4*>(xc + t);
                    const float4 b = *reinterpret_cast<const float4*>(xu + t);
                    s = __builtin_fmaf(a.x, b.x, s); s = __builtin_fmaf(a.y, b.y, s);
                    s = __builtin_fmaf(a.z, b.z, s); s = __builtin_fmaf(a.w, b.w, s);
                }
            } else {
                for (int t = tl; t < dim; t += 16) s = __builtin_fmaf(xc[t], xu[t], s);
            }
        }
#pragma unroll
        for (int off = 8; off > 0; off >>= 1) s += __shfl_down(s, off, 16);
        if (tl == 0) {
            if (c < 0 || c >= n) { sd[i] = INFINITY; si[i] = INT32_MAX; }
            else if (c == u) { sd[i] = kSelf; si[i] = c; }
            else { sd[i] = pair_formula(s, nu, METRIC == SWANN_METRIC_L2 ? xn[c] : 0.f, METRIC); si[i] = c; }
        }
    }
    __syncthreads();
    for (int size = 2; size <= np; size <<= 1)
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int i = tid; i < np; i += 256) {
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
    for (int t = tid; t < C; t += 256) {
        const bool ok = si[t] != INT32_MAX;
        cand[u * C + t] = ok ? si[t] : -1;
        cdist[u * C + t] = ok ? sd[t] : INFINITY;
    }
}

inline int64_t align256(int64_t b) { return ((b + 255) / 256) * 256; }

int sweep_cap(int C) {
    int cap = C + 512;
    return cap > 1024 ? 1024 : cap;
}

bool use_mfma(int dim) { return dim % 8 == 0; }

// An fp32 corpus on the MFMA path is swept on an fp16 screen and its lists
// re-ranked in exact fp32; fp16 corpora and the fp32 SIMT sweep are exact.
bool screened(int x_dtype, int dim) { return x_dtype == SWANN_DTYPE_F32 && use_mfma(dim); }

// Candidates the fp32 screen keeps per row before the exact re-rank (at
// least C: when C + 32 exceeds n or the sweep's list limit the screen keeps
// what it can, and the re-rank still replaces every distance by the exact one).
int screen_count(int C, int64_t n, int x_dtype, int dim) {
    if (!screened(x_dtype, dim)) return C;
    int64_t cs = C + 32;
    if (cs > kMaxC) cs = kMaxC;
    if (cs > n) cs = n;
    return (int)(cs < C ? C : cs);
}

}  // namespace
}  // namespace swann

using namespace swann;

#define SWANN_BY_DTYPE(DT, CALL_F32, CALL_F16) \
    do { if ((DT) == SWANN_DTYPE_F16) { CALL_F16; } else { CALL_F32; } } while (0)

extern "C" {

int64_t swann_sweep_workspace_size(int64_t n, int dim, int x_dtype, int C) {
    const int Cs = screen_count(C, n, x_dtype, dim);
    const int cap = use_mfma(dim) ? sweep_mfma_cap(Cs) : sweep_cap(C);
    const int64_t G = use_mfma(dim) ? sweep_mfma_splits(n, dim) : 1;
    int64_t b = align256(n * 4) + align256(n * G * cap * 4) * 2 + align256(n * G * 4);
    if (screened(x_dtype, dim)) b += align256(n * (int64_t)Cs * 4) * 2;
    if (use_mfma(dim)) b += sweep_mfma_extra_bytes(n, dim, x_dtype);
    return b;
}

int swann_build_sweep(const void* X, int x_dtype, int64_t n, int dim, int metric, int C,
                      int32_t* cand, float* cdist, void* workspace, void* stream) {
    clear_error();
    SWANN_REQUIRE(metric == SWANN_METRIC_IP || metric == SWANN_METRIC_L2,
                  "metric must be 0 (ip) or 1 (l2)");
    SWANN_REQUIRE(x_dtype == SWANN_DTYPE_F32 || x_dtype == SWANN_DTYPE_F16,
                  "X: float32 or float16");
    SWANN_REQUIRE(n >= 2 && dim >= 1, "sweep: need n >= 2 rows");
    SWANN_REQUIRE(C >= 1 && C <= kMaxC && C <= n, "sweep: candidates must be in 1..min(n, %d)",
                  kMaxC);
    SWANN_REQUIRE(n <= INT32_MAX / 2, "sweep: n too large");
    SWANN_REQUIRE(X && cand && cdist && workspace, "sweep: a required pointer is NULL");
    hipStream_t st = (hipStream_t)stream;
    const bool mf = use_mfma(dim);
    const int Cs = screen_count(C, n, x_dtype, dim);
    const bool rerank = screened(x_dtype, dim);
    SWANN_REQUIRE(!rerank || dim * 4 <= 64 * 1024, "sweep: dimension too large for the re-rank");
    const int cap = mf ? sweep_mfma_cap(Cs) : sweep_cap(C);
    const int G = mf ? sweep_mfma_splits(n, dim) : 1;
    char* ws = (char*)workspace;
    float* xn = (float*)ws; ws += align256(n * 4);
    float* bkey = (float*)ws; ws += align256(n * (int64_t)G * cap * 4);
    int32_t* bid = (int32_t*)ws; ws += align256(n * (int64_t)G * cap * 4);
    int32_t* bcnt = (int32_t*)ws; ws += align256(n * (int64_t)G * 4);
    int32_t* scand = nullptr;
    float* scd = nullptr;
    if (rerank) {
        scand = (int32_t*)ws; ws += align256(n * (int64_t)Cs * 4);
        scd = (float*)ws; ws += align256(n * (int64_t)Cs * 4);
    }
    char* extra = ws;
    int rc;
    int Gu = 1;                      // lists per row the sweep filled
    const int32_t* perm = nullptr;   // the sweep's row order, when not the rows' own
    if (mf) {
        rc = sweep_mfma_run(X, x_dtype, n, dim, metric, Cs, cap, G, bkey, bid, bcnt, extra, st,
                            &Gu, &perm);
    } else {
        const unsigned nb = (unsigned)((n + 3) / 4);
        if (metric == SWANN_METRIC_L2)
            SWANN_BY_DTYPE(x_dtype,
                hipLaunchKernelGGL(norms_kernel<float>, dim3(nb), dim3(256), 0, st, (const float*)X, n, dim, xn),
                hipLaunchKernelGGL(norms_kernel<_Float16>, dim3(nb), dim3(256), 0, st, (const _Float16*)X, n, dim, xn));
        SweepArgs a{X, xn, n, dim, metric, C, cap, bkey, bid, bcnt};
        const unsigned grid = (unsigned)((n + kRT - 1) / kRT);
        SWANN_BY_DTYPE(x_dtype,
            hipLaunchKernelGGL(sweep_kernel<float>, dim3(grid), dim3(256), 0, st, a),
            hipLaunchKernelGGL(sweep_kernel<_Float16>, dim3(grid), dim3(256), 0, st, a));
        rc = launch_status("sweep");
    }
    if (rc) return rc;
    // one list holds up to cap; G > 1 lists were each cut to Cs by the sweep
    const int most = Gu > 1 ? Gu * Cs : cap;
    int np = 2;
    while (np < most) np <<= 1;
    if (!rerank) {
        hipLaunchKernelGGL(sweep_final, dim3((unsigned)n), dim3(256), (size_t)np * 8, st, bkey, bid,
                           bcnt, n, cap, Gu, C, mf ? 1 : 0, perm, cand, cdist);
        return launch_status("sweep final");
    }
    hipLaunchKernelGGL(sweep_final, dim3((unsigned)n), dim3(256), (size_t)np * 8, st, bkey, bid,
                       bcnt, n, cap, Gu, Cs, mf ? 1 : 0, perm, scand, scd);
    rc = launch_status("sweep final");
    if (rc) return rc;
    // the re-rank's row order, in the sweep's lists (free once sweep_final has
    // read them: n * G * cap >= 4 n words)
    const int32_t* order = neighbourhood_order(scand, Cs, n, (int32_t*)bkey, st);
    rc = launch_status("sweep re-rank order");
    if (rc) return rc;
    // exact fp32 re-rank of the screened lists; the norms are the sweep's
    const float* xnorm = (const float*)extra;
    if (metric == SWANN_METRIC_IP)
        hipLaunchKernelGGL(rerank_kernel<SWANN_METRIC_IP>, dim3((unsigned)n), dim3(256),
                           (size_t)dim * 4, st, (const float*)X, n, dim, xnorm, scand, Cs, C,
                           order, cand, cdist);
    else
        hipLaunchKernelGGL(rerank_kernel<SWANN_METRIC_L2>, dim3((unsigned)n), dim3(256),
                           (size_t)dim * 4, st, (const float*)X, n, dim, xnorm, scand, Cs, C,
                           order, cand, cdist);
    return launch_status("sweep re-rank");
}

int64_t swann_prune_workspace_size(int64_t n, int dim, int x_dtype) {
    // the node order (4 n words), then the fp32 rows' plane scales
    return align256(n * 16) + (x_dtype == SWANN_DTYPE_F32 && dim % 8 == 0 ? align256(n * 4) : 0);
}

}  // extern "C"

namespace swann {
namespace {
// The prune's launches: `order` (or NULL) the node order, `rscale` (or NULL)
// n words for an fp32 corpus's plane scales.
int prune_run(const void* X, int x_dtype, int64_t n, int dim, int metric, const int32_t* cand,
              const float* cdist, int C, int deg, float alpha, const int32_t* deg_per_node,
              const uint8_t* protect, int32_t* out, const int32_t* order, float* rscale,
              hipStream_t st) {
    // the Gram on MFMA: fp16 rows with 16-byte aligned 16-wide K steps, fp32
    // rows with 16-byte aligned 8-wide K steps
    const bool simt = option_on(kOptPruneSimt);
    const bool mfma16 = x_dtype == SWANN_DTYPE_F16 && dim % 16 == 0 && (uintptr_t)X % 16 == 0;
    const bool mfma32 = x_dtype == SWANN_DTYPE_F32 && dim % 8 == 0 && (uintptr_t)X % 16 == 0;
    // fp32 rows with a workspace for their scales: the Gram on split fp16
    // planes (option prune_f32 keeps the fp32 MFMA Gram)
    const bool planes = mfma32 && rscale && !option_on(kOptPruneF32);
    if (!simt && mfma16)
        hipLaunchKernelGGL((prune_kernel<_Float16, true>), dim3((unsigned)n), dim3(256), 0, st,
                           (const _Float16*)X, n, dim, metric, cand, cdist, C, deg, alpha,
                           deg_per_node, protect, out, nullptr, order);
    else if (!simt && planes) {
        hipLaunchKernelGGL(row_scale, dim3((unsigned)((n + 3) / 4)), dim3(256), 0, st,
                           (const float*)X, n, dim, rscale);
        hipLaunchKernelGGL((prune_kernel<float, true, true>), dim3((unsigned)n), dim3(256), 0,
                           st, (const float*)X, n, dim, metric, cand, cdist, C, deg, alpha,
                           deg_per_node, protect, out, rscale, order);
    } else if (!simt && mfma32)
        hipLaunchKernelGGL((prune_kernel<float, true>), dim3((unsigned)n), dim3(256), 0, st,
                           (const float*)X, n, dim, metric, cand, cdist, C, deg, alpha,
                           deg_per_node, protect, out, nullptr, order);
    else
        SWANN_BY_DTYPE(x_dtype,
            hipLaunchKernelGGL((prune_kernel<float, false>), dim3((unsigned)n), dim3(256), 0, st,
                               (const float*)X, n, dim, metric, cand, cdist, C, deg, alpha,
                               deg_per_node, protect, out, nullptr, order),
            hipLaunchKernelGGL((prune_kernel<_Float16, false>), dim3((unsigned)n), dim3(256), 0,
                               st, (const _Float16*)X, n, dim, metric, cand, cdist, C, deg, alpha,
                               deg_per_node, protect, out, nullptr, order));
    return launch_status("prune");
}
}  // namespace
}  // namespace swann

extern "C" {

int swann_build_prune(const void* X, int x_dtype, int64_t n, int dim, int metric,
                      const int32_t* cand, const float* cdist, int C, int deg, float alpha,
                      const int32_t* deg_per_node, const uint8_t* protect, int32_t* out,
                      void* workspace, void* stream) {
    clear_error();
    SWANN_REQUIRE(metric == SWANN_METRIC_IP || metric == SWANN_METRIC_L2,
                  "metric must be 0 (ip) or 1 (l2)");
    SWANN_REQUIRE(x_dtype == SWANN_DTYPE_F32 || x_dtype == SWANN_DTYPE_F16,
                  "X: float32 or float16");
    SWANN_REQUIRE(C >= 1 && C <= kPruneMaxC, "prune: candidates per node must be in 1..%d",
                  kPruneMaxC);
    SWANN_REQUIRE(deg >= 1 && deg <= kPruneMaxC, "prune: degree must be in 1..%d", kPruneMaxC);
    SWANN_REQUIRE(n >= 1 && n <= INT32_MAX, "prune: n out of range");
    SWANN_REQUIRE(X && cand && cdist && out, "prune: a required pointer is NULL");
    hipStream_t st = (hipStream_t)stream;
    // with a workspace, nodes run grouped by shared candidates (each node's
    // prune is the same computation in any order): their candidate rows then
    // come from L2 and the memory-side cache on a clustered corpus
    const int32_t* order = nullptr;
    if (workspace) {
        order = neighbourhood_order(cand, C, n, (int32_t*)workspace, st);
        const int rc = launch_status("prune order");
        if (rc) return rc;
    }
    float* rscale = workspace ? (float*)((char*)workspace + align256(n * 16)) : nullptr;
    return prune_run(X, x_dtype, n, dim, metric, cand, cdist, C, deg, alpha, deg_per_node,
                     protect, out, order, rscale, st);
}

int64_t swann_reverse_workspace_size(int64_t n, int deg, int max_in) {
    const int keepn = (deg + max_in) < kPruneMaxC ? (deg + max_in) : kPruneMaxC;
    // then the re-prune's workspace (swann_prune_workspace_size for fp32)
    return align256(n * 4) * 3 + align256(n * (int64_t)deg * 4) +
           align256(n * (int64_t)keepn * 4) * 2 + align256(n * 16) + align256(n * 4);
}

int swann_build_reverse(const void* X, int x_dtype, int64_t n, int dim, int metric,
                        const int32_t* G, int deg, float alpha, int max_in,
                        const int32_t* deg_per_node, int32_t* out, void* workspace,
                        void* stream) {
    clear_error();
    SWANN_REQUIRE(metric == SWANN_METRIC_IP || metric == SWANN_METRIC_L2,
                  "metric must be 0 (ip) or 1 (l2)");
    SWANN_REQUIRE(x_dtype == SWANN_DTYPE_F32 || x_dtype == SWANN_DTYPE_F16,
                  "X: float32 or float16");
    SWANN_REQUIRE(deg >= 1 && max_in >= 0 && deg + max_in <= 512,
                  "reverse: need deg >= 1, max_in >= 0, deg + max_in <= 512");
    SWANN_REQUIRE(deg <= kPruneMaxC, "reverse: degree must be in 1..%d (the re-prune's)",
                  kPruneMaxC);
    SWANN_REQUIRE(n >= 1 && n * (int64_t)deg < INT32_MAX, "reverse: n * deg must fit in int32");
    SWANN_REQUIRE(X && G && out && workspace, "reverse: a required pointer is NULL");
    hipStream_t st = (hipStream_t)stream;
    const int keepn = (deg + max_in) < kPruneMaxC ? (deg + max_in) : kPruneMaxC;
    char* ws = (char*)workspace;
    int32_t* cnt = (int32_t*)ws; ws += align256(n * 4);
    int32_t* fill = (int32_t*)ws; ws += align256(n * 4);
    int32_t* start = (int32_t*)ws; ws += align256(n * 4);
    int32_t* src = (int32_t*)ws; ws += align256(n * (int64_t)deg * 4);
    int32_t* cand2 = (int32_t*)ws; ws += align256(n * (int64_t)keepn * 4);
    float* cd2 = (float*)ws; ws += align256(n * (int64_t)keepn * 4);
    void* prune_ws = ws;
    // counters are cleared by a kernel, not a memset, so the pass can be captured
    const unsigned nbk = (unsigned)((n + 255) / 256);
    hipLaunchKernelGGL(fill_i32, dim3(nbk), dim3(256), 0, st, cnt, n, 0);
    hipLaunchKernelGGL(fill_i32, dim3(nbk), dim3(256), 0, st, fill, n, 0);
    const int64_t E = n * deg;
    const unsigned eb = (unsigned)((E + 255) / 256);
    hipLaunchKernelGGL(rev_count, dim3(eb), dim3(256), 0, st, G, n, deg, cnt);
    hipLaunchKernelGGL(scan_kernel, dim3(1), dim3(1024), 0, st, cnt, n, start);
    hipLaunchKernelGGL(rev_scatter, dim3(eb), dim3(256), 0, st, G, n, deg, start, fill, src);
    int rc = launch_status("reverse scatter");
    if (rc) return rc;
    // one node order, from the graph's rows, for both the assembly and the
    // re-prune: both gather the rows of a node's neighbours
    const int32_t* order = neighbourhood_order(G, deg, n, (int32_t*)prune_ws, st);
    float* rscale = (float*)((char*)prune_ws + align256(n * 16));
    SWANN_BY_DTYPE(x_dtype,
        hipLaunchKernelGGL(rev_assemble<float>, dim3((unsigned)n), dim3(256), 0, st,
                           (const float*)X, n, dim, metric, G, deg, max_in, cnt, start, src,
                           keepn, cand2, cd2, order),
        hipLaunchKernelGGL(rev_assemble<_Float16>, dim3((unsigned)n), dim3(256), 0, st,
                           (const _Float16*)X, n, dim, metric, G, deg, max_in, cnt, start, src,
                           keepn, cand2, cd2, order));
    rc = launch_status("reverse assemble");
    if (rc) return rc;
    return prune_run(X, x_dtype, n, dim, metric, cand2, cd2, keepn, deg, alpha, deg_per_node,
                     nullptr, out, order, rscale, st);
}

}  // extern "C"
