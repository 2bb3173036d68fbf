// Multi-branch graph search on gfx950: branch init, best-first advance,
// per-query merge, and the asynchronous overflow readback.
//
// Semantics follow swann/csrc/local_search.cu (reference) exactly where the
// result depends on them -- the distance's summation order (:185-203), the
// (distance, id) order (:87-89), the slot rule and stop radius (:451-517), the
// candidate filter (:607-625), merge-path with its tie behaviour (:637-650),
// the bound (:655-658), crowd and stall retirement (:659-682), the shared
// table and claims (:169-183, :541-592) -- and are MI355X-native in how they
// run:
//   * one workgroup per (query, branch) over a 1-D grid (no 65535-query cap),
//     XCD-remapped so a query's branches share one L2;
//   * BLOCK = 64 (one wave; every barrier folds away) for batch work, 256
//     for small batches, 1024 for grids too small to give every CU two
//     branches, where the serial chain of expansions is the latency;
//   * the neighbour list of an expansion is screened lane-parallel first
//     (visited insert, table probe, claim), then only the survivors are
//     scored, TEAM lanes per distance, with every 16-byte row load of a lane
//     issued before its arithmetic;
//   * queue, candidates and the query vector stay in LDS; counters stay in
//     registers/LDS until the call ends;
//   * the per-query table, claims and bound use agent-scope atomics, because
//     L2 is per XCD and plain loads are not coherent across XCDs.
#include <float.h>
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdlib.h>

#include "common.h"
#include "lanes.h"

namespace swann {
namespace {

constexpr int kMaxL = SWANN_MAXL;
constexpr int kMaxD = SWANN_MAXD;
constexpr int kMaxV = SWANN_MAXV;
constexpr int kNctr = SWANN_NCTR;
constexpr int kCprobe = 32;            // bounded probe into the shared table
#ifndef SWANN_MAX_CHUNKS
#define SWANN_MAX_CHUNKS 16
#endif
constexpr int kMaxChunks = SWANN_MAX_CHUNKS;   // 16-byte loads a lane keeps in flight
// Scope of the per-query table and bound operations.  A query's branches are
// placed on one XCD (xcd_remap) when they all fit there at once, and spread
// over the XCDs otherwise (remap_branches), so these must be agent scope,
// which is coherent across the XCDs' separate L2s.
#ifndef SWANN_TABLE_SCOPE
#define SWANN_TABLE_SCOPE __HIP_MEMORY_SCOPE_AGENT
#endif
constexpr size_t kMaxLds = 64 * 1024;

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float float4v __attribute__((ext_vector_type(4)));

// The query vector in LDS: every 32 floats are followed by 4 unused ones, so
// element i sits at qpad(i).  Lanes that read the same 16-byte column of
// different 32-float groups (the code estimate: one code word per lane, 128 B
// apart in the plain layout) then fall in different LDS banks instead of all
// in one; a 4- or 8-float vector never crosses a group, so the distance's
// 16-byte reads stay contiguous.
__host__ __device__ constexpr int qpad(int i) { return i + ((i >> 5) << 2); }
__host__ __device__ constexpr int qpad_floats(int dim) { return ((dim + 31) >> 5) * 36; }

template <typename XT> struct Vec;
template <> struct Vec<float> { static constexpr int N = 4; };
template <> struct Vec<_Float16> { static constexpr int N = 8; };

__device__ __forceinline__ bool lt(float da, int ia, float db, int ib) {
    return (da < db) || (da == db && ia < ib);
}

template <int METRIC>
__device__ __forceinline__ float term(float q, float x) {
    if (METRIC == SWANN_METRIC_IP) return q * x;
    const float df = q - x;
    return df * df;
}

// One distance: lane tl of a TEAM owns the VEC-element blocks at tl*VEC,
// tl*VEC + TEAM*VEC, ...; each lane sums its terms in order, then the team
// folds with off = TEAM/2 .. 1 (lane tl takes tl+off).  Built with
// -ffp-contract=off so product and sum round separately.  The result is
// meaningful in lane tl == 0.
template <int TEAM, typename XT, int METRIC>
__device__ __forceinline__ float team_dist(const float* __restrict__ sq,
                                           const XT* __restrict__ x, int dim, int tl,
                                           bool vec_ok) {
    constexpr int VEC = Vec<XT>::N;
    constexpr int STRIDE = TEAM * VEC;
    float acc = 0.f;
    if (vec_ok) {
        for (int b0 = tl * VEC; b0 < dim; b0 += STRIDE * kMaxChunks) {
            // With STRIDE a multiple of 32 the chunks' padded offsets are one
            // base plus constants: qpad(b0 + c*STRIDE) = qpad(b0) + c*STRIDE*36/32
            // because c*STRIDE adds whole 32-float groups.
            const float* qb = sq + qpad(b0);
            auto qat = [&](int c, int base) -> const float* {
                if constexpr (STRIDE % 32 == 0) return qb + c * (STRIDE / 32 * 36);
                else return sq + qpad(base);
            };
            uint4 raw[kMaxChunks];
#pragma unroll
            for (int c = 0; c < kMaxChunks; ++c) {
                const int base = b0 + c * STRIDE;
                if (base < dim) raw[c] = *reinterpret_cast<const uint4*>(x + base);
            }
#pragma unroll
            for (int c = 0; c < kMaxChunks; ++c) {
                const int base = b0 + c * STRIDE;
                if (base < dim) {
                    if constexpr (VEC == 4) {
                        const float4v xv = __builtin_bit_cast(float4v, raw[c]);
                        const float4v qv = *reinterpret_cast<const float4v*>(qat(c, base));
#pragma unroll
                        for (int i = 0; i < 4; ++i) acc = acc + term<METRIC>(qv[i], xv[i]);
                    } else {
                        const half8 hv = __builtin_bit_cast(half8, raw[c]);
                        const float4v q0 = *reinterpret_cast<const float4v*>(qat(c, base));
                        const float4v q1 = *reinterpret_cast<const float4v*>(qat(c, base) + 4);
#pragma unroll
                        for (int i = 0; i < 4; ++i) acc = acc + term<METRIC>(q0[i], (float)hv[i]);
#pragma unroll
                        for (int i = 0; i < 4; ++i)
                            acc = acc + term<METRIC>(q1[i], (float)hv[4 + i]);
                    }
                }
            }
        }
    } else {
        // Any dimension: element loads, same order, nothing read past the row.
        for (int base = tl * VEC; base < dim; base += STRIDE) {
#pragma unroll
            for (int i = 0; i < VEC; ++i) {
                if (base + i < dim)
                    acc = acc + term<METRIC>(sq[qpad(base + i)], (float)x[base + i]);
            }
        }
    }
    acc = team_fold_add<TEAM>(acc);      // DPP row shifts, no LDS round trip
    return METRIC == SWANN_METRIC_IP ? 1.f - acc : acc;
}

template <int TEAM, typename XT>
__device__ __forceinline__ float team_dist_m(const float* sq, const XT* x, int dim, int tl,
                                             bool vec_ok, int metric) {
    return metric == SWANN_METRIC_IP ? team_dist<TEAM, XT, SWANN_METRIC_IP>(sq, x, dim, tl, vec_ok)
                                     : team_dist<TEAM, XT, SWANN_METRIC_L2>(sq, x, dim, tl, vec_ok);
}

// Sign-code estimate of the IP distance (local_search.cu:205-243): with the
// node's code b in {-1, +1}^dim taken around the corpus mean mu and its scale
// alpha, <q, x> ~ alpha * <q, b> + <q, mu> and <q, b> = 2 * (sum of q over set
// bits) - sum(q).  Lane tl of a TEAM owns code words tl, tl + TEAM, ...; each
// lane adds q over its set bits in ascending dimension, then the team folds
// with off = TEAM/2 .. 1.  Meaningful in tl == 0.
//
// A whole word is added branch-free: q[i] where bit i is set, +0.0 where it is
// not (q[i]'s bits ANDed with the bit spread to a full-word mask), in
// ascending i.  acc + 0.0 == acc for every acc but -0.0 (which becomes
// +0.0), and the sign of a zero partial changes no later sum and no estimate,
// so this equals the set-bits-only loop bit for bit; its 32 LDS reads are
// independent of the code, so they issue together instead of one per set bit.
// The word that straddles dim walks its set bits below dim.
//
// A lane's words come in chunks of kCodeWords (words w0, w0 + TEAM, ...),
// each chunk's loads issued together; the caller fetches the first chunk
// (code_fetch) and passes it in.
constexpr int kCodeWords = 4;

template <int TEAM>
__device__ __forceinline__ void code_fetch(const int32_t* __restrict__ code, int w0, int cwords,
                                           unsigned* wb) {
#pragma unroll
    for (int j = 0; j < kCodeWords; ++j) {
        const int w = w0 + j * TEAM;
        wb[j] = w < cwords ? (unsigned)code[w] : 0u;
    }
}

template <int TEAM>
__device__ __forceinline__ float code_chunk(const float* __restrict__ sq, const unsigned* wb,
                                            int w0, int cwords, int dim, float acc) {
#pragma unroll
    for (int j = 0; j < kCodeWords; ++j) {
        const int w = w0 + j * TEAM;
        if (w >= cwords) break;
        unsigned bits = wb[j];
        const int base = w * 32;
        if (base + 32 <= dim) {
            const float4v* s4 = reinterpret_cast<const float4v*>(sq + qpad(base));
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                const float4v v = s4[c];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    // bit 4c+i spread over the word (one signed bitfield
                    // extract), then q & mask: q or +0.0 without a compare
                    const int m = (int)(bits << (31 - (4 * c + i))) >> 31;
                    acc = acc + __int_as_float(__float_as_int(v[i]) & m);
                }
            }
            continue;
        }
        while (bits) {
            const int i = base + __builtin_ctz(bits);
            if (i >= dim) break;
            acc = acc + sq[qpad(i)];
            bits &= bits - 1u;
        }
    }
    return acc;
}

// `head` holds the lane's first chunk (code_fetch(code, tl, ...)).
template <int TEAM>
__device__ __forceinline__ float team_code_ip(const float* __restrict__ sq,
                                              const int32_t* __restrict__ code,
                                              const unsigned* head, float alpha, float qmu,
                                              float qsum, int dim, int cwords, int tl) {
    float acc = code_chunk<TEAM>(sq, head, tl, cwords, dim, 0.f);
    for (int w0 = tl + kCodeWords * TEAM; w0 < cwords; w0 += kCodeWords * TEAM) {
        unsigned wb[kCodeWords];
        code_fetch<TEAM>(code, w0, cwords, wb);
        acc = code_chunk<TEAM>(sq, wb, w0, cwords, dim, acc);
    }
    acc = team_fold_add<TEAM>(acc);
    return 1.f - (alpha * (2.f * acc - qsum) + qmu);
}

// A cheap, bounded stand-in for the estimate's sum, so that the exact
// summation above runs only where the decision is close.  The query is
// quantised once per call to integers k_i = rint(q_i / s), |k_i| <= 2047,
// s = max |q| / 2047, stored as twelve bit planes of u_i = k_i + 2048 (plane
// b of code word w: bit j set when bit b of u_{32w + j} is), so that over a
// code word's set bits sum k_i = sum_b 2^b popcount(bits & plane_b) - 2048
// popcount(bits): two VALU a plane and word (and, count) where the exact sum
// takes three a bit.  Integer sums are exact, so S' = s * K differs from the
// exact real sum S over the set bits by at most E = sum_i |q_i - s k_i|, and
// S from the reference-order fp32 sum by at most (dim + 64) u sum |q_i|
// (u = 2^-24; no summation path in the lane loop and team fold is longer).
// The estimate 1 - (alpha (2 S - sum q) + <q, mu>) is monotone in S in fp32
// too (every operation rounds monotonically), so evaluating it at
// S' + delta and S' - delta brackets the value the reference computes:
// when both ends fall on one side of the line the decision is the
// reference's, bit for bit; otherwise the exact sum decides.
constexpr int kPlanes = 12;
constexpr int kPlaneOff = 1 << (kPlanes - 1);

// Sum of k_i over the set bits of a lane's words (w = tl, tl + TEAM, ...)
// folded over the team: exact integer arithmetic, the total in lane 0.
// `head` holds the lane's first chunk (code_fetch(code, tl, nw32, ...)).
template <int TEAM>
__device__ __forceinline__ int team_code_k(const uint32_t* __restrict__ cpl,
                                           const int32_t* __restrict__ code,
                                           const unsigned* head, int nw32, int dim, int tl) {
    uint32_t cnt[kPlanes];
#pragma unroll
    for (int b = 0; b < kPlanes; ++b) cnt[b] = 0u;
    uint32_t nb = 0u;
    for (int w0 = tl; w0 < nw32; w0 += kCodeWords * TEAM) {
        unsigned wb[kCodeWords];
        if (w0 == tl) {
#pragma unroll
            for (int j = 0; j < kCodeWords; ++j) wb[j] = head[j];
        } else {
            code_fetch<TEAM>(code, w0, nw32, wb);
        }
#pragma unroll
        for (int j = 0; j < kCodeWords; ++j) {
            const int w = w0 + j * TEAM;
            if (w >= nw32) break;
            uint32_t bits = wb[j];
            const int base = w * 32;
            if (base + 32 > dim) bits &= (1u << (dim - base)) - 1u;
            const uint4* p4 = reinterpret_cast<const uint4*>(cpl + w * kPlanes);
#pragma unroll
            for (int c = 0; c < kPlanes / 4; ++c) {
                const uint4 p = p4[c];
                cnt[4 * c + 0] += __builtin_popcount(bits & p.x);
                cnt[4 * c + 1] += __builtin_popcount(bits & p.y);
                cnt[4 * c + 2] += __builtin_popcount(bits & p.z);
                cnt[4 * c + 3] += __builtin_popcount(bits & p.w);
            }
            nb += __builtin_popcount(bits);
        }
    }
    int k = -kPlaneOff * (int)nb;
#pragma unroll
    for (int b = 0; b < kPlanes; ++b) k += (int)(cnt[b] << b);
    return team_fold_add_i32<TEAM>(k);
}

// Per-branch visited set: open addressing, linear probe, slot = key + 1
// (local_search.cu:94-110).  Private to the workgroup.
__device__ __forceinline__ int vis_insert(int* tab, int H, int key, int* fail) {
    const unsigned mask = (unsigned)(H - 1);
    unsigned pos = (2654435761u * (unsigned)key) & mask;
    for (int probe = 0; probe < H; ++probe) {
        int cur = __hip_atomic_load(&tab[pos], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        if (cur == 0) {
            int expected = 0;
            if (__hip_atomic_compare_exchange_strong(&tab[pos], &expected, key + 1,
                                                     __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_WORKGROUP))
                return 1;
            cur = expected;
        }
        if (cur == key + 1) return 0;
        pos = (pos + 1) & mask;
    }
    *fail += 1;
    return 0;
}

// Per-query shared table and claims (local_search.cu:169-183).  Agent scope:
// the branches of one query may run on different XCDs.  `ts` is the table's
// stride in words: 1 for separate id and distance arrays, 2 when they are
// interleaved (id, d) pairs, so that a claim and the distance stored into it
// later share one cache line (half the table's DRAM activations).
__device__ __forceinline__ int cache_slot(int* cid, int Hc, int ts, int key, int* claimed) {
    const unsigned mask = (unsigned)(Hc - 1);
    unsigned pos = (2654435761u * (unsigned)key) & mask;
    for (int probe = 0; probe < kCprobe; ++probe) {
        int cur = __hip_atomic_load(&cid[pos * ts], __ATOMIC_RELAXED, SWANN_TABLE_SCOPE);
        if (cur == key + 1) return (int)pos;
        if (cur == 0) {
            int expected = 0;
            if (__hip_atomic_compare_exchange_strong(&cid[pos * ts], &expected, key + 1,
                                                     __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                                     SWANN_TABLE_SCOPE)) {
                *claimed = 1;
                return (int)pos;
            }
            if (expected == key + 1) return (int)pos;
        }
        pos = (pos + 1) & mask;
    }
    return -1;
}

// The same probe over interleaved pairs, one 64-bit word per slot: low half
// the id (key + 1, 0 = empty), high half the distance (FLT_MAX until the
// claimer stores it).  An empty slot is exactly (0, FLT_MAX) -- init writes
// that and only a claim changes the id -- so one 64-bit compare-and-swap
// against it either claims the slot or returns what the slot holds: a found
// key comes back with its distance in the same round trip.  Reading the id
// and the distance in one access is one of the orders the word-by-word probe
// allows (id, then distance).
__device__ __forceinline__ int cache_slot_pair(unsigned long long* tab, int Hc, int key,
                                               int* claimed, float* d) {
    const unsigned mask = (unsigned)(Hc - 1);
    unsigned pos = (2654435761u * (unsigned)key) & mask;
    const unsigned long long empty = (unsigned long long)__float_as_uint(FLT_MAX) << 32;
    const unsigned long long mine = empty | (unsigned)(key + 1);
    for (int probe = 0; probe < kCprobe; ++probe) {
        unsigned long long cur = empty;
        if (__hip_atomic_compare_exchange_strong(&tab[pos], &cur, mine, __ATOMIC_RELAXED,
                                                 __ATOMIC_RELAXED, SWANN_TABLE_SCOPE)) {
            *claimed = 1;
            *d = FLT_MAX;
            return (int)pos;
        }
        if ((unsigned)cur == (unsigned)(key + 1)) {
            *d = __uint_as_float((unsigned)(cur >> 32));
            return (int)pos;
        }
        pos = (pos + 1) & mask;
    }
    return -1;
}

// Claims without cached distances: one bit per corpus row (Hc >= n bits a
// query).  Under exclusive claims a branch that finds a row in the shared
// table never takes it as a candidate (local_search.cu:541-592): it skips it
// when the distance is stored and, when the claimer has not stored it yet,
// scores it again only to drop it.  The distance is therefore never read, and
// a bit per row decides the same thing: the first to set it owns the row.  A
// query's 128 KiB at a million rows stays in L2 and the MALL while its
// branches run, where a 4 MiB table of (id, d) pairs does not; and there is
// no probe chain to run out.  The sign-code filter keeps the table: a row it
// skips stays claimed but unscored, and another branch may score it later.
__device__ __forceinline__ bool claim_bit(int32_t* bits, int key) {
    const uint32_t bit = 1u << (key & 31);
    const uint32_t old = __hip_atomic_fetch_or(reinterpret_cast<uint32_t*>(bits) + (key >> 5),
                                               bit, __ATOMIC_RELAXED, SWANN_TABLE_SCOPE);
    return (old & bit) == 0;
}

__device__ __forceinline__ float load_agent_f(const float* p) {
    const int b = __hip_atomic_load(reinterpret_cast<const int*>(p), __ATOMIC_RELAXED,
                                    SWANN_TABLE_SCOPE);
    return __int_as_float(b);
}

__device__ __forceinline__ void store_agent_f(float* p, float v) {
    __hip_atomic_store(reinterpret_cast<int*>(p), __float_as_int(v), __ATOMIC_RELAXED,
                       SWANN_TABLE_SCOPE);
}

__device__ __forceinline__ int pow2_ge(int x, int lo, int cap) {
    int n = lo;
    while (n < x && n < cap) n <<= 1;
    return n;
}

template <int BLOCK>
__device__ __forceinline__ void block_add(int* dst, int v) {
    // wave reduce then one LDS atomic per wave
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    if ((threadIdx.x & 63) == 0 && v != 0) atomicAdd(dst, v);
}

// ---------------------------------------------------------------------------
// init: local_search.cu:271-351
struct InitArgs {
    const void* X; const float* Qv; const int32_t* seeds;
    int32_t* ids; float* dist; uint8_t* expd; uint8_t* lin; int32_t* visited; int32_t* counters;
    int dim, J, V, L, H, metric;
    int64_t Q, n;
    int32_t* cache_id; float* cache_d; int Hc; float* bound; int ts;
    int vec_ok;
};

template <int TEAM, typename XT, int BLOCK>
__global__ __launch_bounds__(BLOCK) void init_kernel(InitArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    constexpr int NT = BLOCK / TEAM;
    const int tid = threadIdx.x, team = tid / TEAM, tl = tid % TEAM;
    const int64_t nb = a.Q * a.J;
    const int64_t flat = xcd_remap(blockIdx.x, nb);
    const int64_t q = flat / a.J;
    const int j = (int)(flat % a.J);
    const int dimp = qpad_floats(a.dim);
    const int nsort = pow2_ge(a.V, 2, kMaxD);

    float* sq = reinterpret_cast<float*>(smem);
    int* c_id = reinterpret_cast<int*>(sq + dimp);
    float* c_d = reinterpret_cast<float*>(c_id + nsort);
    int* s_id = reinterpret_cast<int*>(c_d + nsort);
    float* s_d = reinterpret_cast<float*>(s_id + nsort);
    uint8_t* c_l = reinterpret_cast<uint8_t*>(s_d + nsort);
    uint8_t* s_l = c_l + nsort;
    uint8_t* s_new = s_l + nsort;
    __shared__ int s_evals, s_fail;

    int32_t* vis = a.visited + flat * (int64_t)a.H;
    int32_t* ctr = a.counters + flat * kNctr;
    const float* qrow = a.Qv + q * (int64_t)a.dim;
    const XT* X = reinterpret_cast<const XT*>(a.X);

    for (int t = tid; t < a.dim; t += BLOCK) sq[qpad(t)] = qrow[t];
    if (a.H > 1) {
        if ((a.H & 3) == 0) {
            int4* v4 = reinterpret_cast<int4*>(vis);
            for (int t = tid; t < a.H / 4; t += BLOCK) v4[t] = make_int4(0, 0, 0, 0);
        } else {
            for (int t = tid; t < a.H; t += BLOCK) vis[t] = 0;
        }
    }
    // The query's table and bound belong to all J branches; they clear it
    // between them (local_search.cu:302-313).
    if (a.Hc > 0 && a.ts == 0) {
        // claim bits, Hc / 32 words a query
        const int64_t nw = a.Hc >> 5;
        int32_t* bw = a.cache_id + q * nw;
        if ((nw & 3) == 0 && (reinterpret_cast<uintptr_t>(bw) & 15) == 0) {
            int4* b4 = reinterpret_cast<int4*>(bw);
            for (int64_t t = j * BLOCK + tid; t < nw / 4; t += a.J * BLOCK)
                b4[t] = make_int4(0, 0, 0, 0);
        } else {
            for (int64_t t = j * BLOCK + tid; t < nw; t += a.J * BLOCK) bw[t] = 0;
        }
    } else if (a.Hc > 0 && a.ts == 2) {
        // interleaved (id, d) pairs, one 8-byte store each
        int2* p2 = reinterpret_cast<int2*>(a.cache_id + q * (int64_t)a.Hc * 2);
        const int fm = __float_as_int(FLT_MAX);
        for (int t = j * BLOCK + tid; t < a.Hc; t += a.J * BLOCK) p2[t] = make_int2(0, fm);
    } else if (a.Hc > 0) {
        int32_t* cid = a.cache_id + q * (int64_t)a.Hc;
        float* cdd = a.cache_d + q * (int64_t)a.Hc;
        if ((a.Hc & 3) == 0) {
            int4* i4 = reinterpret_cast<int4*>(cid);
            float4* f4 = reinterpret_cast<float4*>(cdd);
            for (int t = j * BLOCK + tid; t < a.Hc / 4; t += a.J * BLOCK) {
                i4[t] = make_int4(0, 0, 0, 0);
                f4[t] = make_float4(FLT_MAX, FLT_MAX, FLT_MAX, FLT_MAX);
            }
        } else {
            for (int t = j * BLOCK + tid; t < a.Hc; t += a.J * BLOCK) {
                cid[t] = 0;
                cdd[t] = FLT_MAX;
            }
        }
    }
    if (a.bound && j == 0 && tid == 0) a.bound[q] = FLT_MAX;
    for (int i = tid; i < nsort; i += BLOCK) { c_id[i] = -1; c_d[i] = FLT_MAX; c_l[i] = 0; s_new[i] = 0; }
    if (tid == 0) { s_evals = 0; s_fail = 0; }
    __syncthreads();

    // Seeds: a repeated seed is kept once, the first occurrence winning
    // (the visited table dedups, local_search.cu:318-340).  One lane inserts
    // them in seed order so the surviving lineage never depends on a race.
    const int32_t* sd = a.seeds + flat * (int64_t)a.V;
    if (tid == 0) {
        int fail = 0;
        for (int si = 0; si < a.V; ++si) {
            const int v = sd[si];
            if (v < 0 || v >= a.n) continue;            // out-of-range ids are empty slots
            int isnew = 1;
            if (a.H > 1) isnew = vis_insert(vis, a.H, v, &fail);
            s_new[si] = (uint8_t)isnew;
        }
        s_fail = fail;
    }
    __syncthreads();
    int evals = 0;
    for (int si = team; si < a.V; si += NT) {
        if (!s_new[si]) continue;                        // uniform within the team
        const int v = sd[si];
        const float d = team_dist_m<TEAM, XT>(sq, X + (int64_t)v * a.dim, a.dim, tl,
                                             a.vec_ok, a.metric);
        // A NaN distance (NaN in the query or the row) cannot be ordered:
        // the seed is scored but left out, so the rank sort below stays a
        // permutation.
        if (tl == 0) {
            ++evals;
            if (d == d) { c_id[si] = v; c_d[si] = d; c_l[si] = (uint8_t)si; }
        }
    }
    block_add<BLOCK>(&s_evals, evals);
    __syncthreads();
    // rank sort of the nsort slots by (d, id), ties by slot (a stable sort)
    for (int i = tid; i < nsort; i += BLOCK) {
        const int id = c_id[i]; const float d = c_d[i];
        int r = 0;
        for (int t = 0; t < nsort; ++t) {
            const int it = c_id[t]; const float dt = c_d[t];
            r += (lt(dt, it, d, id) || (dt == d && it == id && t < i)) ? 1 : 0;
        }
        s_id[r] = id; s_d[r] = d; s_l[r] = c_l[i];
    }
    __syncthreads();
    const int64_t qb = flat * (int64_t)a.L;
    for (int i = tid; i < a.L; i += BLOCK) {
        const bool ok = (i < nsort) && (s_id[i] >= 0);
        a.ids[qb + i] = ok ? s_id[i] : -1;
        a.dist[qb + i] = ok ? s_d[i] : FLT_MAX;
        a.expd[qb + i] = ok ? 0 : 1;
        a.lin[qb + i] = ok ? s_l[i] : 0;
    }
    for (int i = tid; i < kNctr; i += BLOCK)
        ctr[i] = (i == 1) ? s_evals : (i == 2) ? s_fail : 0;
}

// ---------------------------------------------------------------------------
// advance: local_search.cu:353-688
struct AdvArgs {
    const void* X; const int32_t* G; const float* Qv;
    int32_t* ids; float* dist; uint8_t* expd; uint8_t* lin; int32_t* visited; int32_t* counters;
    int dim, D, J, L, H, metric, delta, max_exp, policy, V;
    float stop_eps; int kstop;
    int32_t* cache_id; float* cache_d; int Hc; float* bound; int exclusive; int ts;
    int stall_patience; float crowd_frac;
    const int32_t* active; int64_t nblocks, nbranch, n;
    int vec_ok;
    const int32_t* codes; const float* calpha; const float* cmu; int cwords; float cmargin;
    int remap;                   // xcd_remap the blocks (a query's branches on one XCD)
};

// The advance of one branch a workgroup.  CODES: the sign-code pre-filter
// runs (a.codes set); a template parameter, so that the plain search's kernel
// carries none of the filter's registers.
template <int TEAM, typename XT, int BLOCK, bool CODES>
__device__ __forceinline__ void advance_body(const AdvArgs& a) {
    extern __shared__ __align__(16) unsigned char smem[];
    constexpr int NT = BLOCK / TEAM;
    const int tid = threadIdx.x, team = tid / TEAM, tl = tid % TEAM;
    const int lane = tid & 63, wave = tid >> 6;
    const int64_t pos = a.remap ? xcd_remap(blockIdx.x, a.nblocks) : (int64_t)blockIdx.x;
    const int64_t flat = a.active ? (int64_t)a.active[pos] : pos;
    if (flat < 0 || flat >= a.nbranch) return;          // a bad active entry: no work
    const int64_t q = flat / a.J;
    const int L = a.L, D = a.D;
    const int dimp = qpad_floats(a.dim);
    const int nsort = pow2_ge(D, 2, kMaxD);

    // LDS carve-up; sizes must match advance_lds() on the host
    float* sq = reinterpret_cast<float*>(smem);
    // the query's bit planes for the code estimate (code_planes words)
    const int nw32 = (a.dim + 31) >> 5;
    uint32_t* cpl = reinterpret_cast<uint32_t*>(sq + dimp);
    int* qa_id = reinterpret_cast<int*>(cpl + (CODES ? nw32 * kPlanes : 0));
    float* qa_d = reinterpret_cast<float*>(qa_id + L);
    int* qb_id = reinterpret_cast<int*>(qa_d + L);
    float* qb_d = reinterpret_cast<float*>(qb_id + L);
    int* c_id = reinterpret_cast<int*>(qb_d + L);
    float* c_d = reinterpret_cast<float*>(c_id + nsort);
    int* u_id = reinterpret_cast<int*>(c_d + nsort);
    float* u_d = reinterpret_cast<float*>(u_id + nsort);
    int* k_id = reinterpret_cast<int*>(u_d + nsort);
    float* k_d = reinterpret_cast<float*>(k_id + nsort);
    int* w_v = reinterpret_cast<int*>(k_d + nsort);
    int* w_slot = w_v + nsort;
    int* w_nidx = w_slot + nsort;
    uint8_t* qa_e = reinterpret_cast<uint8_t*>(w_nidx + nsort);
    uint8_t* qa_l = qa_e + L;
    uint8_t* qb_e = qa_l + L;
    uint8_t* qb_l = qb_e + L;
    uint8_t* c_l = qb_l + L;
    uint8_t* u_l = c_l + nsort;
    uint8_t* k_l = u_l + nsort;

    __shared__ int s_ctr[kNctr];
    __shared__ int s_slot, s_p, s_plin, s_nkeep, s_nwork, s_nbr, s_cov, s_stall, s_crowd_run;
    __shared__ int s_npass;
    __shared__ unsigned s_retired[8];
    __shared__ float s_best_k, s_rad, s_qmu, s_qsum;
    __shared__ float s_cscale, s_cdelta;
    __shared__ int s_namb;

    int32_t* vis = a.visited + flat * (int64_t)a.H;
    int32_t* ctr = a.counters + flat * kNctr;
    const int64_t qb = flat * (int64_t)L;
    const int ts = a.ts;
    int32_t* cid = a.Hc == 0 ? nullptr
                 : a.cache_id + q * (ts == 0 ? (int64_t)(a.Hc >> 5) : (int64_t)a.Hc * ts);
    float* cdd = a.Hc > 0 && ts > 0 ? a.cache_d + q * (int64_t)a.Hc * ts : nullptr;
    const float* qrow = a.Qv + q * (int64_t)a.dim;
    const XT* X = reinterpret_cast<const XT*>(a.X);

    for (int t = tid; t < a.dim; t += BLOCK) sq[qpad(t)] = qrow[t];
    for (int i = tid; i < L; i += BLOCK) {
        qa_id[i] = a.ids[qb + i]; qa_d[i] = a.dist[qb + i];
        qa_e[i] = a.expd[qb + i]; qa_l[i] = a.lin[qb + i];
    }
    if (tid < kNctr) s_ctr[tid] = ctr[tid];
    if (tid < 8) s_retired[tid] = 0u;
    if (tid == 0) { s_best_k = FLT_MAX; s_stall = 0; s_crowd_run = 0; }
    __syncthreads();

    if (CODES && wave == 0) {
        // <q, mu> and sum(q), once per call, in a fixed order that does not
        // depend on BLOCK: lane l sums t = l, l + 64, ..., then the wave folds
        // with off = 32 .. 1.  (The reference sums through shared-memory
        // atomics, local_search.cu:430-441, whose order is unspecified.)
        float m = 0.f, s = 0.f;
        for (int t = lane; t < a.dim; t += 64) {
            const float qt = sq[qpad(t)];
            m = m + qt * a.cmu[t];
            s = s + qt;
        }
        m = team_fold_add<64>(m);
        s = team_fold_add<64>(s);
        if (lane == 0) { s_qmu = m; s_qsum = s; }
        // the cheap estimate's quantisation: scale, bit planes, error bound
        // (any summation order: these only bound, they decide nothing alone)
        float amax = 0.f, sabs = 0.f;
        for (int t = lane; t < a.dim; t += 64) {
            const float qt = fabsf(sq[qpad(t)]);
            amax = fmaxf(amax, qt);
            sabs = sabs + qt;
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
            amax = fmaxf(amax, __shfl_xor(amax, off, 64));
            sabs = sabs + __shfl_xor(sabs, off, 64);
        }
        const float cs = amax / (float)(kPlaneOff - 1);
        const float inv = cs > 0.f ? 1.f / cs : 0.f;
        float err = 0.f;
        for (int w = lane; w < nw32; w += 64) {
            uint32_t pl[kPlanes];
#pragma unroll
            for (int b = 0; b < kPlanes; ++b) pl[b] = 0u;
            for (int j = 0; j < 32 && w * 32 + j < a.dim; ++j) {
                const float qt = sq[qpad(w * 32 + j)];
                float kq = rintf(qt * inv);
                kq = fminf(fmaxf(kq, -(float)(kPlaneOff - 1)), (float)(kPlaneOff - 1));
                err = err + fabsf(qt - cs * kq);
                const uint32_t u = (uint32_t)((int)kq + kPlaneOff);
#pragma unroll
                for (int b = 0; b < kPlanes; ++b) pl[b] |= ((u >> b) & 1u) << j;
            }
#pragma unroll
            for (int b = 0; b < kPlanes; ++b) cpl[w * kPlanes + b] = pl[b];
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) err = err + __shfl_xor(err, off, 64);
        if (lane == 0) {
            // E as summed here rounds: bound it from above (dim u relative for
            // the sum, 4 u |q_i| a term for the rounded products and
            // differences), then add the reference sum's own rounding
            const float u = 5.9604645e-08f;
            const float e = err * 1.002f + 8.f * u * sabs;
            const float dl = (e + ((float)a.dim + 64.f) * u * 1.01f * sabs + u * (sabs + e)) *
                             1.001f;
            s_cscale = cs;
            // a query with a NaN or infinity leaves no usable bound: every
            // decision then takes the exact sum
            s_cdelta = (dl == dl && dl < INFINITY && cs == cs && cs < INFINITY) ? dl : INFINITY;
        }
    }
    if (CODES) __syncthreads();

    int r_evals = 0, r_fail = 0, r_hits = 0, r_claim = 0;
    const bool early = (a.stop_eps >= 0.f);
    const int kr = (a.kstop < L) ? a.kstop : L;

    for (int step = 0; step < a.delta; ++step) {
        // ---- pick the slot to expand (wave 0; local_search.cu:452-517) ----
        // The budget test is made here, by wave 0 alone, and published with
        // the slot: the other waves never read a counter wave 0 may be moving.
        if (wave == 0 && s_ctr[0] >= a.max_exp) {
            if (lane == 0) s_slot = -2;
        } else if (wave == 0) {
            float radius = (kr > 0 && qa_id[kr - 1] >= 0) ? qa_d[kr - 1] : FLT_MAX;
            if (a.bound) {
                const float gb = load_agent_f(a.bound + q);
                if (gb < radius) radius = gb;
            }
            const float limit = (radius == FLT_MAX) ? FLT_MAX : radius * (1.f + a.stop_eps);
            int slot = -1;
            if (a.policy == SWANN_POLICY_ROUND_ROBIN && a.V > 1) {
                for (int turn = 0; turn < a.V && slot < 0; ++turn) {
                    const int want = (s_ctr[0] + turn) % a.V;
                    if (s_retired[want >> 5] & (1u << (want & 31))) continue;
                    int found = -1;
                    for (int b = 0; b < L && found < 0; b += 64) {
                        const int i = b + lane;
                        const bool ok = i < L && qa_id[i] >= 0 && qa_e[i] == 0 && qa_l[i] == want;
                        const uint64_t m = __ballot(ok);
                        if (m) found = b + __builtin_ctzll(m);
                    }
                    if (found < 0 || (early && qa_d[found] > limit)) {
                        if (lane == 0) s_retired[want >> 5] |= (1u << (want & 31));
                        continue;
                    }
                    slot = found;
                }
                if (slot < 0 && !early) {
                    for (int b = 0; b < L && slot < 0; b += 64) {
                        const int i = b + lane;
                        const uint64_t m = __ballot(i < L && qa_id[i] >= 0 && qa_e[i] == 0);
                        if (m) slot = b + __builtin_ctzll(m);
                    }
                }
            } else {
                int found = -1;
                for (int b = 0; b < L && found < 0; b += 64) {
                    const int i = b + lane;
                    bool ok = i < L && qa_id[i] >= 0 && qa_e[i] == 0;
                    if (ok) {
                        const unsigned li = qa_l[i];
                        ok = !(s_retired[li >> 5] & (1u << (li & 31)));
                    }
                    const uint64_t m = __ballot(ok);
                    if (m) found = b + __builtin_ctzll(m);
                }
                if (found >= 0 && (!early || qa_d[found] <= limit)) slot = found;
            }
            if (lane == 0) {
                s_slot = slot;
                s_rad = limit;                  // the code filter's line (:471-478)
                if (slot >= 0) {
                    qa_e[slot] = 1;
                    s_p = qa_id[slot];
                    s_plin = qa_l[slot];
                    s_ctr[0] += 1;
                } else {
                    s_ctr[3] = 1;
                }
                s_nwork = 0; s_nkeep = 0; s_nbr = 0; s_cov = 0; s_npass = 0; s_namb = 0;
            }
        }
        for (int i = tid; i < nsort; i += BLOCK) { c_id[i] = -1; c_d[i] = FLT_MAX; c_l[i] = 0; }
        __syncthreads();
        if (s_slot < 0) break;
        const int p = s_p;
        const uint8_t plin = (uint8_t)s_plin;

        // ---- screen the neighbours, one lane each ----
        // (a queue id is always a corpus row; the range test keeps a corrupt
        // state from indexing the graph out of bounds)
        int nbr = 0, cov = 0;
        const int deg = (p >= 0 && p < a.n) ? D : 0;
        for (int nidx = tid; nidx < deg; nidx += BLOCK) {
            const int v = a.G[(int64_t)p * D + nidx];
            if (v < 0 || v >= a.n) continue;                 // -1 (or out of range): no edge
            ++nbr;
            int isnew = 1;
            if (a.H > 1) isnew = vis_insert(vis, a.H, v, &r_fail);
            if (!isnew) { ++cov; continue; }
            int slot = -1, claimed = 0;
            float d = FLT_MAX;
            if (a.Hc > 0 && ts == 0) {
                if (!claim_bit(cid, v)) { ++r_hits; ++cov; continue; }  // owned elsewhere
                ++r_claim;
            } else if (a.Hc > 0 && ts == 2) {
                slot = cache_slot_pair(reinterpret_cast<unsigned long long*>(cid), a.Hc, v,
                                       &claimed, &d);
            } else if (a.Hc > 0) {
                slot = cache_slot(cid, a.Hc, ts, v, &claimed);
                d = (slot >= 0 && !claimed) ? load_agent_f(cdd + (int64_t)slot * ts) : FLT_MAX;
            }
            if (a.exclusive && slot >= 0 && !claimed && d != FLT_MAX) {
                ++r_hits; ++cov;                                // another branch owns it
            } else if (d == FLT_MAX) {
                const int w = atomicAdd(&s_nwork, 1);
                w_v[w] = v; w_slot[w] = slot; w_nidx[w] = nidx | (claimed << 16);
            } else {
                ++r_hits;                                       // cached distance
                c_id[nidx] = v; c_d[nidx] = d; c_l[nidx] = plin;
            }
        }
        __syncthreads();

        // ---- score the survivors, TEAM lanes per distance ----
        const int nw = s_nwork;
        auto record = [&](int w, int v, float d) {
            const int slot = w_slot[w];
            const int packed = w_nidx[w];
            const int nidx = packed & 0xffff, claimed = packed >> 16;
            if (slot >= 0) { store_agent_f(cdd + (int64_t)slot * ts, d); ++r_claim; }
            ++r_evals;
            const bool taken = a.exclusive && slot >= 0 && !claimed && d != FLT_MAX;
            if (taken) ++cov;
            else { c_id[nidx] = v; c_d[nidx] = d; c_l[nidx] = plin; }
        };
        if (!CODES) {
            for (int w = team; w < nw; w += NT) {
                const int v = w_v[w];
                const float d = team_dist_m<TEAM, XT>(sq, X + (int64_t)v * a.dim, a.dim, tl,
                                                     a.vec_ok, a.metric);
                if (tl == 0) record(w, v, d);
            }
        } else {
            // decide from the code before reading the row (:560-575); a
            // skipped neighbour stays a candidate at FLT_MAX, unscored, with
            // its table slot claimed but never filled.  Three passes: every
            // item is bracketed by the cheap estimate (team_code_k) and is
            // skipped, listed to read (u_id) or, when the bracket straddles
            // the line, listed for the exact estimate (k_id; both free until
            // the keep step); then the exact estimate decides those; then the
            // teams score the listed rows, so no team waits on a row that
            // another team's item needs.
            const float rad = s_rad;
            const float line = rad + a.cmargin;
            auto skip = [&](int w, int v) {
                const int nidx = w_nidx[w] & 0xffff;
                atomicAdd(&s_ctr[3], 1);
                c_id[nidx] = v; c_d[nidx] = FLT_MAX; c_l[nidx] = plin;
            };
            // An item's estimate waits on two loads, its code words and its
            // scale; the next item's are issued before this one's estimate,
            // so a team waits for them once an item, not twice, and behind
            // the current item's arithmetic.
            unsigned nxt[kCodeWords];
            float nal = 0.f;
            if (rad != FLT_MAX && team < nw) {
                const int v0 = w_v[team];
                code_fetch<TEAM>(a.codes + (int64_t)v0 * a.cwords, tl, nw32, nxt);
                nal = a.calpha[v0];
            }
            for (int w = team; w < nw; w += NT) {
                const int v = w_v[w];
                if (rad == FLT_MAX) {            // no line yet: nothing is skipped
                    if (tl == 0) u_id[atomicAdd(&s_npass, 1)] = w;
                    continue;
                }
                unsigned cur[kCodeWords];
#pragma unroll
                for (int j = 0; j < kCodeWords; ++j) cur[j] = nxt[j];
                const float al = nal;
                if (w + NT < nw) {
                    const int vn = w_v[w + NT];
                    code_fetch<TEAM>(a.codes + (int64_t)vn * a.cwords, tl, nw32, nxt);
                    nal = a.calpha[vn];
                }
                const int kt = team_code_k<TEAM>(cpl, a.codes + (int64_t)v * a.cwords, cur,
                                                 nw32, a.dim, tl);
                if (tl == 0) {
                    const float sc = s_cscale * (float)kt;
                    const float dl = s_cdelta + 1e-6f * (fabsf(sc) + s_cdelta) + 1e-30f;
                    auto est = [&](float sum) { return 1.f - (al * (2.f * sum - s_qsum) + s_qmu); };
                    // the two ends bracket the reference's value for either
                    // sign of alpha; a NaN end fails both tests
                    const float e1 = est(sc + dl), e2 = est(sc - dl);
                    if (e1 > line && e2 > line) skip(w, v);
                    else if (e1 <= line && e2 <= line) u_id[atomicAdd(&s_npass, 1)] = w;
                    else k_id[atomicAdd(&s_namb, 1)] = w;
                }
            }
            __syncthreads();
            const int namb = s_namb;
            for (int k = team; k < namb; k += NT) {
                const int w = k_id[k];
                const int v = w_v[w];
                unsigned head[kCodeWords];
                code_fetch<TEAM>(a.codes + (int64_t)v * a.cwords, tl, a.cwords, head);
                const float est = team_code_ip<TEAM>(sq, a.codes + (int64_t)v * a.cwords,
                                                     head, a.calpha[v], s_qmu, s_qsum, a.dim,
                                                     a.cwords, tl);
                if (tl == 0) {                   // the team's total is in its lane 0
                    if (est > line) skip(w, v);
                    else u_id[atomicAdd(&s_npass, 1)] = w;
                }
            }
            __syncthreads();
            const int npass = s_npass;
            for (int k = team; k < npass; k += NT) {
                const int w = u_id[k];
                const int v = w_v[w];
                const float d = team_dist_m<TEAM, XT>(sq, X + (int64_t)v * a.dim, a.dim, tl,
                                                     a.vec_ok, a.metric);
                if (tl == 0) record(w, v, d);
            }
        }
        if (a.crowd_frac > 0.f) { block_add<BLOCK>(&s_nbr, nbr); block_add<BLOCK>(&s_cov, cov); }
        __syncthreads();

        // ---- keep what can still enter the queue (:607-625) ----
        const float worst = (qa_id[L - 1] >= 0) ? qa_d[L - 1] : FLT_MAX;
        for (int i = tid; i < nsort; i += BLOCK) {
            const int v = c_id[i];
            const float d = c_d[i];
            // d == d drops a NaN distance, which has no place in the (d, id)
            // order the rank sort and the merge rely on
            if (v >= 0 && d == d && (worst == FLT_MAX || d <= worst)) {
                const int k = atomicAdd(&s_nkeep, 1);
                u_id[k] = v; u_d[k] = d; u_l[k] = c_l[i];
            }
        }
        __syncthreads();
        const int nk = s_nkeep;
        int msort = 2;
        while (msort < nk) msort <<= 1;
        if (msort > nsort) msort = nsort;
        // rank sort by (d, id); exact duplicates keep their order
        for (int i = tid; i < nk; i += BLOCK) {
            const int id = u_id[i]; const float d = u_d[i];
            int r = 0;
            for (int t = 0; t < nk; ++t) {
                const int it = u_id[t]; const float dt = u_d[t];
                r += (lt(dt, it, d, id) || (dt == d && it == id && t < i)) ? 1 : 0;
            }
            k_id[r] = id; k_d[r] = d; k_l[r] = u_l[i];
        }
        for (int i = nk + tid; i < msort; i += BLOCK) { k_id[i] = -1; k_d[i] = FLT_MAX; k_l[i] = 0; }
        if (tid == 0) { s_ctr[8] += nk; s_ctr[9] += 1; }
        __syncthreads();

        // ---- merge-path into the other buffer (:637-650) ----
        for (int o = tid; o < L; o += BLOCK) {
            int lo = o - msort > 0 ? o - msort : 0;
            int hi = o < L ? o : L;
            while (lo < hi) {
                const int i = (lo + hi) >> 1, jj = o - i;
                if (jj > 0 && !lt(k_d[jj - 1], k_id[jj - 1], qa_d[i], qa_id[i])) lo = i + 1;
                else hi = i;
            }
            const int i = lo, jj = o - i;
            const bool takeA = (jj >= msort) || (i < L && lt(qa_d[i], qa_id[i], k_d[jj], k_id[jj]));
            int nid; float nd; uint8_t ne, nl;
            if (takeA) { nid = qa_id[i]; nd = qa_d[i]; ne = qa_e[i]; nl = qa_l[i]; }
            else { nid = k_id[jj]; nd = k_d[jj]; ne = 0; nl = k_l[jj]; }
            if (nid < 0) { nd = FLT_MAX; ne = 1; nl = 0; }
            qb_id[o] = nid; qb_d[o] = nd; qb_e[o] = ne; qb_l[o] = nl;
        }
        __syncthreads();
        { int* t = qa_id; qa_id = qb_id; qb_id = t; }
        { float* t = qa_d; qa_d = qb_d; qb_d = t; }
        { uint8_t* t = qa_e; qa_e = qb_e; qb_e = t; }
        { uint8_t* t = qa_l; qa_l = qb_l; qb_l = t; }

        // ---- bound, crowd, stall (:655-682) ----
        if (tid == 0) {
            if (a.bound && kr > 0 && qa_id[kr - 1] >= 0)
                __hip_atomic_fetch_min(reinterpret_cast<int*>(a.bound + q),
                                       __float_as_int(qa_d[kr - 1]), __ATOMIC_RELAXED,
                                       SWANN_TABLE_SCOPE);
            if (a.crowd_frac > 0.f) {
                const float cf = (s_nbr > 0) ? ((float)s_cov / (float)s_nbr) : 0.f;
                if (cf >= a.crowd_frac) {
                    if (++s_crowd_run >= 2) {
                        const unsigned li = (unsigned)plin;
                        s_retired[li >> 5] |= (1u << (li & 31));
                        s_ctr[7] += 1;
                        s_crowd_run = 0;
                    }
                } else {
                    s_crowd_run = 0;
                }
            }
            if (a.stall_patience > 0) {
                const float bk = (kr > 0 && qa_id[kr - 1] >= 0) ? qa_d[kr - 1] : FLT_MAX;
                if (bk < s_best_k) { s_best_k = bk; s_stall = 0; } else { s_stall += 1; }
                if (s_stall >= a.stall_patience) s_ctr[6] = 1;
            }
        }
        __syncthreads();
        if (a.stall_patience > 0 && s_stall >= a.stall_patience) break;
    }

    block_add<BLOCK>(&s_ctr[1], r_evals);
    block_add<BLOCK>(&s_ctr[2], r_fail);
    block_add<BLOCK>(&s_ctr[4], r_hits);
    block_add<BLOCK>(&s_ctr[5], r_claim);
    __syncthreads();
    for (int i = tid; i < L; i += BLOCK) {
        a.ids[qb + i] = qa_id[i]; a.dist[qb + i] = qa_d[i];
        a.expd[qb + i] = qa_e[i]; a.lin[qb + i] = qa_l[i];
    }
    if (tid < kNctr) ctr[tid] = s_ctr[tid];
}

template <int TEAM, typename XT, int BLOCK>
__global__ __launch_bounds__(BLOCK) void advance_kernel(AdvArgs a) {
    advance_body<TEAM, XT, BLOCK, false>(a);
}

template <int TEAM, typename XT, int BLOCK>
__global__ __launch_bounds__(BLOCK) void advance_codes_kernel(AdvArgs a) {
    advance_body<TEAM, XT, BLOCK, true>(a);
}

// ---------------------------------------------------------------------------
// merge (semantics of local_search.cu:863-919): a query's n = V*kk branch
// results in (distance, id) order with invalid ids after everything; an entry
// whose id equals its predecessor's in that order is dropped; the first k
// kept, padded with (-1, +inf).
//
// Each entry becomes one 64-bit key ordered as (distance, id) is: the high
// word is the distance's bit pattern made monotone (+0 and -0 share a value,
// as the float comparison has them equal), the low word 2*id plus 1 for a
// distance of -0, so keys of different ids order by id and a zero's sign
// rides along.  An invalid id is the key (+inf, INT32_MAX), where the walk
// ends.  The walk through the sorted order is a chain of successor queries --
// the least key >= lo, then lo = that key + 1 -- each one wave-wide minimum
// over keys held in registers; nothing is sorted.  Equal keys are visited
// once, which drops their later copies as the predecessor rule does.
constexpr int kMergeWaveMax = 32;      // keys per lane in the one-wave kernel
constexpr int kMergeBlockThreads = 1024;

__device__ __forceinline__ uint64_t merge_key(int32_t id, float d) {
    if (id < 0) id = INT32_MAX, d = INFINITY;
    uint32_t b = __float_as_uint(d);
    const uint32_t neg0 = b == 0x80000000u;
    if (neg0) b = 0;
    const uint32_t m = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return ((uint64_t)m << 32) | ((uint32_t)id << 1) | neg0;
}

__device__ __forceinline__ float merge_key_dist(uint64_t key) {
    if (key & 1) return -0.0f;
    const uint32_t m = (uint32_t)(key >> 32);
    return __uint_as_float((m & 0x80000000u) ? (m & 0x7FFFFFFFu) : ~m);
}

// One step of the walk, shared by both kernels: `m` is the least key >= lo
// (all ones when none is left).  Returns false when the walk is over.
__device__ __forceinline__ bool merge_visit(uint64_t m, int& prev_id, int& w, uint64_t& lo,
                                            int32_t* __restrict__ oi, float* __restrict__ od,
                                            int64_t row, bool writer) {
    const int id = (int)((uint32_t)m >> 1);
    if (id == INT32_MAX) return false;       // invalid entries (or nothing) remain
    if (id != prev_id) {
        if (writer) { oi[row + w] = id; od[row + w] = merge_key_dist(m); }
        ++w;
    }
    prev_id = id;
    lo = m + 1;
    return true;
}

// Branch results sit in rows of `ld` slots, `kk` of them used: entry i of a
// query (i < V*kk) is branch i / kk, slot i % kk.  A thread walks its entries
// t, t + S, t + 2S, ... by carrying (branch, slot) and adding (S / kk, S % kk).
struct MergeWalk {
    int64_t v, j;
    __device__ MergeWalk(int64_t i, int kk) : v(i / kk), j(i % kk) {}
    __device__ __forceinline__ int64_t at(int64_t ld) const { return v * ld + j; }
    __device__ __forceinline__ void step(int64_t sv, int sj, int kk) {
        v += sv;
        j += sj;
        if (j >= kk) { j -= kk; ++v; }
    }
};

// n <= 64*R: one wave per query, R keys per lane in registers.
template <int R>
__global__ __launch_bounds__(64) void merge_wave_kernel(const int32_t* __restrict__ bids,
                                                        const float* __restrict__ bdist,
                                                        int32_t* __restrict__ oi,
                                                        float* __restrict__ od, int64_t q0,
                                                        int n, int kk, int64_t ld, int k) {
    const int64_t q = q0 + blockIdx.x;
    const int lane = threadIdx.x;
    const int64_t base = q * (int64_t)(n / kk) * ld;
    uint64_t key[R];
    MergeWalk at(lane, kk);
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int i = lane + 64 * r;
        const int64_t a = base + at.at(ld);
        key[r] = i < n ? merge_key(bids[a], bdist[a]) : ~0ull;
        at.step(64 / kk, 64 % kk, kk);
    }
    const int64_t row = q * (int64_t)k;
    uint64_t lo = 0;
    int prev_id = -1, w = 0;
    for (int step = 0; step < n && w < k; ++step) {     // each step passes one key
        uint64_t m = ~0ull;
#pragma unroll
        for (int r = 0; r < R; ++r) m = key[r] >= lo ? umin64(m, key[r]) : m;
        m = wave_min_u64(m);
        if (!merge_visit(m, prev_id, w, lo, oi, od, row, lane == 0)) break;
    }
    for (int t = w + lane; t < k; t += 64) { oi[row + t] = -1; od[row + t] = INFINITY; }
}

// Any n: one 1024-thread workgroup per query; each step re-reads the keys
// (the query's n entries stay in L1/L2 after the first pass), the waves'
// minima meet in LDS, double-buffered so one barrier per step suffices.
__global__ __launch_bounds__(kMergeBlockThreads) void merge_block_kernel(
    const int32_t* __restrict__ bids, const float* __restrict__ bdist, int32_t* __restrict__ oi,
    float* __restrict__ od, int64_t q0, int64_t n, int kk, int64_t ld, int k) {
    constexpr int kWaves = kMergeBlockThreads / 64;
    __shared__ uint64_t part[2][kWaves];
    const int64_t q = q0 + blockIdx.x;
    const int64_t base = q * (n / kk) * ld;
    const int64_t row = q * (int64_t)k;
    uint64_t lo = 0;
    int prev_id = -1, w = 0;
    for (int64_t step = 0; step < n && w < k; ++step) {
        uint64_t m = ~0ull;
        MergeWalk at(threadIdx.x, kk);
        for (int64_t i = threadIdx.x; i < n; i += kMergeBlockThreads) {
            const int64_t a = base + at.at(ld);
            const uint64_t x = merge_key(bids[a], bdist[a]);
            m = x >= lo ? umin64(m, x) : m;
            at.step(kMergeBlockThreads / kk, kMergeBlockThreads % kk, kk);
        }
        m = wave_min_u64(m);
        if ((threadIdx.x & 63) == 0) part[step & 1][threadIdx.x >> 6] = m;
        __syncthreads();
        m = ~0ull;
#pragma unroll
        for (int v = 0; v < kWaves; ++v) m = umin64(m, part[step & 1][v]);
        if (!merge_visit(m, prev_id, w, lo, oi, od, row, threadIdx.x == 0)) break;
    }
    for (int t = w + (int)threadIdx.x; t < k; t += kMergeBlockThreads) {
        oi[row + t] = -1;
        od[row + t] = INFINITY;
    }
}

// Sum of counters[:, 2] into *out, one workgroup, no atomics: *out is
// written, never accumulated, so no clear is needed before it.
__global__ __launch_bounds__(1024) void overflow_kernel(const int32_t* __restrict__ ctr,
                                                        int64_t nbranch, int32_t* out) {
    __shared__ int part[16];
    int s = 0;
    for (int64_t i = threadIdx.x; i < nbranch; i += 1024) s += ctr[i * kNctr + 2];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
    __syncthreads();
    if (threadIdx.x == 0) {
        int t = 0;
        for (int w = 0; w < 16; ++w) t += part[w];
        *out = t;
    }
}

// ---------------------------------------------------------------------------
// host side
size_t init_lds(int dim, int V) {
    const int nsort = pow2_at_least(V, 2, kMaxD);
    return (size_t)qpad_floats(dim) * 4 + (size_t)nsort * (4 + 4 + 4 + 4 + 1 + 1 + 1);
}

// `codes`: the sign-code filter is on (the query's bit planes join the LDS)
size_t advance_lds(int dim, int D, int L, bool codes) {
    const int nsort = pow2_at_least(D, 2, kMaxD);
    return (size_t)qpad_floats(dim) * 4 + (codes ? (size_t)((dim + 31) / 32) * kPlanes * 4 : 0) +
           (size_t)L * (4 + 4 + 4 + 4) + (size_t)nsort * (4 * 9) + (size_t)L * 4 +
           (size_t)nsort * 3;
}

// The table is interleaved (id, d) pairs when cache_d is the word right after
// cache_id: two separate [Q, Hc] arrays cannot overlap that way.  Pairs are
// probed as 64-bit words, so they must start 8-byte aligned (checked by the
// entry points).  With no cache_d it is claim bits: Hc bits a query, stride 0.
int table_stride(const int32_t* cache_id, const float* cache_d, int Hc) {
    if (Hc > 0 && cache_id && !cache_d) return 0;
    if (Hc > 0 && cache_id &&
        reinterpret_cast<const char*>(cache_d) == reinterpret_cast<const char*>(cache_id) + 4)
        return 2;
    return 1;
}

int search_block_for(int64_t nbranch) {
    // option search_block = 64|256|1024 pins the workgroup size (tests use it
    // to run every layout on the same inputs)
    const int forced = option(kOptSearchBlock);
    if (forced == 64 || forced == 256 || forced == 1024) return forced;
    // Batch work fills 256 CUs with one-wave branches.  A smaller batch gets
    // four waves per branch, and a grid smaller than two branches per CU
    // (batch 1-8 at 32 branches) sixteen: an expansion's neighbours are then
    // scored by BLOCK / team teams at once instead of a few in turn, and a
    // branch's chain of expansions -- the latency at small batch -- is
    // shorter.  Four waves still beat one at 8,192 and 16,384 branches (C4,
    // team 32: 11.8 against 12.3 ms, 23.3 against 24.4 ms, the same
    // recall); one wave wins again at 65,536.
    if (nbranch >= 32768) return 64;
    return nbranch >= 512 ? 256 : 1024;
}

bool rows_vec_ok(const void* X, int dim, int x_dtype) {
    const int vec = x_dtype == SWANN_DTYPE_F16 ? 8 : 4;
    return (dim % vec == 0) && ((uintptr_t)X % 16 == 0);
}

#define SWANN_DISPATCH(KERNEL, TEAMV, DT, BLK, GRID, LDS, ST, ARGS)                         \
    do {                                                                                  \
        if ((DT) == SWANN_DTYPE_F32) {                                                    \
            SWANN_DISPATCH_T(KERNEL, float, TEAMV, BLK, GRID, LDS, ST, ARGS);             \
        } else {                                                                          \
            SWANN_DISPATCH_T(KERNEL, _Float16, TEAMV, BLK, GRID, LDS, ST, ARGS);          \
        }                                                                                 \
    } while (0)

#define SWANN_DISPATCH_B(KERNEL, T, TM, BLK, GRID, LDS, ST, ARGS)                          \
    do {                                                                                  \
        if ((BLK) == 64)                                                                  \
            hipLaunchKernelGGL((KERNEL<TM, T, 64>), GRID, dim3(64), LDS, ST, ARGS);       \
        else if ((BLK) == 256)                                                            \
            hipLaunchKernelGGL((KERNEL<TM, T, 256>), GRID, dim3(256), LDS, ST, ARGS);     \
        else                                                                              \
            hipLaunchKernelGGL((KERNEL<TM, T, 1024>), GRID, dim3(1024), LDS, ST, ARGS);   \
    } while (0)

#define SWANN_DISPATCH_T(KERNEL, T, TEAMV, BLK, GRID, LDS, ST, ARGS)                       \
    do {                                                                                  \
        switch (TEAMV) {                                                                  \
            case 4: SWANN_DISPATCH_B(KERNEL, T, 4, BLK, GRID, LDS, ST, ARGS); break;      \
            case 8: SWANN_DISPATCH_B(KERNEL, T, 8, BLK, GRID, LDS, ST, ARGS); break;      \
            case 16: SWANN_DISPATCH_B(KERNEL, T, 16, BLK, GRID, LDS, ST, ARGS); break;    \
            case 32: SWANN_DISPATCH_B(KERNEL, T, 32, BLK, GRID, LDS, ST, ARGS); break;    \
            default: SWANN_DISPATCH_B(KERNEL, T, 64, BLK, GRID, LDS, ST, ARGS); break;    \
        }                                                                                 \
    } while (0)

// Workgroups of one advance_kernel instance a CU holds at once (registers
// and LDS), from the runtime's occupancy query; 0 if the query fails.
template <int TEAM, typename XT>
int advance_occupancy(int block, size_t lds, bool codes) {
    int v = 0;
    hipError_t e;
    if (block == 64)
        e = codes ? hipOccupancyMaxActiveBlocksPerMultiprocessor(
                        &v, advance_codes_kernel<TEAM, XT, 64>, 64, lds)
                  : hipOccupancyMaxActiveBlocksPerMultiprocessor(
                        &v, advance_kernel<TEAM, XT, 64>, 64, lds);
    else if (block == 256)
        e = codes ? hipOccupancyMaxActiveBlocksPerMultiprocessor(
                        &v, advance_codes_kernel<TEAM, XT, 256>, 256, lds)
                  : hipOccupancyMaxActiveBlocksPerMultiprocessor(
                        &v, advance_kernel<TEAM, XT, 256>, 256, lds);
    else
        e = codes ? hipOccupancyMaxActiveBlocksPerMultiprocessor(
                        &v, advance_codes_kernel<TEAM, XT, 1024>, 1024, lds)
                  : hipOccupancyMaxActiveBlocksPerMultiprocessor(
                        &v, advance_kernel<TEAM, XT, 1024>, 1024, lds);
    return e == hipSuccess ? v : 0;
}

// Whether the advance puts a query's branches on one XCD (xcd_remap), where
// they share an L2: only when they are a small share of the workgroups one
// XCD holds at once (below).  Otherwise they would start in successive
// rounds, and the late ones find the early ones' nodes claimed and their
// bound set (at 128 branches a query, 256 or 1024 threads a branch, recall@10
// fell from 0.79 to 0.72 and 0.53), so the blocks keep their dispatch order
// instead, which spreads a query's branches over the XCDs; the table's and
// bound's atomics are agent scope and stay coherent across XCDs.
bool remap_branches(int J, int team, int x_dtype, int block, size_t lds, bool codes) {
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    int per_cu = 0;
    const bool f32 = x_dtype == SWANN_DTYPE_F32;
    switch (team) {
        case 4: per_cu = f32 ? advance_occupancy<4, float>(block, lds, codes)
                             : advance_occupancy<4, _Float16>(block, lds, codes); break;
        case 8: per_cu = f32 ? advance_occupancy<8, float>(block, lds, codes)
                             : advance_occupancy<8, _Float16>(block, lds, codes); break;
        case 16: per_cu = f32 ? advance_occupancy<16, float>(block, lds, codes)
                              : advance_occupancy<16, _Float16>(block, lds, codes); break;
        case 32: per_cu = f32 ? advance_occupancy<32, float>(block, lds, codes)
                              : advance_occupancy<32, _Float16>(block, lds, codes); break;
        default: per_cu = f32 ? advance_occupancy<64, float>(block, lds, codes)
                              : advance_occupancy<64, _Float16>(block, lds, codes); break;
    }
    if (per_cu <= 0) (void)hipGetLastError();
    // Grouped only while a query's branches take at most a quarter of the
    // XCD's resident slots.  In steady state a new query's branches enter one
    // freed slot at a time; when J is a large share of the XCD, the late ones
    // start after the early ones have set the bound and claimed the nodes,
    // and the search turns toward a serial schedule: C4 at 128 branches (J =
    // 0.44 of an XCD's one-wave slots) fell to recall 0.773 grouped against
    // 0.802 for branches that start together, while J = 0.11-0.17 of the
    // slots (C2, C3, C4 at 32 branches) matched it within 0.002.  Spread over
    // the eight XCDs, a query's branches are dispatched about together.
    return 4 * (int64_t)J <= (int64_t)(cus / kNumXcd) * per_cu;
}

}  // namespace
}  // namespace swann

using namespace swann;

extern "C" {

int swann_validate_init(int64_t n, int dim, int x_dtype, int64_t Q, int J, int V, int L,
                        int H, int metric, int team_size, int Hc) {
    clear_error();
    SWANN_REQUIRE(n > 0 && dim > 0, "X must be a non-empty [n, dim] matrix");
    SWANN_REQUIRE(x_dtype == SWANN_DTYPE_F32 || x_dtype == SWANN_DTYPE_F16,
                  "X: float32 or float16");
    SWANN_REQUIRE(metric == SWANN_METRIC_IP || metric == SWANN_METRIC_L2,
                  "metric must be 0 (ip) or 1 (l2)");
    SWANN_REQUIRE(team_size == 4 || team_size == 8 || team_size == 16 || team_size == 32 ||
                      team_size == 64,
                  "team_size must be 4, 8, 16, 32 or 64");
    SWANN_REQUIRE(Q >= 0 && J >= 1, "need Q >= 0 queries and J >= 1 branches");
    SWANN_REQUIRE(V >= 1 && V <= kMaxV, "seeds per branch must be in 1..%d (the init sort buffer)",
                  kMaxV);
    SWANN_REQUIRE(L >= 1 && L <= kMaxL, "L must be in 1..%d", kMaxL);
    SWANN_REQUIRE(is_pow2(H), "visited table size must be a power of two");
    SWANN_REQUIRE(Hc == 0 || is_pow2(Hc), "cache size must be a power of two");
    SWANN_REQUIRE(Q * (int64_t)J <= (int64_t)INT32_MAX / 64,
                  "Q*J = %lld branches exceed the launch limit", (long long)(Q * J));
    const size_t lds = init_lds(dim, V);
    SWANN_REQUIRE(lds <= kMaxLds, "init needs %zu B of LDS (limit %zu); lower the dimension", lds,
                  kMaxLds);
    return SWANN_OK;
}

int swann_validate_advance(int64_t n, int dim, int x_dtype, int D, int64_t Q, int J, int L,
                           int H, int metric, int team_size, int policy, int V, int Hc,
                           int64_t nactive, int cwords) {
    clear_error();
    SWANN_REQUIRE(n > 0 && dim > 0, "X must be a non-empty [n, dim] matrix");
    SWANN_REQUIRE(x_dtype == SWANN_DTYPE_F32 || x_dtype == SWANN_DTYPE_F16,
                  "X: float32 or float16");
    SWANN_REQUIRE(metric == SWANN_METRIC_IP || metric == SWANN_METRIC_L2,
                  "metric must be 0 (ip) or 1 (l2)");
    SWANN_REQUIRE(team_size == 4 || team_size == 8 || team_size == 16 || team_size == 32 ||
                      team_size == 64,
                  "team_size must be 4, 8, 16, 32 or 64");
    SWANN_REQUIRE(D >= 1 && D <= kMaxD, "graph degree exceeds MAXD (%d)", kMaxD);
    SWANN_REQUIRE(L >= 1 && L <= kMaxL, "L exceeds MAXL (%d)", kMaxL);
    SWANN_REQUIRE(V >= 1 && V <= 256, "lineage count exceeds 256 (lineage is a uint8)");
    SWANN_REQUIRE(policy == SWANN_POLICY_BEST || policy == SWANN_POLICY_ROUND_ROBIN,
                  "policy must be 0 (best) or 1 (round robin)");
    SWANN_REQUIRE(is_pow2(H), "visited table size must be a power of two");
    SWANN_REQUIRE(Hc == 0 || is_pow2(Hc), "cache size must be a power of two");
    SWANN_REQUIRE(Q >= 0 && J >= 1, "need Q >= 0 queries and J >= 1 branches");
    SWANN_REQUIRE(nactive >= 0 && nactive <= Q * (int64_t)J, "active list longer than Q*J");
    SWANN_REQUIRE(Q * (int64_t)J <= (int64_t)INT32_MAX / 64,
                  "Q*J = %lld branches exceed the launch limit", (long long)(Q * J));
    SWANN_REQUIRE(cwords >= 0, "cwords must be >= 0 (0: no sign codes)");
    SWANN_REQUIRE(cwords == 0 || metric == SWANN_METRIC_IP,
                  "the sign-code filter is written for the normalised inner-product corpora; "
                  "an unnormalised L2 corpus needs int8 codes and a stored squared norm");
    SWANN_REQUIRE(cwords == 0 || (int64_t)cwords * 32 >= dim,
                  "code words do not cover the dimension");
    const size_t lds = advance_lds(dim, D, L, cwords > 0);
    SWANN_REQUIRE(lds <= kMaxLds, "advance needs %zu B of LDS (limit %zu); lower L or the dimension",
                  lds, kMaxLds);
    return SWANN_OK;
}

int swann_init_states(const void* X, int x_dtype, int64_t n, int dim, const float* Qv, int64_t Q,
                      const int32_t* seeds, int J, int V, int32_t* ids, float* dist,
                      uint8_t* expd, uint8_t* lin, int L, int32_t* visited, int H,
                      int32_t* counters, int metric, int team_size, int32_t* cache_id,
                      float* cache_d, int Hc, float* bound, void* stream) {
    int rc = swann_validate_init(n, dim, x_dtype, Q, J, V, L, H, metric, team_size, Hc);
    if (rc) return rc;
    SWANN_REQUIRE(Q == 0 || (X && Qv && seeds && ids && dist && expd && lin && visited && counters),
                  "init_states: a required pointer is NULL");
    SWANN_REQUIRE(Hc == 0 || cache_id, "init_states: Hc > 0 needs cache_id");
    SWANN_REQUIRE(table_stride(cache_id, cache_d, Hc) != 2 ||
                      (reinterpret_cast<uintptr_t>(cache_id) & 7) == 0,
                  "init_states: an interleaved (id, d) table must be 8-byte aligned");
    SWANN_REQUIRE(table_stride(cache_id, cache_d, Hc) != 0 || (Hc >= n && Hc >= 32),
                  "init_states: claim bits (no cache_d) need Hc >= n and >= 32, got Hc = %d for "
                  "n = %lld", Hc, (long long)n);
    if (Q == 0) return SWANN_OK;
    InitArgs a{X, Qv, seeds, ids, dist, expd, lin, visited, counters, dim, J, V, L, H, metric,
               Q, n, Hc ? cache_id : nullptr, Hc ? cache_d : nullptr, Hc, bound,
               table_stride(cache_id, cache_d, Hc),
               rows_vec_ok(X, dim, x_dtype) ? 1 : 0};
    const int64_t nb = Q * J;
    const int block = search_block_for(nb);
    SWANN_DISPATCH(init_kernel, team_size, x_dtype, block, dim3((unsigned)nb), init_lds(dim, V),
                   (hipStream_t)stream, a);
    return launch_status("init_states");
}

int swann_advance(const void* X, int x_dtype, int64_t n, int dim, const int32_t* G, int D,
                  const float* Qv, int64_t Q, int J, int32_t* ids, float* dist, uint8_t* expd,
                  uint8_t* lin, int L, int32_t* visited, int H, int32_t* counters, int metric,
                  int team_size, int delta, int max_expansions, int policy, int V, float stop_eps,
                  int kstop, int32_t* cache_id, float* cache_d, int Hc, float* bound,
                  int exclusive, int stall_patience, float crowd_frac, const int32_t* active,
                  int64_t nactive, const int32_t* codes, int cwords, const float* alpha,
                  const float* cmu, float code_margin, void* stream) {
    int rc = swann_validate_advance(n, dim, x_dtype, D, Q, J, L, H, metric, team_size, policy, V,
                                    Hc, active ? nactive : 0, codes ? cwords : 0);
    if (rc) return rc;
    SWANN_REQUIRE(!codes || cwords > 0, "advance: codes given with cwords = 0");
    SWANN_REQUIRE(!codes || (alpha && cmu), "advance: codes need alpha and cmu");
    SWANN_REQUIRE(Q == 0 || (X && G && Qv && ids && dist && expd && lin && visited && counters),
                  "advance: a required pointer is NULL");
    SWANN_REQUIRE(Hc == 0 || cache_id, "advance: Hc > 0 needs cache_id");
    SWANN_REQUIRE(table_stride(cache_id, cache_d, Hc) != 2 ||
                      (reinterpret_cast<uintptr_t>(cache_id) & 7) == 0,
                  "advance: an interleaved (id, d) table must be 8-byte aligned");
    SWANN_REQUIRE(!exclusive || Hc > 0, "advance: exclusive claims need the shared table");
    SWANN_REQUIRE(table_stride(cache_id, cache_d, Hc) != 0 || (Hc >= n && Hc >= 32 && exclusive &&
                                                                 !codes),
                  "advance: claim bits (no cache_d) need Hc >= n and >= 32, exclusive claims and "
                  "no sign codes, got Hc = %d for n = %lld", Hc, (long long)n);
    const int64_t nb = active ? nactive : Q * J;
    if (nb == 0 || delta <= 0) return SWANN_OK;
    AdvArgs a{X, G, Qv, ids, dist, expd, lin, visited, counters, dim, D, J, L, H, metric,
              delta, max_expansions, policy, V, stop_eps, kstop,
              Hc ? cache_id : nullptr, Hc ? cache_d : nullptr, Hc, bound, exclusive ? 1 : 0,
              table_stride(cache_id, cache_d, Hc),
              stall_patience, crowd_frac, active, nb, Q * J, n,
              rows_vec_ok(X, dim, x_dtype) ? 1 : 0,
              codes, codes ? alpha : nullptr, codes ? cmu : nullptr, codes ? cwords : 0,
              code_margin};
    const int block = search_block_for(nb);
    const size_t lds = advance_lds(dim, D, L, codes != nullptr);
    a.remap = remap_branches(J, team_size, x_dtype, block, lds, codes != nullptr) ? 1 : 0;
    if (codes)
        SWANN_DISPATCH(advance_codes_kernel, team_size, x_dtype, block, dim3((unsigned)nb),
                       lds, (hipStream_t)stream, a);
    else
        SWANN_DISPATCH(advance_kernel, team_size, x_dtype, block, dim3((unsigned)nb),
                       lds, (hipStream_t)stream, a);
    return launch_status("advance");
}

int swann_merge_branches_strided(const int32_t* bids, const float* bdist, int64_t Q, int V, int kk,
                                 int64_t ld, int k, int32_t* out_ids, float* out_dist,
                                 void* stream) {
    clear_error();
    SWANN_REQUIRE(V >= 1 && kk >= 1, "expected (Q, V, kk) branch results with V, kk >= 1");
    SWANN_REQUIRE(ld >= kk, "row stride ld must be >= kk");
    const int64_t n = (int64_t)V * kk;
    SWANN_REQUIRE(k > 0 && k <= n, "k must be in 1..V*kk");
    SWANN_REQUIRE(Q >= 0, "Q out of range");
    if (Q == 0) return SWANN_OK;
    SWANN_REQUIRE(bids && bdist && out_ids && out_dist, "merge: a required pointer is NULL");
    const hipStream_t st = (hipStream_t)stream;
    // one workgroup per query, launched in slices of at most 2^20 queries
    constexpr int64_t kSlice = 1 << 20;
    for (int64_t q0 = 0; q0 < Q; q0 += kSlice) {
        const unsigned nq = (unsigned)(Q - q0 < kSlice ? Q - q0 : kSlice);
        if (n <= 64 * kMergeWaveMax) {
            const int r = (int)((n + 63) / 64);
            const int ni = (int)n;
            if (r <= 1)
                hipLaunchKernelGGL(merge_wave_kernel<1>, dim3(nq), dim3(64), 0, st, bids, bdist,
                                   out_ids, out_dist, q0, ni, kk, ld, k);
            else if (r <= 2)
                hipLaunchKernelGGL(merge_wave_kernel<2>, dim3(nq), dim3(64), 0, st, bids, bdist,
                                   out_ids, out_dist, q0, ni, kk, ld, k);
            else if (r <= 4)
                hipLaunchKernelGGL(merge_wave_kernel<4>, dim3(nq), dim3(64), 0, st, bids, bdist,
                                   out_ids, out_dist, q0, ni, kk, ld, k);
            else if (r <= 8)
                hipLaunchKernelGGL(merge_wave_kernel<8>, dim3(nq), dim3(64), 0, st, bids, bdist,
                                   out_ids, out_dist, q0, ni, kk, ld, k);
            else if (r <= 16)
                hipLaunchKernelGGL(merge_wave_kernel<16>, dim3(nq), dim3(64), 0, st, bids, bdist,
                                   out_ids, out_dist, q0, ni, kk, ld, k);
            else
                hipLaunchKernelGGL(merge_wave_kernel<32>, dim3(nq), dim3(64), 0, st, bids, bdist,
                                   out_ids, out_dist, q0, ni, kk, ld, k);
        } else {
            hipLaunchKernelGGL(merge_block_kernel, dim3(nq), dim3(kMergeBlockThreads), 0, st, bids,
                               bdist, out_ids, out_dist, q0, n, kk, ld, k);
        }
        const int rc = launch_status("merge_branches");
        if (rc) return rc;
    }
    return SWANN_OK;
}

int swann_merge_branches(const int32_t* bids, const float* bdist, int64_t Q, int V, int kk, int k,
                         int32_t* out_ids, float* out_dist, void* stream) {
    return swann_merge_branches_strided(bids, bdist, Q, V, kk, kk, k, out_ids, out_dist, stream);
}

int swann_overflow_async(const int32_t* counters, int64_t nbranch, int32_t* out, void* stream) {
    clear_error();
    SWANN_REQUIRE(nbranch >= 0 && out, "overflow: need an output pointer");
    SWANN_REQUIRE(nbranch == 0 || counters, "overflow: counters is NULL");
    hipLaunchKernelGGL(overflow_kernel, dim3(1), dim3(1024), 0, (hipStream_t)stream, counters,
                       nbranch, out);
    return launch_status("overflow");
}

}  // extern "C"
