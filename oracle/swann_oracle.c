/*
 * swann_oracle.c -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C CPU restatement of the reference algorithm for SWANN's search and
 * build path.  It is the checker the HIP library is compared against; it is
 * never linked into, loaded by, or called from the product library
 * (swann_amd/), which fails loudly when its HIP build is missing.
 *
 * Reference files followed (paths relative to the reference checkout):
 *   distance            swann/_refcpu.py:21-48, swann/csrc/local_search.cu:185-203
 *   branch init         swann/csrc/local_search.cu:271-351, swann/_refcpu.py:58-79
 *   branch step         swann/csrc/local_search.cu:451-683, swann/_refcpu.py:82-143
 *   visited table       swann/csrc/local_search.cu:94-110
 *   shared cache/claims swann/csrc/local_search.cu:169-183, :541-592
 *   bound               swann/csrc/local_search.cu:78-80, :466-469, :655-658
 *   branch merge        swann/csrc/local_search.cu:863-919, swann/_engine.py:377-402
 *   seed selection      swann/_select.py:93-128
 *   build sweep         swann/build.py:14-43
 *   robust prune        swann/build.py:46-91
 *   reverse edges       swann/build.py:94-150
 *
 * Where swann/_refcpu.py and local_search.cu differ, the kernel is followed:
 * the stop radius uses the min(kstop, L)-th queue entry (local_search.cu:464-465,
 * _refcpu.py:96 uses +inf when kstop > L), and an fp16 corpus is read with
 * vec = 8 (local_search.cu:131-133).
 *
 * Arithmetic: every distance is summed in fp32 in the kernel's lane-strided
 * order with the product and the sum rounded separately; build with
 * -ffp-contract=off.  Build-stage distances (sweep, prune, reverse, select) are
 * not bit-matched to any BLAS: dots are accumulated in double and the
 * reference's formula is applied in fp32.  The built graph is compared by
 * recall, not bit for bit.
 */
#include <float.h>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define SO_NCTR 10
#define SO_CPROBE 32
#define SO_SCHED_SERIAL 0   /* so_search_query: bound read as the previous step left it */
#define SO_SCHED_ROUNDS 1   /* ... as it was when the round began */
#define SO_SCHED_ROUNDS2 2  /* ... as it was when the round before began */
#define SO_MAXD 128
#define SO_MAXL 512

enum { SO_METRIC_IP = 0, SO_METRIC_L2 = 1 };
enum { SO_POLICY_BEST = 0, SO_POLICY_RR = 1 };
enum { SO_F32 = 0, SO_F16 = 1 };

/* ------------------------------------------------------------------ */
/* fp16 -> fp32, exact (IEEE binary16 is a subset of binary32).        */
static float so_half_to_float(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else {                      /* subnormal: renormalise */
            int e = -1;
            do { man <<= 1; ++e; } while ((man & 0x400u) == 0);
            man &= 0x3ffu;
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
        }
    } else if (exp == 31) {
        bits = sign | 0x7f800000u | (man << 13);
    } else {
        bits = sign | ((exp - 15 + 127) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

float so_half_to_float_export(uint16_t h) { return so_half_to_float(h); }

/* The same conversion through a 64K-entry table, filled once (thread-safe:
 * every writer stores identical values). */
static float so_h2f_table[65536];
static volatile int so_h2f_ready = 0;

static void so_h2f_init(void) {
    if (so_h2f_ready) return;
    for (uint32_t h = 0; h < 65536u; ++h) so_h2f_table[h] = so_half_to_float((uint16_t)h);
    __sync_synchronize();
    so_h2f_ready = 1;
}

static inline float so_elem(const void* X, int dt, int64_t i) {
    return dt == SO_F16 ? so_h2f_table[((const uint16_t*)X)[i]] : ((const float*)X)[i];
}

/* One distance in the kernel's order: lane l owns the blocks of `vec`
 * elements starting at l*vec, l*vec + team*vec, ...; lanes are then folded by
 * the halving tree off = team/2 .. 1.  IP returns 1 - dot. */
float so_team_distance(const float* q, const void* X, int dt, int64_t row, int dim,
                       int metric, int team) {
    if (dt == SO_F16) so_h2f_init();
    float lanes[64];
    const int vec = (dt == SO_F16) ? 8 : 4;
    const int64_t off0 = row * (int64_t)dim;
    for (int lane = 0; lane < team; ++lane) {
        float acc = 0.0f;
        for (int base = lane * vec; base < dim; base += team * vec) {
            for (int i = 0; i < vec; ++i) {
                const int t = base + i;
                if (t >= dim) break;
                const float xv = so_elem(X, dt, off0 + t);
                float term;
                if (metric == SO_METRIC_IP) {
                    term = q[t] * xv;
                } else {
                    const float df = q[t] - xv;
                    term = df * df;
                }
                acc = acc + term;
            }
        }
        lanes[lane] = acc;
    }
    for (int off = team / 2; off > 0; off >>= 1)
        for (int lane = 0; lane < off; ++lane) lanes[lane] = lanes[lane] + lanes[lane + off];
    return metric == SO_METRIC_IP ? 1.0f - lanes[0] : lanes[0];
}

/* (distance, id) strict order, local_search.cu:87-89 */
static inline int so_lt(float da, int ia, float db, int ib) {
    return (da < db) || (da == db && ia < ib);
}

/* Open addressing, linear probe, slot = key + 1, local_search.cu:94-110. */
static int so_vis_insert(int32_t* tab, int H, int key, int32_t* fail) {
    const uint32_t mask = (uint32_t)(H - 1);
    uint32_t pos = (2654435761u * (uint32_t)key) & mask;
    for (int probe = 0; probe < H; ++probe) {
        const int32_t cur = tab[pos];
        if (cur == 0) { tab[pos] = key + 1; return 1; }
        if (cur == key + 1) return 0;
        pos = (pos + 1) & mask;
    }
    *fail += 1;
    return 0;
}

/* Shared per-query table: bounded probe, local_search.cu:169-183. */
static int so_cache_slot(int32_t* cid, int Hc, int key, int* claimed) {
    const uint32_t mask = (uint32_t)(Hc - 1);
    uint32_t pos = (2654435761u * (uint32_t)key) & mask;
    for (int probe = 0; probe < SO_CPROBE; ++probe) {
        const int32_t cur = cid[pos];
        if (cur == key + 1) return (int)pos;
        if (cur == 0) { cid[pos] = key + 1; *claimed = 1; return (int)pos; }
        pos = (pos + 1) & mask;
    }
    return -1;
}

typedef struct { int id; float d; uint8_t l; int ord; } so_ent;

static int so_ent_cmp(const void* a, const void* b) {
    const so_ent* x = (const so_ent*)a;
    const so_ent* y = (const so_ent*)b;
    if (so_lt(x->d, x->id, y->d, y->id)) return -1;
    if (so_lt(y->d, y->id, x->d, x->id)) return 1;
    return (x->ord > y->ord) - (x->ord < y->ord);
}

static inline int so_pow2_cap(int x, int cap) {
    int n = 2;
    while (n < x && n < cap) n <<= 1;
    return n;
}

/* ------------------------------------------------------------------ */
/* Branch init, local_search.cu:271-351.  seeds: V ints.               */
void so_init_branch(const void* X, int dt, int dim, const float* q,
                    const int32_t* seeds, int V, int L, int H, int metric, int team,
                    int32_t* ids, float* dist, uint8_t* expd, uint8_t* lin,
                    int32_t* visited, int32_t* ctr) {
    const int nsort = so_pow2_cap(V, SO_MAXD);
    so_ent c[SO_MAXD];
    for (int i = 0; i < nsort; ++i) { c[i].id = -1; c[i].d = FLT_MAX; c[i].l = 0; c[i].ord = i; }
    for (int t = 0; t < H; ++t) visited[t] = 0;
    for (int i = 0; i < SO_NCTR; ++i) ctr[i] = 0;
    for (int si = 0; si < V; ++si) {
        const int v = seeds[si];
        if (v < 0) continue;
        int isnew = 1;
        if (H > 1) isnew = so_vis_insert(visited, H, v, &ctr[2]);
        if (!isnew) continue;
        c[si].id = v;
        c[si].d = so_team_distance(q, X, dt, v, dim, metric, team);
        c[si].l = (uint8_t)si;
        ctr[1] += 1;
    }
    qsort(c, (size_t)nsort, sizeof(so_ent), so_ent_cmp);
    for (int i = 0; i < L; ++i) {
        const int ok = (i < nsort) && (c[i].id >= 0);
        ids[i] = ok ? c[i].id : -1;
        dist[i] = ok ? c[i].d : FLT_MAX;
        expd[i] = ok ? 0 : 1;
        lin[i] = ok ? c[i].l : 0;
    }
}

/* Per-call branch locals, re-derived on every advance call
 * (local_search.cu:445-448). */
typedef struct {
    uint32_t retired[8];
    float best_k;
    int stall, crowd_run;
    int done;                       /* loop left: budget, exhaustion or stall */
} so_locals;

static void so_locals_reset(so_locals* s) {
    memset(s->retired, 0, sizeof(s->retired));
    s->best_k = FLT_MAX;
    s->stall = 0;
    s->crowd_run = 0;
    s->done = 0;
}

typedef struct {
    const void* X; int dt; int dim;
    const int32_t* G; int D;
    const float* q;
    int L, H, metric, team;
    int max_exp, policy, V;
    float stop_eps; int kstop;
    int32_t* cid; float* cdd; int Hc; float* bound; int exclusive;
    /* claim bits in place of the table (Hc < 0 at the entry points: -Hc
     * bits, one per row); NULL: off */
    uint32_t* cbits;
    /* where a step reads the bound (NULL: *bound itself).  The rounds
     * schedule points it at the value the bound had when the round began. */
    const float* bound_rd;
    int stall_patience; float crowd_frac;
    /* sign-code filter (local_search.cu:205-243, :560-575); codes == NULL: off */
    const int32_t* codes; int cwords; const float* calpha; float qmu, qsum, cmargin;
} so_cfg;

/* <q, mu> and sum(q) of the code filter, in the kernel's fixed order: 64
 * partial sums over t = l, l + 64, ..., folded with off = 32 .. 1.  (The
 * reference's shared-memory atomics, local_search.cu:430-441, leave the order
 * unspecified; any order is a legal reference result.) */
void so_code_sums(const float* q, const float* mu, int dim, float* qmu, float* qsum) {
    float m[64], s[64];
    for (int l = 0; l < 64; ++l) {
        m[l] = 0.0f; s[l] = 0.0f;
        for (int t = l; t < dim; t += 64) {
            const float p = q[t] * mu[t];
            m[l] = m[l] + p;
            s[l] = s[l] + q[t];
        }
    }
    for (int off = 32; off > 0; off >>= 1)
        for (int l = 0; l < off; ++l) { m[l] = m[l] + m[l + off]; s[l] = s[l] + s[l + off]; }
    *qmu = m[0]; *qsum = s[0];
}

/* The code's IP estimate, team_code_ip (local_search.cu:222-243): lane l of
 * the team adds q over the set bits of words l, l + team, ..., in ascending
 * dimension; the team folds with off = team/2 .. 1; then
 * 1 - (alpha * (2 acc - qsum) + qmu), every operation rounded on its own. */
float so_code_ip(const float* q, const int32_t* code, float alpha, float qmu, float qsum,
                 int dim, int cwords, int team) {
    float acc[64];
    for (int l = 0; l < team; ++l) {
        float a = 0.0f;
        for (int w = l; w < cwords; w += team) {
            const uint32_t bits = (uint32_t)code[w];
            for (int b = 0; b < 32; ++b) {
                const int i = w * 32 + b;
                if (i >= dim) break;
                if (bits & (1u << b)) a = a + q[i];
            }
        }
        acc[l] = a;
    }
    for (int off = team / 2; off > 0; off >>= 1)
        for (int l = 0; l < off; ++l) acc[l] = acc[l] + acc[l + off];
    const float t = 2.0f * acc[0];
    const float u = t - qsum;
    const float v = alpha * u;
    const float w = v + qmu;
    return 1.0f - w;
}

/* One expansion step of one branch, local_search.cu:451-683.  Returns 0 when
 * the branch's loop ends (budget spent, exhausted, or stalled). */
static int so_step(const so_cfg* c, int32_t* ids, float* dist, uint8_t* expd, uint8_t* lin,
                   int32_t* visited, int32_t* ctr, so_locals* lo) {
    const int L = c->L;
    if (ctr[0] >= c->max_exp) return 0;
    const int early = (c->stop_eps >= 0.0f);
    const int kr = (c->kstop < L) ? c->kstop : L;
    float radius = (kr > 0 && ids[kr - 1] >= 0) ? dist[kr - 1] : FLT_MAX;
    if (c->bound) {
        const float gb = c->bound_rd ? *c->bound_rd : *c->bound;
        if (gb < radius) radius = gb;
    }
    const float limit = (radius == FLT_MAX) ? FLT_MAX : radius * (1.0f + c->stop_eps);
    const float rad = limit;               /* the code filter's line, :471-478 */
    int slot = -1;
    if (c->policy == SO_POLICY_RR && c->V > 1) {
        for (int turn = 0; turn < c->V && slot < 0; ++turn) {
            const int want = (ctr[0] + turn) % c->V;
            if (lo->retired[want >> 5] & (1u << (want & 31))) continue;
            int found = -1;
            for (int i = 0; i < L; ++i)
                if (ids[i] >= 0 && expd[i] == 0 && lin[i] == want) { found = i; break; }
            if (found < 0) { lo->retired[want >> 5] |= (1u << (want & 31)); continue; }
            if (early && dist[found] > limit) {
                lo->retired[want >> 5] |= (1u << (want & 31));
                continue;
            }
            slot = found;
        }
        if (slot < 0 && !early) {
            for (int i = 0; i < L; ++i)
                if (ids[i] >= 0 && expd[i] == 0) { slot = i; break; }
        }
    } else {
        for (int i = 0; i < L; ++i) {
            if (ids[i] >= 0 && expd[i] == 0) {
                const unsigned li = lin[i];
                if (lo->retired[li >> 5] & (1u << (li & 31))) continue;
                if (!early || dist[i] <= limit) slot = i;
                break;
            }
        }
    }
    if (slot < 0) { ctr[3] = 1; return 0; }
    expd[slot] = 1;
    const int p = ids[slot];
    const uint8_t plin = lin[slot];
    ctr[0] += 1;

    const int nsort = so_pow2_cap(c->D, SO_MAXD);
    so_ent cand[SO_MAXD];
    for (int i = 0; i < nsort; ++i) { cand[i].id = -1; cand[i].d = FLT_MAX; cand[i].l = 0; cand[i].ord = i; }
    int nbr = 0, cov = 0;
    for (int nidx = 0; nidx < c->D; ++nidx) {
        const int v = c->G[(int64_t)p * c->D + nidx];
        if (v < 0) continue;
        nbr += 1;
        int isnew = 1;
        if (c->H > 1) isnew = so_vis_insert(visited, c->H, v, &ctr[2]);
        if (!isnew) { cov += 1; continue; }
        int cs = -1, claimed = 0;
        float d = FLT_MAX;
        if (c->cbits) {
            /* exclusive claims decide by the row's bit alone: the first
             * branch to set it owns the row, everyone else skips it */
            const uint32_t bit = 1u << (v & 31);
            if (c->cbits[v >> 5] & bit) { ctr[4] += 1; cov += 1; continue; }
            c->cbits[v >> 5] |= bit;
            ctr[5] += 1;
        } else if (c->Hc > 0) {
            cs = so_cache_slot(c->cid, c->Hc, v, &claimed);
            d = (cs >= 0 && !claimed) ? c->cdd[cs] : FLT_MAX;
        }
        if (c->exclusive && cs >= 0 && !claimed && d != FLT_MAX) {
            ctr[4] += 1;                              /* taken by another branch */
        } else if (d == FLT_MAX) {
            int skip = 0;
            if (c->codes) {
                const float est = so_code_ip(c->q, c->codes + (int64_t)v * c->cwords,
                                             c->calpha[v], c->qmu, c->qsum, c->dim, c->cwords,
                                             c->team);
                skip = (rad != FLT_MAX) && (est > rad + c->cmargin);
                if (skip) ctr[3] += 1;         /* the reference counts skips in [3] */
            }
            if (!skip) {
                d = so_team_distance(c->q, c->X, c->dt, v, c->dim, c->metric, c->team);
                if (cs >= 0) { c->cdd[cs] = d; ctr[5] += 1; }
                ctr[1] += 1;
            }
        } else {
            ctr[4] += 1;                              /* cache hit */
        }
        const int taken = c->exclusive && cs >= 0 && !claimed && d != FLT_MAX;
        if (taken) cov += 1;
        else { cand[nidx].id = v; cand[nidx].d = d; cand[nidx].l = plin; }
    }

    /* keep what can still reach the queue, local_search.cu:607-625 */
    const float worst = (ids[L - 1] >= 0) ? dist[L - 1] : FLT_MAX;
    so_ent kept[SO_MAXD];
    int nkeep = 0;
    for (int i = 0; i < nsort; ++i) {
        if (cand[i].id >= 0 && (worst == FLT_MAX || cand[i].d <= worst)) {
            kept[nkeep] = cand[i];
            kept[nkeep].ord = nkeep;
            ++nkeep;
        }
    }
    ctr[8] += nkeep;
    ctr[9] += 1;
    int msort = 2;
    while (msort < nkeep) msort <<= 1;
    if (msort > nsort) msort = nsort;
    for (int i = nkeep; i < msort; ++i) { kept[i].id = -1; kept[i].d = FLT_MAX; kept[i].l = 0; kept[i].ord = i; }
    qsort(kept, (size_t)msort, sizeof(so_ent), so_ent_cmp);

    /* merge-path, local_search.cu:637-650 */
    int32_t nid[SO_MAXL]; float nd[SO_MAXL]; uint8_t ne[SO_MAXL], nl[SO_MAXL];
    for (int o = 0; o < L; ++o) {
        int lo_ = o - msort > 0 ? o - msort : 0;
        int hi = o < L ? o : L;
        while (lo_ < hi) {
            const int i = (lo_ + hi) >> 1, j = o - i;
            if (j > 0 && !so_lt(kept[j - 1].d, kept[j - 1].id, dist[i], ids[i])) lo_ = i + 1;
            else hi = i;
        }
        const int i = lo_, j = o - i;
        const int takeA = (j >= msort) || (i < L && so_lt(dist[i], ids[i], kept[j].d, kept[j].id));
        if (takeA) { nid[o] = ids[i]; nd[o] = dist[i]; ne[o] = expd[i]; nl[o] = lin[i]; }
        else { nid[o] = kept[j].id; nd[o] = kept[j].d; ne[o] = 0; nl[o] = kept[j].l; }
        if (nid[o] < 0) { nd[o] = FLT_MAX; ne[o] = 1; nl[o] = 0; }
    }
    for (int i = 0; i < L; ++i) { ids[i] = nid[i]; dist[i] = nd[i]; expd[i] = ne[i]; lin[i] = nl[i]; }

    if (c->bound && kr > 0 && nid[kr - 1] >= 0) {
        int32_t cur, nv;
        memcpy(&cur, c->bound, 4);
        memcpy(&nv, &nd[kr - 1], 4);
        if (nv < cur) memcpy(c->bound, &nv, 4);   /* integer atomicMin on the bits */
    }
    if (c->crowd_frac > 0.0f) {
        const float cf = (nbr > 0) ? ((float)cov / (float)nbr) : 0.0f;
        if (cf >= c->crowd_frac) {
            if (++lo->crowd_run >= 2) {
                const unsigned li = plin;
                lo->retired[li >> 5] |= (1u << (li & 31));
                ctr[7] += 1;
                lo->crowd_run = 0;
            }
        } else {
            lo->crowd_run = 0;
        }
    }
    if (c->stall_patience > 0) {
        const float bk = (kr > 0 && nid[kr - 1] >= 0) ? nd[kr - 1] : FLT_MAX;
        if (bk < lo->best_k) { lo->best_k = bk; lo->stall = 0; } else { lo->stall += 1; }
        if (lo->stall >= c->stall_patience) { ctr[6] = 1; return 0; }
    }
    return 1;
}

/* Advance one branch by up to `delta` expansions (no shared state). */
void so_advance_branch(const void* X, int dt, int dim, const int32_t* G, int D,
                       const float* q, int32_t* ids, float* dist, uint8_t* expd,
                       uint8_t* lin, int L, int32_t* visited, int H, int32_t* ctr,
                       int metric, int team, int delta, int max_exp, int policy,
                       int V, float stop_eps, int kstop, int stall_patience,
                       float crowd_frac, const int32_t* codes, int cwords, const float* calpha,
                       const float* cmu, float cmargin) {
    so_cfg c;
    memset(&c, 0, sizeof(c));
    if (codes) {
        c.codes = codes; c.cwords = cwords; c.calpha = calpha; c.cmargin = cmargin;
        so_code_sums(q, cmu, dim, &c.qmu, &c.qsum);
    }
    c.X = X; c.dt = dt; c.dim = dim; c.G = G; c.D = D; c.q = q;
    c.L = L; c.H = H; c.metric = metric; c.team = team;
    c.max_exp = max_exp; c.policy = policy; c.V = V;
    c.stop_eps = stop_eps; c.kstop = kstop;
    c.stall_patience = stall_patience; c.crowd_frac = crowd_frac;
    so_locals lo;
    so_locals_reset(&lo);
    for (int s = 0; s < delta; ++s)
        if (!so_step(&c, ids, dist, expd, lin, visited, ctr, &lo)) break;
}

/* ------------------------------------------------------------------ */
/* Per-query merge, local_search.cu:863-919: (d, id) order with invalid
 * ids last, then the first copy of each id, padded with (-1, +inf). */
typedef struct { float d; int id; } so_pair;

static int so_pair_cmp(const void* a, const void* b) {
    const so_pair* x = (const so_pair*)a;
    const so_pair* y = (const so_pair*)b;
    if (so_lt(x->d, x->id, y->d, y->id)) return -1;
    if (so_lt(y->d, y->id, x->d, x->id)) return 1;
    return 0;
}

void so_merge(const int32_t* bids, const float* bdist, int64_t Q, int V, int kk, int k,
              int32_t* out_ids, float* out_dist) {
    const int n = V * kk;
    so_pair* buf = (so_pair*)malloc(sizeof(so_pair) * (size_t)(n > 0 ? n : 1));
    for (int64_t q = 0; q < Q; ++q) {
        for (int i = 0; i < n; ++i) {
            const int id = bids[q * n + i];
            buf[i].id = id >= 0 ? id : INT32_MAX;
            buf[i].d = id >= 0 ? bdist[q * n + i] : INFINITY;
        }
        qsort(buf, (size_t)n, sizeof(so_pair), so_pair_cmp);
        int w = 0;
        for (int i = 0; i < n && w < k; ++i) {
            if (buf[i].id == INT32_MAX) break;
            if (i > 0 && buf[i].id == buf[i - 1].id) continue;
            out_ids[q * k + w] = buf[i].id;
            out_dist[q * k + w] = buf[i].d;
            ++w;
        }
        for (; w < k; ++w) { out_ids[q * k + w] = -1; out_dist[q * k + w] = INFINITY; }
    }
    free(buf);
}

/* ------------------------------------------------------------------ */
/* A whole search of one query with J branches in one legal schedule of the
 * kernel: init every branch, then step the branches in turn (branch 0 step s,
 * branch 1 step s, ...).  Shared cache, bound and claims behave as in
 * local_search.cu with every step atomic.  With the cache, bound and claims
 * off the branches are independent and the result equals J separate branch
 * runs.
 *
 * sched SO_SCHED_SERIAL: each step reads the bound as the steps before it
 * left it.  SO_SCHED_ROUNDS: every step of round s reads the bound as it was
 * when round s began (updates still land at once, claims are still seen at
 * once).  Both are interleavings the kernel allows -- a branch's bound read
 * (local_search.cu:466-469) may come before another branch's lowering
 * (:655-658) and its claims after them.  Rounds is the concurrent launch's
 * shape, where a query's branches start together and a step sees the
 * others' previous steps; serial lets branch 0's first expansion set the
 * bound before any other branch has expanded its seed. */
void so_search_query(const void* X, int dt, int dim, const int32_t* G, int D,
                     const float* q, const int32_t* seeds /* [J][V] */, int J, int V,
                     int L, int B, int H, int metric, int team, int policy,
                     float stop_eps, int kstop, int Hc, int use_bound, int exclusive,
                     int stall_patience, float crowd_frac,
                     int32_t* ids, float* dist, uint8_t* expd, uint8_t* lin,
                     int32_t* visited, int32_t* counters,
                     int32_t* cache_id, float* cache_d, float* bound_out,
                     const int32_t* codes, int cwords, const float* calpha, const float* cmu,
                     float cmargin, int sched) {
    for (int t = 0; t < Hc; ++t) { cache_id[t] = 0; cache_d[t] = FLT_MAX; }
    for (int t = 0; t < (-Hc + 31) / 32; ++t) cache_id[t] = 0;     /* claim bits */
    float bound = FLT_MAX;
    for (int j = 0; j < J; ++j)
        so_init_branch(X, dt, dim, q, seeds + (int64_t)j * V, V, L, H, metric, team,
                       ids + (int64_t)j * L, dist + (int64_t)j * L, expd + (int64_t)j * L,
                       lin + (int64_t)j * L, visited + (int64_t)j * H,
                       counters + (int64_t)j * SO_NCTR);
    so_cfg c;
    memset(&c, 0, sizeof(c));
    c.X = X; c.dt = dt; c.dim = dim; c.G = G; c.D = D; c.q = q;
    c.L = L; c.H = H; c.metric = metric; c.team = team;
    c.max_exp = B; c.policy = policy; c.V = V;
    c.stop_eps = stop_eps; c.kstop = kstop;
    c.cid = Hc > 0 ? cache_id : NULL; c.cdd = Hc > 0 ? cache_d : NULL; c.Hc = Hc > 0 ? Hc : 0;
    c.cbits = Hc < 0 ? (uint32_t*)cache_id : NULL;
    c.bound = use_bound ? &bound : NULL;
    c.exclusive = exclusive;
    c.stall_patience = stall_patience; c.crowd_frac = crowd_frac;
    if (codes) {
        c.codes = codes; c.cwords = cwords; c.calpha = calpha; c.cmargin = cmargin;
        so_code_sums(q, cmu, dim, &c.qmu, &c.qsum);
    }
    so_locals* lo = (so_locals*)malloc(sizeof(so_locals) * (size_t)J);
    for (int j = 0; j < J; ++j) so_locals_reset(&lo[j]);
    float prev = bound;                     /* the bound when the previous round began */
    for (int s = 0; s < B; ++s) {
        int alive = 0;
        const float snap = bound;
        const float lag2 = prev;
        prev = snap;
        c.bound_rd = (sched == SO_SCHED_ROUNDS) ? &snap : (sched == SO_SCHED_ROUNDS2) ? &lag2 : NULL;
        for (int j = 0; j < J; ++j) {
            if (lo[j].done) continue;
            if (!so_step(&c, ids + (int64_t)j * L, dist + (int64_t)j * L,
                         expd + (int64_t)j * L, lin + (int64_t)j * L,
                         visited + (int64_t)j * H, counters + (int64_t)j * SO_NCTR, &lo[j]))
                lo[j].done = 1;
            else
                alive = 1;
        }
        if (!alive) break;
    }
    free(lo);
    if (bound_out) *bound_out = bound;
}

/* Batch of queries through so_search_query + merge, OpenMP over queries.
 * Used as the CPU baseline and for statistical parity; per-thread scratch. */
void so_search_batch(const void* X, int dt, int dim, const int32_t* G, int D,
                     const float* Qv, int64_t nq, const int32_t* seeds, int J, int V,
                     int L, int B, int H, int metric, int team, int policy,
                     float stop_eps, int kstop, int Hc, int use_bound, int exclusive,
                     int k, int32_t* out_ids, float* out_dist, int32_t* out_counters,
                     int nthreads, int sched) {
    const int kk = k < L ? k : L;
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel
#endif
    {
        int32_t* ids = (int32_t*)malloc(sizeof(int32_t) * (size_t)J * L);
        float* dist = (float*)malloc(sizeof(float) * (size_t)J * L);
        uint8_t* expd = (uint8_t*)malloc((size_t)J * L);
        uint8_t* lin = (uint8_t*)malloc((size_t)J * L);
        int32_t* vis = (int32_t*)malloc(sizeof(int32_t) * (size_t)J * H);
        int32_t* ctr = (int32_t*)malloc(sizeof(int32_t) * (size_t)J * SO_NCTR);
        int32_t* cid = (int32_t*)malloc(sizeof(int32_t) *
                                        (size_t)(Hc > 0 ? Hc : Hc < 0 ? (-Hc + 31) / 32 : 1));
        float* cdd = (float*)malloc(sizeof(float) * (size_t)(Hc > 0 ? Hc : 1));
        int32_t* bi = (int32_t*)malloc(sizeof(int32_t) * (size_t)J * kk);
        float* bd = (float*)malloc(sizeof(float) * (size_t)J * kk);
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 1)
#endif
        for (int64_t qi = 0; qi < nq; ++qi) {
            so_search_query(X, dt, dim, G, D, Qv + qi * dim, seeds + qi * (int64_t)J * V, J, V,
                            L, B, H, metric, team, policy, stop_eps, kstop, Hc, use_bound,
                            exclusive, 0, 0.0f, ids, dist, expd, lin, vis, ctr, cid, cdd, NULL,
                            NULL, 0, NULL, NULL, 0.0f, sched);
            for (int j = 0; j < J; ++j)
                for (int t = 0; t < kk; ++t) {
                    bi[j * kk + t] = ids[j * L + t];
                    bd[j * kk + t] = dist[j * L + t];
                }
            so_merge(bi, bd, 1, J, kk, k, out_ids + qi * k, out_dist + qi * k);
            if (out_counters)
                memcpy(out_counters + qi * (int64_t)J * SO_NCTR, ctr,
                       sizeof(int32_t) * (size_t)J * SO_NCTR);
        }
        free(ids); free(dist); free(expd); free(lin); free(vis); free(ctr);
        free(cid); free(cdd); free(bi); free(bd);
    }
}

/* ------------------------------------------------------------------ */
/* Build stages (swann/build.py).  Distances: dot in double, then the
 * reference formula in fp32. */
static double so_dot_d(const float* a, const float* b, int d) {
    double s = 0.0;
    for (int i = 0; i < d; ++i) s += (double)a[i] * (double)b[i];
    return s;
}

/* pairwise formula, build.py:14-25 */
static inline float so_pair_dist(float dot, float na, float nb, int metric) {
    if (metric == SO_METRIC_IP) return 1.0f - dot;
    float v = nb - 2.0f * dot + na;
    return v < 0.0f ? 0.0f : v;
}

typedef struct { float d; int id; } so_di;

/* max-heap on (d, id) for a running top-C */
static inline int so_di_gt(so_di a, so_di b) { return so_lt(b.d, b.id, a.d, a.id); }

static void so_heap_push(so_di* h, int* n, int cap, so_di x) {
    if (*n < cap) {
        int i = (*n)++;
        h[i] = x;
        while (i > 0) {
            int p = (i - 1) / 2;
            if (!so_di_gt(h[i], h[p])) break;
            so_di t = h[i]; h[i] = h[p]; h[p] = t; i = p;
        }
    } else if (so_lt(x.d, x.id, h[0].d, h[0].id)) {
        h[0] = x;
        int i = 0;
        for (;;) {
            int l = 2 * i + 1, r = l + 1, m = i;
            if (l < *n && so_di_gt(h[l], h[m])) m = l;
            if (r < *n && so_di_gt(h[r], h[m])) m = r;
            if (m == i) break;
            so_di t = h[i]; h[i] = h[m]; h[m] = t; i = m;
        }
    }
}

static int so_di_cmp(const void* a, const void* b) {
    const so_di* x = (const so_di*)a;
    const so_di* y = (const so_di*)b;
    if (so_lt(x->d, x->id, y->d, y->id)) return -1;
    if (so_lt(y->d, y->id, x->d, x->id)) return 1;
    return 0;
}

/* Exact top-C per row of X against all rows of Y (rows of X are rows
 * row0.. of Y when self_offset >= 0, and are then excluded with 3.4e38).
 * build.py:28-43 and _select.py:93-128. */
void so_topk_rows(const float* Xr, int64_t nr, const float* Y, int64_t ny, int dim,
                  int metric, int C, int64_t self_offset, int32_t* out_idx, float* out_d,
                  int nthreads) {
    float* yn = (float*)malloc(sizeof(float) * (size_t)ny);
    for (int64_t j = 0; j < ny; ++j) yn[j] = (float)so_dot_d(Y + j * dim, Y + j * dim, dim);
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel
#endif
    {
        so_di* h = (so_di*)malloc(sizeof(so_di) * (size_t)C);
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 16)
#endif
        for (int64_t i = 0; i < nr; ++i) {
            const float* a = Xr + i * dim;
            const float na = (float)so_dot_d(a, a, dim);
            int n = 0;
            for (int64_t j = 0; j < ny; ++j) {
                so_di x;
                x.id = (int)j;
                if (self_offset >= 0 && j == self_offset + i) x.d = 3.4e38f;
                else x.d = so_pair_dist((float)so_dot_d(a, Y + j * dim, dim), na, yn[j], metric);
                so_heap_push(h, &n, C, x);
            }
            qsort(h, (size_t)n, sizeof(so_di), so_di_cmp);
            for (int t = 0; t < C; ++t) {
                out_idx[i * C + t] = t < n ? h[t].id : -1;
                out_d[i * C + t] = t < n ? h[t].d : INFINITY;
            }
        }
        free(h);
    }
    free(yn);
}

/* Sequential alpha rule over one node's ascending candidate list,
 * build.py:46-91.  cand/cd: C entries; at most `cap` kept; a candidate whose
 * `protect` flag is set survives the detour test (build.py:80-81); writes
 * `width` ids (-1 padded). */
static void so_prune_row(const float* X, int dim, int metric, const int32_t* cand,
                         const float* cd, int C, int cap, int width, float alpha,
                         const uint8_t* protect, int32_t* out, float* vn_scratch,
                         int* kept_scratch) {
    int nk = 0;
    for (int i = 0; i < C; ++i) {
        const int ci = cand[i];
        if (nk >= cap) break;
        if (ci < 0) continue;
        int viol = 0;
        if (!(protect && protect[i])) {
            for (int t = 0; t < nk && !viol; ++t) {
                const int w = kept_scratch[t];
                const int cw = cand[w];
                const float dot = (float)so_dot_d(X + (int64_t)cw * dim, X + (int64_t)ci * dim, dim);
                const float pr = so_pair_dist(dot, vn_scratch[w], vn_scratch[i], metric);
                if (alpha * pr <= cd[i]) viol = 1;
            }
        }
        if (!viol) kept_scratch[nk++] = i;
    }
    for (int t = 0; t < width; ++t) out[t] = t < nk ? cand[kept_scratch[t]] : -1;
}

/* deg: the row width (and every node's cap when deg_per_node is NULL);
 * deg_per_node [n] caps node u at min(deg_per_node[u], deg); protect [n, C]
 * (0/1 bytes) or NULL. */
void so_robust_prune(const float* X, int64_t n, int dim, int metric, const int32_t* cand,
                     const float* cdist, int C, int deg, float alpha,
                     const int32_t* deg_per_node, const uint8_t* protect, int32_t* out,
                     int nthreads) {
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel
#endif
    {
        float* vn = (float*)malloc(sizeof(float) * (size_t)C);
        int* kept = (int*)malloc(sizeof(int) * (size_t)C);
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 64)
#endif
        for (int64_t u = 0; u < n; ++u) {
            const int32_t* cr = cand + u * C;
            for (int i = 0; i < C; ++i) {
                const int ci = cr[i] >= 0 ? cr[i] : 0;
                vn[i] = (float)so_dot_d(X + (int64_t)ci * dim, X + (int64_t)ci * dim, dim);
            }
            int cap = deg;
            if (deg_per_node && deg_per_node[u] < cap) cap = deg_per_node[u];
            so_prune_row(X, dim, metric, cr, cdist + u * C, C, cap, deg, alpha,
                         protect ? protect + u * C : NULL, out + u * deg, vn, kept);
        }
        free(vn); free(kept);
    }
}

static int so_i32_cmp(const void* a, const void* b) {
    const int32_t x = *(const int32_t*)a, y = *(const int32_t*)b;
    return (x > y) - (x < y);
}

/* Reverse edges and re-prune, build.py:94-150.  In-edges are kept in
 * ascending source order, at most max_in per target; a row is
 * [G_u | in_u] minus self, deduped, scored exactly (1 - <v,u> or the
 * direct sum of squares), sorted ascending, cut to 128, then pruned. */
void so_add_reverse(const float* X, int64_t n, int dim, int metric, const int32_t* G,
                    int deg, float alpha, int max_in, const int32_t* deg_per_node,
                    int32_t* out, int nthreads) {
    int32_t* cnt = (int32_t*)calloc((size_t)n, sizeof(int32_t));
    int32_t* in = (int32_t*)malloc(sizeof(int32_t) * (size_t)n * max_in);
    for (int64_t i = 0; i < n * max_in; ++i) in[i] = -1;
    for (int64_t u = 0; u < n; ++u)             /* ascending source order */
        for (int t = 0; t < deg; ++t) {
            const int v = G[u * deg + t];
            if (v < 0) continue;
            if (cnt[v] < max_in) in[(int64_t)v * max_in + cnt[v]] = (int32_t)u;
            cnt[v] += 1;
        }
    const int W = deg + max_in;
    const int keepn = W < 128 ? W : 128;
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel
#endif
    {
        int32_t* row = (int32_t*)malloc(sizeof(int32_t) * (size_t)W);
        so_di* sc = (so_di*)malloc(sizeof(so_di) * (size_t)W);
        int32_t* cand = (int32_t*)malloc(sizeof(int32_t) * (size_t)W);
        float* cd = (float*)malloc(sizeof(float) * (size_t)W);
        float* vn = (float*)malloc(sizeof(float) * (size_t)W);
        int* kept = (int*)malloc(sizeof(int) * (size_t)W);
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 64)
#endif
        for (int64_t u = 0; u < n; ++u) {
            int m = 0;
            for (int t = 0; t < deg; ++t) row[m++] = G[u * deg + t];
            for (int t = 0; t < max_in; ++t) row[m++] = in[u * max_in + t];
            for (int t = 0; t < W; ++t)
                if (row[t] == (int32_t)u || row[t] < 0) row[t] = 1 << 30;
            qsort(row, (size_t)W, sizeof(int32_t), so_i32_cmp);
            /* every later copy of an id goes, judged on the sorted values */
            for (int t = W - 1; t > 0; --t)
                if (row[t] == row[t - 1]) row[t] = 1 << 30;
            const float* xu = X + u * dim;
            for (int t = 0; t < W; ++t) {
                const int valid = row[t] < (1 << 30);
                const int id = valid ? row[t] : 0;
                float d;
                if (!valid) d = INFINITY;
                else if (metric == SO_METRIC_IP) d = 1.0f - (float)so_dot_d(X + (int64_t)id * dim, xu, dim);
                else {
                    double s = 0.0;
                    const float* xv = X + (int64_t)id * dim;
                    for (int e = 0; e < dim; ++e) { double df = (double)xv[e] - (double)xu[e]; s += df * df; }
                    d = (float)s;
                }
                sc[t].d = d; sc[t].id = id;
            }
            qsort(sc, (size_t)W, sizeof(so_di), so_di_cmp);
            for (int t = 0; t < keepn; ++t) {
                cand[t] = sc[t].id; cd[t] = sc[t].d;
                vn[t] = (float)so_dot_d(X + (int64_t)cand[t] * dim, X + (int64_t)cand[t] * dim, dim);
            }
            int cap = deg;
            if (deg_per_node && deg_per_node[u] < cap) cap = deg_per_node[u];
            so_prune_row(X, dim, metric, cand, cd, keepn, cap, deg, alpha, NULL, out + u * deg,
                         vn, kept);
        }
        free(row); free(sc); free(cand); free(cd); free(vn); free(kept);
    }
    free(cnt); free(in);
}

/* ------------------------------------------------------------------ */
/* Sign codes for the filter.  The reference ships the consumer
 * (local_search.cu:205-243, _engine.py:320-337) but not the builder; the
 * definition here is the one the consumer's estimator assumes: mu is the
 * corpus mean (double sums, rounded to fp32, unless given), bit b of word w is
 * set when x[32w + b] > mu[32w + b], and alpha = sum |x - mu| / dim (double
 * sum of the fp32 differences, rounded to fp32). */
void so_build_codes(const float* X, int64_t n, int dim, const float* mu_in, int32_t* codes,
                    float* alpha, float* mu_out) {
    const int cwords = (dim + 31) / 32;
    if (mu_in) {
        memcpy(mu_out, mu_in, sizeof(float) * (size_t)dim);
    } else {
        double* acc = (double*)calloc((size_t)dim, sizeof(double));
        for (int64_t r = 0; r < n; ++r)
            for (int t = 0; t < dim; ++t) acc[t] += (double)X[r * dim + t];
        for (int t = 0; t < dim; ++t) mu_out[t] = (float)(acc[t] / (double)n);
        free(acc);
    }
    for (int64_t r = 0; r < n; ++r) {
        double l1 = 0.0;
        for (int w = 0; w < cwords; ++w) {
            uint32_t bits = 0;
            for (int b = 0; b < 32; ++b) {
                const int t = w * 32 + b;
                if (t >= dim) break;
                const float df = X[r * dim + t] - mu_out[t];
                if (df > 0.0f) bits |= (1u << b);
                l1 += (double)fabsf(df);
            }
            codes[r * cwords + w] = (int32_t)bits;
        }
        alpha[r] = (float)(l1 / (double)dim);
    }
}

/* ------------------------------------------------------------------ */
/* The offline builder's extras, offline/build_graph.py. */

typedef struct { float d; int pos; } so_dp;
static int so_dp_cmp(const void* a, const void* b) {
    const so_dp* x = (const so_dp*)a; const so_dp* y = (const so_dp*)b;
    if (x->d < y->d) return -1;
    if (x->d > y->d) return 1;
    return (x->pos > y->pos) - (x->pos < y->pos);
}

/* candidates_from_graph, build_graph.py:63-91: the first C ids of each row
 * of an existing graph Gc [n, gw], exact distances (1 - <a, v>, or the
 * direct sum of squares), -1 entries and self at 3.4e38, ascending
 * (ties in column order). */
void so_candidates_from_graph(const float* X, int64_t n, int dim, int metric,
                              const int32_t* Gc, int gw, int C, int32_t* out_idx,
                              float* out_d, int nthreads) {
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel
#endif
    {
        so_dp* row = (so_dp*)malloc(sizeof(so_dp) * (size_t)C);
#ifdef _OPENMP
#pragma omp for schedule(static)
#endif
        for (int64_t u = 0; u < n; ++u) {
            const float* a = X + u * dim;
            for (int j = 0; j < C; ++j) {
                const int v = Gc[u * gw + j];
                float d;
                if (v < 0 || v == u) d = 3.4e38f;
                else if (metric == SO_METRIC_IP) d = 1.0f - (float)so_dot_d(a, X + (int64_t)v * dim, dim);
                else {
                    double s = 0.0;
                    for (int e = 0; e < dim; ++e) { const double df = (double)a[e] - (double)X[(int64_t)v * dim + e]; s += df * df; }
                    d = (float)s;
                }
                row[j].d = d; row[j].pos = j;
            }
            qsort(row, (size_t)C, sizeof(so_dp), so_dp_cmp);
            for (int j = 0; j < C; ++j) {
                out_idx[u * C + j] = Gc[u * gw + row[j].pos];
                out_d[u * C + j] = row[j].d;
            }
        }
        free(row);
    }
}

/* mutual_rank, build_graph.py:93-131: out[u, j] = 1 when j < M, cand[u, j]
 * = v >= 0 and u is among cand[v, :M]. */
void so_mutual_rank(const int32_t* cand, int64_t n, int C, int M, uint8_t* out) {
    if (M > C) M = C;
    for (int64_t u = 0; u < n; ++u)
        for (int j = 0; j < C; ++j) {
            uint8_t m = 0;
            const int v = cand[u * C + j];
            if (j < M && v >= 0)
                for (int t = 0; t < M; ++t)
                    if (cand[(int64_t)v * C + t] == (int32_t)u) { m = 1; break; }
            out[u * C + j] = m;
        }
}

static int so_contains(const int32_t* a, int len, int32_t x) {
    for (int i = 0; i < len; ++i) if (a[i] == x) return 1;
    return 0;
}

/* fill_degree, build_graph.py:132-200.  rule 0 near, 1 far, 2 bridge.
 * Chunks of `chunk` nodes in order; a chunk reads the graph as the earlier
 * chunks left it.  Per node: a candidate is free unless it is already an
 * out-neighbour, the node itself or -1 (bridge: or two hops away through the
 * kept neighbours); free candidates go, nearest first (far: farthest first),
 * into the empty slots in ascending position. */
void so_fill_degree(const int32_t* G, int64_t n, int W, const int32_t* cand, int C, int rule,
                    int chunk, int32_t* out) {
    memcpy(out, G, sizeof(int32_t) * (size_t)n * W);
    int32_t* next = (int32_t*)malloc(sizeof(int32_t) * (size_t)chunk * W);
    int32_t* two = (int32_t*)malloc(sizeof(int32_t) * (size_t)W * W);
    int* pick = (int*)malloc(sizeof(int) * (size_t)C);
    int* empty = (int*)malloc(sizeof(int) * (size_t)W);
    for (int64_t s = 0; s < n; s += chunk) {
        const int64_t e = s + chunk < n ? s + chunk : n;
        for (int64_t u = s; u < e; ++u) {
            const int32_t* kept = out + u * W;
            int32_t* nr = next + (u - s) * W;
            memcpy(nr, kept, sizeof(int32_t) * (size_t)W);
            if (rule == 2)
                for (int k = 0; k < W; ++k)
                    for (int t = 0; t < W; ++t)
                        two[k * W + t] = kept[k] >= 0 ? out[(int64_t)kept[k] * W + t] : -1;
            int nfree = 0;
            for (int j = 0; j < C; ++j) {
                const int32_t c = cand[u * C + j];
                int taken = (c < 0) || (c == (int32_t)u) || so_contains(kept, W, c);
                if (!taken && rule == 2 && so_contains(two, W * W, c)) taken = 1;
                if (!taken) pick[nfree++] = j;
            }
            int nempty = 0;
            for (int k = 0; k < W; ++k) if (kept[k] < 0) empty[nempty++] = k;
            const int take = nfree < nempty ? nfree : nempty;
            for (int t = 0; t < take; ++t) {
                const int j = rule == 1 ? pick[nfree - 1 - t] : pick[t];
                nr[empty[t]] = cand[u * C + j];
            }
        }
        memcpy(out + s * W, next, sizeof(int32_t) * (size_t)(e - s) * W);
    }
    free(next); free(two); free(pick); free(empty);
}

/* enforce_min_in, build_graph.py:203-294, in place on G [n, W].  Each round
 * recounts in-degrees; every node short of min_in is offered, column by
 * column of its candidate list, to that candidate, which takes it in place of
 * its farthest out-edge whose head stays above the floor (never its first
 * slot).  One offer per target per column (the lowest offering node); an
 * edge already present is skipped.  In-degree updates follow the reference's
 * indexed assignment: a node that loses several edges in one column is
 * decremented once.  Returns the number of rounds run. */
int so_enforce_min_in(int32_t* G, int64_t n, int W, const int32_t* cand, int C, int min_in,
                      int rounds) {
    int32_t* indeg = (int32_t*)malloc(sizeof(int32_t) * (size_t)n);
    int32_t* remaining = (int32_t*)malloc(sizeof(int32_t) * (size_t)n);
    int32_t* winner = (int32_t*)malloc(sizeof(int32_t) * (size_t)n);
    uint8_t* vflag = (uint8_t*)malloc((size_t)n);
    int r;
    for (r = 0; r < rounds; ++r) {
        memset(indeg, 0, sizeof(int32_t) * (size_t)n);
        for (int64_t i = 0; i < n * W; ++i) if (G[i] >= 0) indeg[G[i]] += 1;
        int64_t nweak = 0;
        for (int64_t u = 0; u < n; ++u) {
            remaining[u] = 0;
            if (indeg[u] < min_in) {
                int need = min_in - indeg[u];
                remaining[u] = need < C ? need : C;
                ++nweak;
            }
        }
        if (nweak == 0) break;
        for (int i = 0; i < C; ++i) {
            int any = 0;
            for (int64_t u = 0; u < n; ++u) winner[u] = -1;
            for (int64_t s = 0; s < n; ++s) {
                if (remaining[s] <= 0) continue;
                any = 1;
                const int32_t t = cand[s * C + i];
                if (t < 0 || t == (int32_t)s) continue;
                if (so_contains(G + (int64_t)t * W, W, (int32_t)s)) continue;
                if (winner[t] < 0) winner[t] = (int32_t)s;     /* lowest s per target */
            }
            if (!any) break;
            memset(vflag, 0, (size_t)n);
            /* decide every slot against the column's starting in-degrees */
            for (int64_t t = 0; t < n; ++t) {
                const int32_t s = winner[t];
                if (s < 0) continue;
                int slot = -1;
                for (int k = 0; k < W; ++k) {
                    const int32_t h = G[t * W + k];
                    if (h >= 0 && indeg[h] > min_in) slot = k;
                }
                if (slot < 1) { winner[t] = -1; continue; }
                vflag[G[t * W + slot]] = 1;
                G[t * W + slot] = -2 - slot;        /* placeholder until the counts move */
            }
            for (int64_t v = 0; v < n; ++v) if (vflag[v]) indeg[v] -= 1;
            for (int64_t t = 0; t < n; ++t) {
                const int32_t s = winner[t];
                if (s < 0) continue;
                for (int k = 0; k < W; ++k)
                    if (G[t * W + k] <= -2) { G[t * W + k] = s; break; }
                indeg[s] += 1;
                remaining[s] -= 1;
            }
        }
    }
    free(indeg); free(remaining); free(winner); free(vflag);
    return r;
}
