/*
 * swann_amd.h -- C ABI of the MI355X (gfx950) library behind swann_amd.
 *
 * Every entry point takes raw device pointers, sizes and a HIP stream passed
 * as `void*` (0 = the null stream); nothing here names a torch or HIP type.
 * Calls are asynchronous on that stream.  All return 0 on success or a
 * negative SWANN_E_* code; swann_last_error() then holds a message for the
 * calling thread.  No entry point on the search path allocates device memory:
 * state and workspaces are owned by the caller, so a search can be captured
 * in a hipGraph.
 *
 * Reference interfaces replaced (paths relative to the reference checkout):
 *   swann_init_states      swann/csrc/local_search.cu:741-776  (pybind init_states)
 *   swann_advance          swann/csrc/local_search.cu:778-841  (pybind advance)
 *   swann_merge_branches   swann/csrc/local_search.cu:925-947  (pybind merge_branches)
 *   swann_merge_branches_strided  swann/_engine.py:340-374  (branch_topk, then merge_branches)
 *   swann_select_nearest   swann/_select.py:93-128             (select_nearest)
 *   swann_build_sweep      swann/build.py:28-43                (knn_candidates)
 *   swann_build_prune      swann/build.py:46-91                (robust_prune)
 *   swann_build_reverse    swann/build.py:94-150               (add_reverse)
 *   swann_overflow_async   swann/_engine.py:155-173            (SearchState.check / overflow)
 *   swann_validate_*       the TORCH_CHECKs of local_search.cu:726-841, host only
 */
#ifndef SWANN_AMD_H
#define SWANN_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* error codes */
#define SWANN_OK 0
#define SWANN_E_INVALID (-1)   /* an argument failed validation */
#define SWANN_E_LAUNCH (-2)    /* the HIP runtime refused a launch */
#define SWANN_E_UNSUPPORTED (-3)
#define SWANN_E_NODEVICE (-4)

/* constants shared with the Python layer (local_search.cu:32-42, _engine.py:31-37) */
#define SWANN_METRIC_IP 0      /* distance = 1 - <q, x>; rows L2-normalised */
#define SWANN_METRIC_L2 1      /* distance = ||q - x||^2 */
#define SWANN_POLICY_BEST 0
#define SWANN_POLICY_ROUND_ROBIN 1
#define SWANN_DTYPE_F32 0
#define SWANN_DTYPE_F16 1
#define SWANN_NCTR 10          /* counters per branch, layout of local_search.cu:35-41 */
#define SWANN_MAXL 512         /* queue width limit */
#define SWANN_MAXD 128         /* graph out-degree limit */
#define SWANN_MAXV 128         /* seeds per branch (init sort buffer) */

/* The message of the last failed call on this thread ("" if none). */
const char* swann_last_error(void);

/* Library version string and the gfx target it was built for. */
const char* swann_version(void);

/* Number of HIP devices visible (0 on a machine without a GPU). */
int swann_device_count(void);

/* Options: switches that select an alternative code path of the same
 * computation, for tests that run every path on the same inputs and for
 * diagnosis.  No counterpart in the reference (its extension has one path
 * per operation).  Process-wide, read at each call, defaults = the
 * production path; the library reads no environment variable.
 *   search_block      0 | 64 | 256 | 1024   advance workgroup size (0: chosen per batch)
 *   prune_simt        0 | 1   prune Gram on fp32 SIMT instead of MFMA
 *   prune_f32         0 | 1   fp32 rows' prune Gram on fp32 MFMA, not split fp16 planes
 *   sweep_sym        -1 | 0 | 1   symmetric sweep by size, never, always (>= 2 panels)
 *   sweep_waves       16 | 8  waves of a direct-load sweep workgroup
 *   sweep_rowscale    0 | 1   fp32 corpus screened on a row-scaled plane always
 *   sweep_regstage    0 | 1   register-staged sweep instead of direct loads
 *   sweep_sym_fcap    0 | k   room of a symmetric sweep row's second list (k < cap
 *                             forces its overflow and the recovery paths)
 *   sweep_noseed      0 | 1   symmetric sweep without the locality order and seeds
 *   sweep_order       1 | 0   seeded sweep on the locality-ordered copy, or in row order
 *   sweep_repair_max  4 | k   overflowed row panels up to which each is repaired
 *                             alone (sixteen ways); more go at once (two ways)
 * Set an option between calls, not while a call that reads it runs on
 * another thread.  Unknown names and out-of-range values: SWANN_E_INVALID. */
int swann_set_option(const char* name, int value);
int swann_get_option(const char* name, int* value);
int swann_reset_options(void);

/* ---- search state ------------------------------------------------------
 * Layout (all row-major, contiguous):
 *   X        [n, dim]  fp32 or fp16 (x_dtype)     corpus
 *   Qv       [Q, dim]  fp32                       queries
 *   seeds    [Q, J, V] int32, -1 = empty
 *   G        [n, D]    int32, -1 = no edge
 *   ids      [Q, J, L] int32, dist [Q, J, L] fp32, expd/lin [Q, J, L] uint8
 *   visited  [Q, J, H] int32 (H a power of two; H == 1 disables it)
 *   counters [Q, J, SWANN_NCTR] int32
 *   cache_id [Q, Hc] int32, cache_d [Q, Hc] fp32 (Hc a power of two; 0 = off);
 *            or one [Q, Hc, 2] allocation of (id, d) pairs, passed as
 *            cache_id = its start and cache_d = cache_id + 1 word (the
 *            kernels detect that adjacency and stride by 2; a claim and the
 *            distance stored into it then share a cache line, and a slot is
 *            probed as one 64-bit word, so the pairs must start 8-byte
 *            aligned -- SWANN_E_INVALID otherwise);
 *            or claim bits: cache_id [Q, Hc / 32] int32 with cache_d = NULL,
 *            one bit per corpus row (Hc a power of two >= n and >= 32).
 *            For exclusive claims without sign codes only: a row whose bit
 *            another branch set is skipped, as the table skips a row it
 *            finds claimed; no distance is cached.  This layout has no
 *            counterpart in the reference's table; it decides claims as
 *            that table does when no probe chain runs out.
 *   bound    [Q] fp32 or NULL
 * A disabled feature is a NULL pointer (and Hc = 0), matching the
 * reference's empty-tensor convention (swann/_engine.py:269-274).
 */

/* Host-only validation of init_states arguments (no GPU needed). */
int swann_validate_init(int64_t n, int dim, int x_dtype, int64_t Q, int J, int V, int L,
                        int H, int metric, int team_size, int Hc);

/* Host-only validation of advance arguments (no GPU needed).  `cwords` is the
 * sign codes' words per row, 0 when the filter is off. */
int swann_validate_advance(int64_t n, int dim, int x_dtype, int D, int64_t Q, int J, int L,
                           int H, int metric, int team_size, int policy, int V, int Hc,
                           int64_t nactive, int cwords);

/* Seed every branch, clear the per-query table and bound (init_kernel,
 * local_search.cu:271-351). */
int swann_init_states(const void* X, int x_dtype, int64_t n, int dim,
                      const float* Qv, int64_t Q, const int32_t* seeds, int J, int V,
                      int32_t* ids, float* dist, uint8_t* expd, uint8_t* lin, int L,
                      int32_t* visited, int H, int32_t* counters,
                      int metric, int team_size,
                      int32_t* cache_id, float* cache_d, int Hc, float* bound,
                      void* stream);

/* Up to `delta` best-first expansions per branch, in place (advance_kernel,
 * local_search.cu:353-688).  `active` (nactive entries of flattened q*J+j)
 * restricts the grid to those branches; NULL = all Q*J.
 *
 * Sign-code pre-filter (local_search.cu:205-243, :560-575; metric ip only):
 * codes [n, cwords] int32 (bit b of word w: dimension 32w + b above the
 * mean), alpha [n] fp32, cmu [dim] fp32; NULL codes = off.  A neighbour that
 * would be scored is first estimated from its code and skipped when the
 * estimate exceeds the step's stop line by more than code_margin; a skip adds
 * 1 to counters[3] (which also holds the exhausted flag, as in the
 * reference), leaves the neighbour a candidate at FLT_MAX and its row
 * unread. */
int swann_advance(const void* X, int x_dtype, int64_t n, int dim,
                  const int32_t* G, int D, const float* Qv, int64_t Q, int J,
                  int32_t* ids, float* dist, uint8_t* expd, uint8_t* lin, int L,
                  int32_t* visited, int H, int32_t* counters,
                  int metric, int team_size, int delta, int max_expansions,
                  int policy, int V, float stop_eps, int kstop,
                  int32_t* cache_id, float* cache_d, int Hc, float* bound, int exclusive,
                  int stall_patience, float crowd_frac,
                  const int32_t* active, int64_t nactive,
                  const int32_t* codes, int cwords, const float* alpha, const float* cmu,
                  float code_margin, void* stream);

/* Sign codes for the pre-filter (no counterpart in the reference, which
 * ships only their consumer and loader, swann/_engine.py:320-337): mu = the
 * column means (or mu_in when given), bit set where x > mu, alpha = mean
 * |x - mu| per row.  codes [n, ceil(dim/32)] int32, alpha [n], mu_out [dim].
 * `workspace`: swann_codes_workspace_size bytes (unused when mu_in is given). */
int64_t swann_codes_workspace_size(int64_t n, int dim);
int swann_build_codes(const void* X, int x_dtype, int64_t n, int dim, const float* mu_in,
                      int32_t* codes, float* alpha, float* mu_out, void* workspace,
                      void* stream);

/* ---- the offline builder's extras (offline/build_graph.py) --------------- */

/* candidates_from_graph (build_graph.py:63-91): the first C entries of each
 * row of an existing graph Gc [n, gw] with exact distances (1 - <a,v>, or the
 * direct sum of squares), -1 entries and self at 3.4e38, ascending by
 * (distance, column).  C <= min(gw, 256). */
int swann_candidates_from_graph(const void* X, int x_dtype, int64_t n, int dim, int metric,
                                const int32_t* Gc, int gw, int C, int32_t* out_idx,
                                float* out_dist, void* stream);

/* mutual_rank (build_graph.py:93-131): out [n, C] bytes, 1 where j < M and
 * u = cand[u, j]'s node is among cand[cand[u, j], :M]. */
int swann_mutual_rank(const int32_t* cand, int64_t n, int C, int M, uint8_t* out, void* stream);

/* fill_degree (build_graph.py:132-200): G [n, W] -> out [n, W] (may equal G);
 * rule 0 near, 1 far, 2 bridge; chunks of `chunk` nodes in order, each
 * reading the graph as the earlier chunks left it.  W <= 128, C <= 256.
 * `workspace`: swann_fill_workspace_size bytes. */
int64_t swann_fill_workspace_size(int64_t n, int W, int chunk);
int swann_fill_degree(const int32_t* G, int64_t n, int W, const int32_t* cand, int C, int rule,
                      int chunk, int32_t* out, void* workspace, void* stream);

/* enforce_min_in (build_graph.py:203-294), in place on G [n, W]: `rounds`
 * rounds of offering every node below min_in in-edges to its candidates,
 * column by column; a target takes the lowest offering node in place of its
 * farthest edge whose head stays above the floor (never slot 0).  (The
 * reference picks among several offers to one target by an unstable sort.)
 * `workspace`: swann_min_in_workspace_size bytes. */
int64_t swann_min_in_workspace_size(int64_t n);
int swann_enforce_min_in(int32_t* G, int64_t n, int W, const int32_t* cand, int C, int min_in,
                         int rounds, void* workspace, void* stream);

/* Per-query dedup top-k of branch results (merge_branches_kernel,
 * local_search.cu:863-919).  bids/bdist [Q, V, kk] -> out [Q, k], 1 <= k <=
 * V*kk: entries in (distance, id) order, invalid ids (< 0) last, an entry
 * dropped when its id equals its predecessor's in that order; missing entries
 * are (-1, +inf).  Any V*kk (no shared-memory limit). */
int swann_merge_branches(const int32_t* bids, const float* bdist, int64_t Q, int V, int kk,
                         int k, int32_t* out_ids, float* out_dist, void* stream);

/* swann_merge_branches over the first kk slots of rows of ld >= kk slots:
 * bids/bdist [Q, V, ld], e.g. a search state's sorted queues, read in place
 * of the [Q, V, kk] copy that branch_topk makes (_engine.py:340-355).  Same
 * output; ld == kk is swann_merge_branches itself. */
int swann_merge_branches_strided(const int32_t* bids, const float* bdist, int64_t Q, int V,
                                 int kk, int64_t ld, int k, int32_t* out_ids, float* out_dist,
                                 void* stream);

/* Sum of counters[..., 2] (visited-table overflows) over nbranch branches,
 * written to *out (device or host-pinned memory) without a host sync. */
int swann_overflow_async(const int32_t* counters, int64_t nbranch, int32_t* out, void* stream);

/* ---- seed selection ----------------------------------------------------
 * The E nearest catalogue rows per query (_select.py:93-128), ascending by
 * distance, as int32 row indices into Vp.  Q [nq, dim] fp32, Vp [P, dim] fp32.
 * Distances: 1 - <q, v> (IP) or ||v||^2 - 2<q, v> + ||q||^2 (L2).
 * `workspace` must hold swann_select_workspace_size(nq, P) bytes. */
int64_t swann_select_workspace_size(int64_t nq, int64_t P);
int swann_select_nearest(const float* Q, int64_t nq, int dim, const float* Vp, int64_t P,
                         int E, int metric, int32_t* out_idx, float* out_dist,
                         void* workspace, void* stream);

/* swann_select_nearest without a workspace argument and without allocating:
 * no counterpart in the reference.  It is for callers that cannot allocate
 * device memory -- code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc.  Its workspace is the library's own
 * fixed array of SWANN_SELECT_SCRATCH_BYTES per GPU, a file-scope __device__
 * array of the selection code: it is reserved on a GPU when that code object
 * first loads there -- any swann_select_nearest call does it, so every
 * Index.search user holds it, not only callers of this entry point -- and
 * held until the process ends; a call whose
 * swann_select_workspace_size(nq, P) exceeds that is refused with
 * SWANN_E_INVALID (32 MiB: e.g. 2,000 queries against a 4,096-row
 * catalogue).  Every call on one GPU shares that GPU's array, so calls that
 * overlap on one GPU (concurrent streams or threads) race; calls ordered on
 * one stream do not.  Results equal swann_select_nearest's. */
#define SWANN_SELECT_SCRATCH_BYTES ((int64_t)32 << 20)
int swann_select_nearest_noalloc(const float* Q, int64_t nq, int dim, const float* Vp, int64_t P,
                                 int E, int metric, int32_t* out_idx, float* out_dist,
                                 void* stream);

/* ---- graph build -------------------------------------------------------
 * X [n, dim] is fp32 or fp16 (x_dtype); an fp16 corpus is read as fp16 and
 * upcast exactly, which equals the reference's X.float() (build.py:167).
 *
 * Sweep (build.py:28-43): exact top-C neighbours of every row, self
 * excluded (3.4e38), ascending, as (cand [n, C] int32, cdist [n, C] fp32) with
 * IP: 1 - <a,b>; L2: max(0, |b|^2 - 2<a,b> + |a|^2).  When dim % 8 == 0 the
 * scores come from fp16 MFMA tiles (fp16 corpus: exact products; fp32 corpus:
 * a power-of-two row-scaled fp16 screen keeps C+32 per row, which are then
 * re-ranked with exact fp32 dot products); otherwise from fp32 SIMT tiles.
 * `workspace`: swann_sweep_workspace_size bytes. */
int64_t swann_sweep_workspace_size(int64_t n, int dim, int x_dtype, int C);
int swann_build_sweep(const void* X, int x_dtype, int64_t n, int dim, int metric, int C,
                      int32_t* cand, float* cdist, void* workspace, void* stream);

/* Tiles of 256 x 256 rows the last swann_build_sweep on this thread scored
 * on MFMA (the symmetric sweep's bands, less the tiles the locality-ordered
 * sweep proved empty, plus any repair); -1 before any sweep.  No counterpart
 * in the reference (its sweep scores every pair): a diagnostic for the
 * executed-FLOP figure of the bench (2 * 256 * 256 * dim FLOP a tile). */
int64_t swann_sweep_tiles_scored(void);

/* Row panels of 256 rows the last swann_build_sweep on this thread handled as
 * dense: panels of the locality-ordered sweep whose rows lie near too many
 * other panels to prune, whose tiles the other panels' workgroups score after
 * the bands and whose rows are then repaired one-sided; 0 when none was, -1
 * before any sweep.  No counterpart in the reference: a diagnostic for tests
 * and tuning. */
int64_t swann_sweep_dense_panels(void);

/* Prune (build.py:46-91): keep candidate i of node u unless an already kept
 * w satisfies alpha * d(w, i) <= d(u, i); rows of `deg` ids, -1 padded.
 * C <= 128, deg <= 128.  deg_per_node [n] (or NULL) caps node u at
 * min(deg_per_node[u], deg) kept; protect [n, C] bytes (or NULL): a nonzero
 * entry exempts that candidate from the detour test (build.py:78-81).
 * `workspace`: swann_prune_workspace_size bytes, or NULL.  With it the nodes
 * run grouped by shared candidates (the same result in any order), and an
 * fp32 corpus whose dim is a multiple of 8 takes the pair Gram from split
 * fp16 planes (a row scale each: hi and lo halves, three fp16 MFMAs per 16 of
 * K); without it, nodes in order and the Gram from fp32 MFMAs (the same rows
 * up to near-ties). */
int64_t swann_prune_workspace_size(int64_t n, int dim, int x_dtype);
int swann_build_prune(const void* X, int x_dtype, int64_t n, int dim, int metric,
                      const int32_t* cand, const float* cdist, int C, int deg, float alpha,
                      const int32_t* deg_per_node, const uint8_t* protect, int32_t* out,
                      void* workspace, void* stream);

/* Reverse (build.py:94-150): offer every edge u->v back to v (ascending
 * source, at most max_in per target), dedup [G_u | in_u] minus self, score
 * exactly, keep the nearest 128 and prune to deg (G and out have deg
 * columns; deg_per_node caps the prune per node as in swann_build_prune).
 * `workspace`: swann_reverse_workspace_size bytes. */
int64_t swann_reverse_workspace_size(int64_t n, int deg, int max_in);
int swann_build_reverse(const void* X, int x_dtype, int64_t n, int dim, int metric,
                        const int32_t* G, int deg, float alpha, int max_in,
                        const int32_t* deg_per_node, int32_t* out, void* workspace,
                        void* stream);

/* The MFMA rate the chip sustains (measurement; no counterpart in the
 * reference): `blocks` workgroups of four waves each run `iters` rounds of four
 * independent v_mfma_f32_32x32x16_f16 on register operands.  The caller times
 * the launch; swann_mfma_probe_flop gives its FLOP.  `sink` is one float the
 * kernel may write. */
int64_t swann_mfma_probe_flop(int iters, int blocks);
int swann_mfma_probe(int iters, int blocks, float* sink, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* SWANN_AMD_H */
