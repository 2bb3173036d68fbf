"""Headline benchmark: QPS at recall@10 = 0.95 on one MI355X, with the search
kernel's achieved HBM bandwidth, and the graph build's seconds per 1M rows.

Default workload: n = 1,000,000 x d = 1536 fp16 corpus,
low-rank (rank 256) Gaussian plus 0.1 isotropic noise, rows L2-normalised,
metric ip; 10,000 fp32 queries from the same generator; graph D = 64 built by
this library (sweep C = 128, alpha = 1.2); k = 10, branches = 32, team = 16,
queue = 12, budget = 64; stop_eps swept over {0.02, 0.05, 0.1, 0.2} and the
fastest setting reaching recall@10 >= 0.95 against exact fp32 ground truth is
the one timed.

A step is one search of the whole 10,000-query batch: seed selection, branch
init, advance, merge, with the corpus, graph and queries resident in HBM.
W untimed steps, then K timed steps between device synchronisations.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--n N] [--config c3]

Prints one JSON line (last line of stdout).
"""
from __future__ import annotations

import argparse
import json
from types import SimpleNamespace
import os
import sys
import time
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

CONFIGS = {
    # name: (n, d, dtype, metric, gen, rank, seed, nq, D, cand, branches, team)
    "c1": dict(n=10_000, d=128, dtype="f32", metric="ip", gen="gauss", rank=0, seed=0,
               nq=200, D=32, cand=64, branches=8, team=16),
    "c2": dict(n=1_000_000, d=960, dtype="f32", metric="l2", gen="gmm", rank=0, seed=2,
               nq=10_000, D=64, cand=128, branches=32, team=16),
    "c3": dict(n=1_000_000, d=1536, dtype="f16", metric="ip", gen="lowrank", rank=256, seed=3,
               nq=10_000, D=64, cand=128, branches=32, team=16),
    "c5": dict(n=1_000_000, d=1024, dtype="f32", metric="l2", gen="gmm", rank=0, seed=5,
               nq=10_000, D=64, cand=128, branches=32, team=16),
    # small-batch latency; --config c4 prints its own line (see run_c4)
    "c4": dict(n=500_000, d=4096, dtype="f16", metric="ip", gen="lowrank", rank=512, seed=4,
               nq=2048, D=64, cand=128, branches=32, team=32),
}
C4_BRANCHES = (32, 128)
C4_BATCHES = (1, 8, 64, 512)
EPS_SWEEP = (0.02, 0.05, 0.1, 0.2)
# If no stop_eps reaches the target at the configured knobs, the search effort
# is raised along this ladder (branches, queue, budget, stop_eps), cheapest first.
LADDER = ((64, 32, 64, 0.3), (64, 44, 64, 0.3), (64, 48, 64, 0.2), (96, 32, 64, 0.3), (64, 48, 128, 0.3),
          (128, 24, 128, 0.2), (128, 32, 64, 0.3), (64, 64, 128, 0.3), (128, 48, 128, 0.3))
TARGET_RECALL = 0.95
HBM_PEAK = 8.0e12
MFMA_F16_PEAK = 2.5e15              # dense fp16/bf16 MFMA, MI355X
# HBM bytes per advance launch measured by rocprofv3 --pmc (FETCH_SIZE x 2.000 +
# WRITE_SIZE x 1.000, the factors a 2 GiB device copy reads; see
# profiles/advance_kernel_c3_hbm_traffic.md).  Valid only for the kernel source it
# was measured on (kernel_source_key of swann_amd/csrc/search.hip: SHA-256 prefix of
# the source without comments), the same workload and knobs and the same per-query
# claims layout (Index._claims: "bits<n>" or the table's slots); otherwise `traffic`
# is reported as null.
PMC_TRAFFIC = {
    ("c3", 1_000_000, 10_000, 64, 44, 64, 0.3, "bits1048576", "86f5d362e82538e5"): 4.860e12,
}


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def generate(cfg, n, nq, dev):
    """Synthetic corpus and queries on the GPU (fp32 originals)."""
    d, seed = cfg["d"], cfg["seed"]
    g = torch.Generator(device=dev)
    if cfg["gen"] == "lowrank":
        r = cfg["rank"]
        g.manual_seed(seed * 1000 + 7)
        W = torch.randn((r, d), generator=g, device=dev)

        def draw(m, s):
            g.manual_seed(s)
            out = torch.empty((m, d), device=dev)
            for a in range(0, m, 131072):
                b = min(m, a + 131072)
                Z = torch.randn((b - a, r), generator=g, device=dev)
                x = Z @ W / r ** 0.5 + 0.1 * torch.randn((b - a, d), generator=g, device=dev)
                out[a:b] = x / x.norm(dim=1, keepdim=True)
            return out
        return draw(n, seed), draw(nq, seed + 1)
    if cfg["gen"] == "gmm":
        g.manual_seed(seed * 1000 + 7)
        centres = torch.randn((1000, d), generator=g, device=dev)

        def draw(m, s):
            g.manual_seed(s)
            lab = torch.randint(0, 1000, (m,), generator=g, device=dev)
            return centres[lab] + 0.3 * torch.randn((m, d), generator=g, device=dev)
        return draw(n, seed), draw(nq, seed + 1)
    g.manual_seed(seed)
    X = torch.randn((n, d), generator=g, device=dev)
    g.manual_seed(seed + 1)
    Q = torch.randn((nq, d), generator=g, device=dev)
    if cfg["metric"] == "ip":
        X = X / X.norm(dim=1, keepdim=True)
        Q = Q / Q.norm(dim=1, keepdim=True)
    return X, Q


def ground_truth(X32, Q, k, metric):
    """Exact fp32 brute force on the fp32 originals (measurement plumbing)."""
    out = torch.empty((Q.shape[0], k), dtype=torch.int64, device=Q.device)
    xn = (X32 * X32).sum(1) if metric == "l2" else None
    for a in range(0, Q.shape[0], 1024):
        q = Q[a:a + 1024]
        best_d = None
        best_i = None
        for c in range(0, X32.shape[0], 262144):
            s = q @ X32[c:c + 262144].T
            d = -s if metric == "ip" else xn[c:c + 262144][None, :] - 2 * s
            v, i = torch.topk(d, k, dim=1, largest=False)
            i = i + c
            if best_d is None:
                best_d, best_i = v, i
            else:
                dd = torch.cat([best_d, v], 1); ii = torch.cat([best_i, i], 1)
                best_d, j = torch.topk(dd, k, dim=1, largest=False)
                best_i = torch.gather(ii, 1, j)
        out[a:a + 1024] = best_i
    return out


def kernel_source_key(path):
    """SHA-256 prefix of a kernel source with its // comments and blank lines
    removed, so that a measured figure stays attached to the code it was
    measured on through comment edits."""
    import hashlib
    import re
    lines = []
    for line in Path(path).read_text().splitlines():
        line = re.sub(r"//.*$", "", line).rstrip()
        if line:
            lines.append(line)
    return hashlib.sha256("\n".join(lines).encode()).hexdigest()[:16]


def timed_build(X, cfg):
    """Index.build's three stages (swann/build.py:153-171) with a sync after
    each: (graph, total seconds, per-stage seconds)."""
    from swann_amd import build as B
    Xg = B._rows(X)
    t = [time.perf_counter()]
    cand, cdist = B.knn_candidates(Xg, cfg["cand"], metric=cfg["metric"])
    torch.cuda.synchronize()
    t.append(time.perf_counter())
    tiles = int(_lib_tiles())
    G = B.robust_prune(Xg, cand, cdist, cfg["D"], alpha=1.2, metric=cfg["metric"])
    torch.cuda.synchronize()
    t.append(time.perf_counter())
    G = B.add_reverse(Xg, G, cfg["D"], alpha=1.2, metric=cfg["metric"]).to(torch.int32).contiguous()
    torch.cuda.synchronize()
    t.append(time.perf_counter())
    del cand, cdist
    stages = dict(candidates=round(t[1] - t[0], 3), prune=round(t[2] - t[1], 3),
                  reverse=round(t[3] - t[2], 3), sweep_tiles=tiles)
    return G, t[3] - t[0], stages


def _lib_tiles():
    """256 x 256 tiles the last sweep scored on MFMA (swann_sweep_tiles_scored)."""
    from swann_amd import _lib
    return _lib.lib().swann_sweep_tiles_scored()


def mfma_probe(dev, seconds=0.4):
    """The dense fp16 MFMA rate the chip sustains (FLOP/s), timed live with
    HIP events: swann_mfma_probe keeps four independent MFMA chains busy on
    register operands in four waves per SIMD on every CU.  The chip holds a
    lower clock under sustained MFMA load than the 2.4 GHz the published 2.5
    PFLOP/s assumes; this is the rate it then delivers (BASELINE's build
    target divides by the measured peak).  A short run sizes a second one of
    about `seconds`, which is the one reported."""
    from swann_amd import _lib
    blocks = 4 * torch.cuda.get_device_properties(dev).multi_processor_count
    sink = torch.zeros(1, dtype=torch.float32, device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
    iters, rate = 20_000, 0.0
    for _ in range(2):
        ev[0].record()
        _lib.call("swann_mfma_probe", iters, blocks, _lib.ptr(sink), stream)
        ev[1].record()
        torch.cuda.synchronize()
        t = ev[0].elapsed_time(ev[1]) / 1e3
        rate = _lib.lib().swann_mfma_probe_flop(iters, blocks) / t
        iters = max(1, int(iters * seconds / max(t, 1e-6)))
    return rate


def build_roofline(n, d, stages, measured=None):
    """The candidate sweep against the dense fp16 MFMA peak, on the MFMAs it
    executes: the 256 x 256 tiles the library reports scoring
    (swann_sweep_tiles_scored: the symmetric sweep's upper triangle, less
    what the locality-ordered sweep proves empty on clustered rows) x
    2 * 256 * 256 * d FLOP, over the candidate stage's time (sweep + list
    merges + the exact re-rank of an fp32 corpus).  `reference_work` is the
    reference's exact sweep, the full Gram's 2 n^2 d FLOP, over the same
    time: the rate an unpruned, one-sided sweep would need to match it (the
    measure the build target is stated in).  When the ordered sweep
    leaves most tiles out (`tiles_of_triangle` small, clustered rows) the
    stage is no longer bound by its MFMAs but by the re-rank's gathers, the
    list merges and the order, and `bound` says so."""
    flop = 2.0 * n * n * d
    executed = 2.0 * 256 * 256 * d * stages["sweep_tiles"]
    t = stages["candidates"]
    ach = executed / t
    nt = (n + 255) // 256
    share = stages["sweep_tiles"] / (nt * (nt + 1) / 2)
    out = {"bound": "mfma" if share > 0.5 else "other (pruned sweep: re-rank, merges, order)",
           "achieved": round(ach / 1e12, 1), "peak": MFMA_F16_PEAK / 1e12,
           "unit": "TFLOP/s", "frac": round(ach / MFMA_F16_PEAK, 4), "kernel": "sweep_dma_kernel",
           "flop_executed": executed, "tiles_scored": stages["sweep_tiles"],
           "tiles_of_triangle": round(share, 4), "stage_s": t,
           "reference_work": {"flop": flop, "rate_tflops": round(flop / t / 1e12, 1),
                              "frac_of_peak": round(flop / t / MFMA_F16_PEAK, 4)}}
    if measured:
        # against the rate the chip sustained in this run (mfma_probe)
        out["measured_peak"] = round(measured / 1e12, 1)
        out["frac_of_measured_peak"] = round(ach / measured, 4)
    return out


def recall(ids, truth, k=10):
    ids = ids[:, :k].long()
    hit = (ids.unsqueeze(2) == truth[:, :k].unsqueeze(1)).any(2).float().sum(1) / k
    return float(hit.mean())


class Searcher:
    """One search of the batch, phase by phase, with events on torch's current
    stream (where every library kernel is launched)."""

    def __init__(self, index, Q, k, cfg):
        from swann_amd import _engine as E
        from swann_amd import _select as S
        self.E, self.S = E, S
        self.ix, self.Q, self.k = index, Q, k
        self.cfg = cfg
        self.codes = None           # (codes, alpha, mu, margin) for the sign-code pre-filter
        self.ws = None
        self.bits, self.slots = False, None     # claims layout, decided on the first step
        self.ev = [torch.cuda.Event(enable_timing=True) for _ in range(5)]

    def step(self, eps, record=False):
        E, S, ix, cfg = self.E, self.S, self.ix, self.cfg
        if self.ws is None:
            self.ws = torch.empty(int(S._ws_size(self.Q.shape[0], ix._cat.shape[0])),
                                  dtype=torch.uint8, device=self.Q.device)
        ev = self.ev
        if self.slots is None:
            knobs = SimpleNamespace(branches=cfg["branches"], budget=cfg["budget"])
            # the sign-code filter needs the (id, d) table; the plain search
            # shares its claims as Index.search does
            self.bits, self.slots = ((False, ix._table_size(self.Q.shape[0], knobs))
                                     if self.codes is not None else
                                     ix._claims(self.Q.shape[0], knobs))
        if record:
            ev[0].record()
        ent = S.select_nearest_i32(self.Q, ix._cat, cfg["branches"], metric=ix._m,
                                   workspace=self.ws)
        seeds = torch.index_select(ix._cat_ids, 0, ent.view(-1)).view(ent.shape)
        if record:
            ev[1].record()
        st = E.init_states(ix.X, self.Q, seeds, L=cfg["queue"], B=cfg["budget"], D=ix.G.shape[1],
                           metric=ix._m, team_size=cfg["team"], stop_eps=eps, kstop=self.k,
                           shared_cache=True, shared_bound=True, exclusive=True,
                           elide_visited=True, cache_slots=None if self.bits else self.slots,
                           claim_bits=self.bits)
        if record:
            ev[2].record()
        E.advance(ix.X, ix.G, self.Q, st, cfg["budget"], codes=self.codes)
        if record:
            ev[3].record()
        ids, dist = E.merge_state(st, self.k)
        if record:
            ev[4].record()
        return ids, dist, st

    def phase_ms(self):
        e = self.ev
        return dict(select=e[0].elapsed_time(e[1]), init=e[1].elapsed_time(e[2]),
                    advance=e[2].elapsed_time(e[3]), merge=e[3].elapsed_time(e[4]))


def cpu_baseline(X, G, Q, seeds, cfg, eps, k, nsample, metric_id, truth, gpu_ids):
    """The oracle's C restatement (a port of the reference algorithm) on this
    host's cores, on a bounded sample of the same workload: the production
    mode (shared table at the reference's size, bound, claims, no visited
    table) in the rounds schedule, where every branch of a query starts
    together as on the GPU.  Its answers are scored against the same ground
    truth, beside the GPU's recall on the same queries from the timed run."""
    import oracle as O
    from swann_amd import _engine as E
    cores = len(os.sched_getaffinity(0))
    Xh = X.cpu().numpy()
    Gh = G.cpu().numpy()
    Qh = Q[:nsample].cpu().numpy()
    Sh = seeds[:nsample].cpu().numpy()
    Hc = E.cache_size(cfg["branches"], cfg["budget"], G.shape[1])
    O.lib()
    t0 = time.perf_counter()
    oi, _ = O.search_batch(Xh, Gh, Qh, Sh, k=k, L=cfg["queue"], B=cfg["budget"],
                           metric=metric_id, team=cfg["team"], stop_eps=eps, H=1, Hc=Hc,
                           bound=True, exclusive=True, nthreads=cores, schedule="rounds")
    dt = time.perf_counter() - t0
    dev = truth.device
    r_cpu = recall(torch.from_numpy(oi).to(dev), truth[:nsample], k)
    r_gpu = recall(gpu_ids[:nsample], truth[:nsample], k)
    return dict(value=round(nsample / dt, 2), unit="queries/s", cores=cores, kind="port",
                sample=f"{nsample} queries of the timed workload at the same knobs "
                       f"(oracle/swann_oracle.c, OpenMP over queries, rounds schedule)",
                seconds=round(dt, 2), recall_at_10=round(r_cpu, 4),
                gpu_recall_at_10_same_queries=round(r_gpu, 4))


SWEEP_GRID = dict(branches=(16, 32, 64, 128), queue=(12, 24, 48), budget=(64, 128),
                  stop_eps=(0.05, 0.1, 0.2, 0.3))
SWEEP_SHARED_V = (8, 16, 32)
FRONTIER_TARGETS = (0.90, 0.95, 0.99)


def cheapest(rows, target):
    """The fastest row that reaches `target` (bench/pick_settings.py:40-43)."""
    ok = [r for r in rows if r["recall"] >= target]
    return max(ok, key=lambda r: r["qps"]) if ok else None


def run_sweep(index, Q, truth, k, cfg, nq):
    """Recall-QPS grid over the production search path (branches, queue,
    budget, stop_eps; shared table, bound and claims on), plus the
    shared-fanout rows of bench/entry_arms.py: one branch holding V seeds
    (best-first and round-robin lineage policies, budget 128).  Each row is
    the best of two timed searches of the whole batch after one warm-up."""
    from swann_amd import _engine as E
    from swann_amd import _select as S
    rows = []

    def timed(fn):
        fn()
        torch.cuda.synchronize()
        best, ids = None, None
        for _ in range(2):
            t1 = time.perf_counter()
            ids = fn()
            torch.cuda.synchronize()
            dt = time.perf_counter() - t1
            best = dt if best is None else min(best, dt)
        return ids, best

    for J in SWEEP_GRID["branches"]:
        for L in SWEEP_GRID["queue"]:
            for Bud in SWEEP_GRID["budget"]:
                for eps in SWEEP_GRID["stop_eps"]:
                    ids, dt = timed(lambda: index.search_async(
                        Q, k=k, branches=J, queue=L, budget=Bud, stop_eps=eps,
                        team=cfg["team"])[0])
                    row = dict(fanout="branch", branches=J, V=1, queue=L, budget=Bud,
                               stop_eps=eps, recall=round(recall(ids, truth, k), 4),
                               qps=round(nq / dt, 1))
                    log(row)
                    rows.append(row)
    for V in SWEEP_SHARED_V:
        ent = S.select_nearest(Q, index._cat, V, metric=index._m)
        seeds = index.catalogue[ent].to(torch.int32).unsqueeze(1).contiguous()   # [Q, 1, V]
        for pol, pname in ((E.POLICY_BEST, "best"), (E.POLICY_ROUND_ROBIN, "rr")):
            for L in (24, 48):
                ids, dt = timed(lambda: E.search(
                    index.X, index.G, Q, seeds, k=k, L=L, B=128, metric=index._m,
                    team_size=cfg["team"], policy=pol, stop_eps=0.3, check=False)[0])
                row = dict(fanout=f"shared/{pname}", branches=1, V=V, queue=L, budget=128,
                           stop_eps=0.3, recall=round(recall(ids, truth, k), 4),
                           qps=round(nq / dt, 1))
                log(row)
                rows.append(row)
    frontier = {f"{t:g}": cheapest(rows, t) for t in FRONTIER_TARGETS}
    return rows, frontier


# (branches, queue, budget, stop_eps, margin): the fastest recall@10 >= 0.95 row
# of `--sweep-codes` on C3
CODES_POINT = (64, 48, 128, 0.1, 0.05)
CODE_KNOBS = ((64, 48, 64, 0.2), (64, 48, 64, 0.1), (64, 48, 128, 0.1), (64, 48, 128, 0.3),
              (32, 48, 64, 0.2), (32, 48, 128, 0.1), (128, 48, 64, 0.1), (128, 48, 128, 0.1))
CODE_MARGINS = (None, 0.0, 0.01, 0.02, 0.05)


def run_code_sweep(index, Q, truth, k, cfg, nq):
    """The production search with the sign-code pre-filter
    (local_search.cu:205-243, :565-572) at the knobs around the frontier and a
    few margins (None = no codes, the same search as the plain rows).  Codes
    are built once on the GPU from the corpus the index holds."""
    from swann_amd import codes as C
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    cd, al, mu = C.build_codes(index.X)
    torch.cuda.synchronize()
    codes_s = time.perf_counter() - t0
    log(f"codes built in {codes_s:.2f}s ({cd.shape[1]} words per row)")
    rows = []
    for J, L, Bud, eps in CODE_KNOBS:
        for m in CODE_MARGINS:
            srch = Searcher(index, Q, k, dict(cfg, branches=J, queue=L, budget=Bud))
            srch.codes = None if m is None else (cd, al, mu, m)
            srch.step(eps)
            torch.cuda.synchronize()
            best, ids, st = None, None, None
            for _ in range(2):
                t1 = time.perf_counter()
                ids, _, st = srch.step(eps)
                torch.cuda.synchronize()
                dt = time.perf_counter() - t1
                best = dt if best is None else min(best, dt)
            ctr = st.counters.sum(dim=(0, 1)).tolist()
            row = dict(fanout="branch" if m is None else "branch+codes", branches=J, V=1,
                       queue=L, budget=Bud, stop_eps=eps, margin=m,
                       recall=round(recall(ids, truth, k), 4), qps=round(nq / best, 1),
                       rows_read_per_query=round(ctr[1] / nq, 1),
                       ctr3_per_query=round(ctr[3] / nq, 1))    # code skips + exhausted branches
            log(row)
            rows.append(row)
            del srch, st
    frontier = {f"{t:g}": cheapest(rows, t) for t in FRONTIER_TARGETS}
    return rows, frontier, codes_s


def c4_rows(dev, n, npool, reps_scale=1.0):
    """Config C4: p50/p99 latency of one batch (1, 8, 64, 512 queries) at
    branches 32 and 128, queue 12, team 32, the other knobs at their defaults,
    each batch drawn uniformly from a pool of queries (bench/batch_torch.py:
    24-41).  The search is captured once per (branches, batch) as a HIP graph
    (`Index.capture`, no overflow guard) and replayed; the eager search is
    timed beside it.  A latency is the host's wall clock from replay to
    completion.  Returns (rows, build seconds, workload text)."""
    import swann_amd
    from swann_amd.build import build_graph
    cfg = dict(CONFIGS["c4"])
    k = 10
    t0 = time.perf_counter()
    X32, Qpool = generate(cfg, n, npool, dev)
    truth = ground_truth(X32, Qpool, k, cfg["metric"])
    X = X32.half()
    del X32
    torch.cuda.empty_cache()
    torch.cuda.synchronize()
    log(f"c4: generated n={n} d={cfg['d']} pool={npool} in {time.perf_counter() - t0:.1f}s")
    tb = time.perf_counter()
    G = build_graph(X, metric="ip", degree=cfg["D"], candidates=cfg["cand"], alpha=1.2)
    torch.cuda.synchronize()
    build_s = time.perf_counter() - tb
    log(f"c4: graph built in {build_s:.1f}s")
    index = swann_amd.Index(X, G, metric="ip")
    rng = np.random.default_rng(0)
    rows = []
    for J in C4_BRANCHES:
        for b in C4_BATCHES:
            knobs = dict(branches=J, queue=12, team=cfg["team"])
            cs = index.capture(b, k=k, **knobs)
            reps = max(5, int({1: 200, 8: 100, 64: 40, 512: 12}[b] * reps_scale))
            lat_g, lat_e, hits = [], [], 0.0
            for r in range(reps + 2):
                idx = torch.from_numpy(rng.choice(npool, size=b, replace=False)).to(dev)
                qb = Qpool[idx].contiguous()
                torch.cuda.synchronize()
                t1 = time.perf_counter()
                ids, _ = cs.run(qb)
                torch.cuda.synchronize()
                tg = time.perf_counter() - t1
                t1 = time.perf_counter()
                index.search_async(qb, k=k, **knobs)
                torch.cuda.synchronize()
                te = time.perf_counter() - t1
                if r >= 2:                                   # two warm replays
                    lat_g.append(tg * 1e3); lat_e.append(te * 1e3)
                    hits += recall(ids, truth[idx], k) * b
            ng = np.array(lat_g); ne = np.array(lat_e)
            row = dict(branches=J, batch=b, replays=reps,
                       p50_ms=round(float(np.percentile(ng, 50)), 4),
                       p99_ms=round(float(np.percentile(ng, 99)), 4),
                       eager_p50_ms=round(float(np.percentile(ne, 50)), 4),
                       eager_p99_ms=round(float(np.percentile(ne, 99)), 4),
                       qps_at_p50=round(b / (float(np.percentile(ng, 50)) / 1e3), 1),
                       recall_at_10=round(hits / (reps * b), 4))
            log(row)
            rows.append(row)
            del cs
            torch.cuda.empty_cache()
    workload = (f"C4: n={n:,} x d={cfg['d']} fp16 ip (lowrank {cfg['rank']}), "
                f"pool of {npool:,} fp32 queries, D={cfg['D']}, k={k}, queue=12, "
                f"team={cfg['team']}, budget=64, stop_eps=0.05, overflow guard off")
    del index, G, X, Qpool, truth
    torch.cuda.empty_cache()
    return rows, build_s, workload


def run_c4(a, dev):
    """`--config c4`: the C4 latency table as its own JSON line."""
    cfg = CONFIGS["c4"]
    rows, build_s, workload = c4_rows(dev, a.n or cfg["n"], a.nq or cfg["nq"])
    out = {
        "metric": "C4 per-batch latency p50/p99 (hipGraph replay) and recall@10",
        "unit": "ms", "higher_is_better": False, "n_gpus": 1, "dtype": "f32",
        "data": "synthetic (generated on the GPU from fixed seeds; graph built by this library)",
        "config": {"workload": workload},
        "build_s": round(build_s, 2),
        "rows": rows,
    }
    print(json.dumps(out), flush=True)


def advance_bytes(st, nq, J, d, elem, D):
    """Algorithmic bytes of one advance launch from the kernel's own counters:
    rows scored x d x element size + expansions x D x 4 (the reference's
    convention, bench/batch_torch.py:121-128); init scored the seeds."""
    evals = int(st.dist_evals.sum()) - int(nq * J)
    exps = int(st.expansions.sum())
    return evals * d * elem + exps * D * 4


def c2_rows(dev, n, nq, steps=3):
    """Config C2 beside the headline: 1M x 960 fp32 l2 mixture, graph D = 64
    from C = 128, the search at the config's knobs (32 branches, queue 12,
    budget 64) over its stop_eps sweep.  Each row: QPS over `steps` timed
    searches of the whole batch (select + init + advance + merge), recall@10
    against exact fp32 ground truth, and the advance kernel's algorithmic
    bytes over its HIP-event time against 8 TB/s."""
    import swann_amd
    cfg = dict(CONFIGS["c2"], queue=12, budget=64)
    k = 10
    t0 = time.perf_counter()
    X, Q = generate(cfg, n, nq, dev)
    truth = ground_truth(X, Q, k, cfg["metric"])
    torch.cuda.synchronize()
    log(f"c2: generated n={n} d={cfg['d']} nq={nq} in {time.perf_counter() - t0:.1f}s")
    G, build_s, stages = timed_build(X, cfg)
    log(f"c2: graph built in {build_s:.2f}s {stages}")
    index = swann_amd.Index(X, G, metric="l2")
    srch = Searcher(index, Q, k, cfg)
    rows = []
    for eps in EPS_SWEEP:
        srch.step(eps)
        torch.cuda.synchronize()
        adv, t1 = [], time.perf_counter()
        for _ in range(steps):
            ids, _, st = srch.step(eps, record=True)
            torch.cuda.synchronize()
            adv.append(srch.phase_ms()["advance"])
        dt = (time.perf_counter() - t1) / steps
        adv_s = float(np.mean(adv)) / 1e3
        nbytes = advance_bytes(st, nq, cfg["branches"], cfg["d"], 4, G.shape[1])
        row = dict(branches=cfg["branches"], queue=12, budget=64, stop_eps=eps,
                   recall=round(recall(ids, truth, k), 4), qps=round(nq / dt, 1),
                   roofline={"bound": "hbm", "achieved": round(nbytes / adv_s / 1e9, 1),
                             "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                             "frac": round(nbytes / adv_s / HBM_PEAK, 4),
                             "kernel": "advance_kernel", "bytes_per_launch": nbytes,
                             "launch_ms": round(adv_s * 1e3, 3)})
        log("c2", row)
        rows.append(row)
    workload = (f"C2: n={n:,} x d={cfg['d']} fp32 l2 (gmm), {nq:,} fp32 queries, "
                f"D={cfg['D']}, C={cfg['cand']}, k={k}, team={cfg['team']}")
    del srch, index, G, X, Q, truth
    torch.cuda.empty_cache()
    return dict(workload=workload, build_s=round(build_s, 2), build_stages_s=stages,
                eps_sweep=rows, best_at_0_95=cheapest(rows, TARGET_RECALL))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--config", default="c3", choices=sorted(CONFIGS))
    ap.add_argument("--n", type=int, default=0, help="override corpus rows")
    ap.add_argument("--nq", type=int, default=0, help="override query count")
    ap.add_argument("--eps", type=float, default=None, help="skip the sweep, use this stop_eps")
    ap.add_argument("--knobs", default=None,
                    help="branches,queue,budget,stop_eps: skip the operating-point search")
    ap.add_argument("--cpu-sample", type=int, default=500)
    ap.add_argument("--no-codes", action="store_true",
                    help="skip the sign-code pre-filter line reported beside the headline")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-c5-build", action="store_true",
                    help="skip the C5 graph build reported beside the C3 headline")
    ap.add_argument("--no-c2", action="store_true",
                    help="skip the C2 search rows reported beside the C3 headline")
    ap.add_argument("--no-c4", action="store_true",
                    help="skip the C4 latency rows reported beside the C3 headline")
    ap.add_argument("--sweep", action="store_true",
                    help="print the recall-QPS grid and its frontier instead of the headline")
    ap.add_argument("--sweep-codes", action="store_true",
                    help="recall-QPS rows with the sign-code pre-filter at knobs around the "
                         "frontier, instead of the headline")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="run a plain 2 GiB device copy first (scale for rocprof FETCH/WRITE_SIZE)")
    a = ap.parse_args()
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(run with --gpus 1)", file=sys.stderr)
        sys.exit(2)

    if a.config == "c4":
        dev = torch.device("cuda:0")
        torch.cuda.set_device(dev)
        run_c4(a, dev)
        return

    import swann_amd
    cfg = dict(CONFIGS[a.config])
    cfg.update(queue=12, budget=64)
    n = a.n or cfg["n"]
    nq = a.nq or cfg["nq"]
    k = 10
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    t0 = time.perf_counter()
    X32, Q = generate(cfg, n, nq, dev)
    torch.cuda.synchronize()
    log(f"generated n={n} d={cfg['d']} nq={nq} in {time.perf_counter() - t0:.1f}s")
    truth = ground_truth(X32, Q, k, cfg["metric"])
    torch.cuda.synchronize()
    log(f"ground truth in {time.perf_counter() - t0:.1f}s")

    # the graph is built from the corpus the index holds (fp16 rows upcast, as the reference)
    X = X32.half() if cfg["dtype"] == "f16" else X32
    del X32
    torch.cuda.empty_cache()
    torch.cuda.synchronize()
    G, build_s, stages = timed_build(X, cfg)
    log(f"graph built in {build_s:.1f}s {stages}")
    mpeak = mfma_probe(dev)
    log(f"sustained fp16 MFMA rate {mpeak / 1e12:.0f} TFLOP/s (register probe)")
    index = swann_amd.Index(X, G, metric=cfg["metric"])
    srch = Searcher(index, Q, k, cfg)

    if a.sweep:
        rows, frontier = run_sweep(index, Q, truth, k, cfg, nq)
        print(json.dumps({
            "metric": f"recall@10-QPS frontier ({a.config.upper()})", "unit": "queries/s",
            "n_gpus": 1, "higher_is_better": True, "dtype": "f32",
            "data": "synthetic (generated on the GPU from fixed seeds)",
            "config": {"workload": f"{a.config.upper()}: n={n:,} x d={cfg['d']} "
                                   f"{cfg['dtype']} {cfg['metric']}, {nq:,} queries, "
                                   f"D={cfg['D']}, k={k}, team={cfg['team']}"},
            "build_s": round(build_s, 2), "frontier": frontier, "rows": rows}), flush=True)
        return

    if a.sweep_codes:
        rows, frontier, codes_s = run_code_sweep(index, Q, truth, k, cfg, nq)
        print(json.dumps({
            "metric": f"recall@10-QPS with the sign-code pre-filter ({a.config.upper()})",
            "unit": "queries/s", "n_gpus": 1, "higher_is_better": True, "dtype": "f32",
            "data": "synthetic (generated on the GPU from fixed seeds)",
            "config": {"workload": f"{a.config.upper()}: n={n:,} x d={cfg['d']} "
                                   f"{cfg['dtype']} {cfg['metric']}, {nq:,} queries, "
                                   f"D={cfg['D']}, k={k}, team={cfg['team']}"},
            "build_s": round(build_s, 2), "codes_build_s": round(codes_s, 2),
            "frontier": frontier, "rows": rows}), flush=True)
        return

    if a.calibrate_copy:
        src = torch.empty(1 << 29, dtype=torch.float32, device=dev).fill_(1.0)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        log("calibration copy: 3 x 2 GiB read + 2 GiB written")
        del src, dst

    # operating point: the configured knobs with stop_eps swept; if the target
    # is not reached, climb the effort ladder; take the fastest setting that
    # reaches the target (or, failing that, the most accurate one)
    def trial(J, L, Bud, eps):
        srch.cfg.update(branches=J, queue=L, budget=Bud)
        srch.step(eps)
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        ids, _, _ = srch.step(eps)
        torch.cuda.synchronize()
        dt = time.perf_counter() - t1
        r = recall(ids, truth, k)
        row = dict(branches=J, queue=L, budget=Bud, stop_eps=eps, recall=round(r, 4),
                   qps=round(nq / dt, 1))
        log(row)
        return row
    sweep = []
    if a.knobs:
        J, L, Bud, eps = a.knobs.split(",")
        sweep.append(trial(int(J), int(L), int(Bud), float(eps)))
    else:
        for eps in ((a.eps,) if a.eps is not None else EPS_SWEEP):
            sweep.append(trial(cfg["branches"], 12, 64, eps))
        if not any(s["recall"] >= TARGET_RECALL for s in sweep):
            for J, L, Bud, eps in LADDER:
                sweep.append(trial(J, L, Bud, eps))
                if sum(s["recall"] >= TARGET_RECALL for s in sweep) >= 2:
                    break
    ok = [s for s in sweep if s["recall"] >= TARGET_RECALL]
    pick = max(ok, key=lambda s: s["qps"]) if ok else max(sweep, key=lambda s: s["recall"])
    eps = pick["stop_eps"]
    srch.cfg.update(branches=pick["branches"], queue=pick["queue"], budget=pick["budget"])
    cfg.update(branches=pick["branches"], queue=pick["queue"], budget=pick["budget"])

    for _ in range(a.warmup):
        srch.step(eps)
    torch.cuda.synchronize()
    adv_ms, phases = [], []
    t1 = time.perf_counter()
    for _ in range(a.steps):
        ids, dist, st = srch.step(eps, record=True)
        torch.cuda.synchronize()           # read this step's events
        ph = srch.phase_ms()
        phases.append(ph)
        adv_ms.append(ph["advance"])
    torch.cuda.synchronize()
    total = time.perf_counter() - t1
    ms_step = total * 1e3 / a.steps
    qps = nq * a.steps / total
    rec = recall(ids, truth, k)

    # algorithmic bytes of the advance kernel, from its own counters
    elem = 2 if cfg["dtype"] == "f16" else 4
    adv_bytes = advance_bytes(st, nq, cfg["branches"], cfg["d"], elem, G.shape[1])
    adv_s = float(np.mean(adv_ms)) / 1e3
    achieved = adv_bytes / adv_s
    ph_mean = {k2: round(float(np.mean([p[k2] for p in phases])), 3) for k2 in phases[0]}
    src_sha = kernel_source_key(ROOT / "swann_amd" / "csrc" / "search.hip")
    bits, slots = index._claims(nq, SimpleNamespace(branches=cfg["branches"],
                                                    budget=cfg["budget"]))
    layout = f"bits{slots}" if bits else slots
    traffic = PMC_TRAFFIC.get((a.config, n, nq, cfg["branches"], cfg["queue"], cfg["budget"],
                               eps, layout, src_sha))

    cpu = None
    if not a.no_cpu and a.cpu_sample > 0:
        ent = swann_amd._select.select_nearest(Q[:a.cpu_sample], index._cat, cfg["branches"],
                                               metric=index._m)
        seeds = index.catalogue[ent].to(torch.int32)
        try:
            cpu = cpu_baseline(X, G, Q, seeds, cfg, eps, k, a.cpu_sample, index._m, truth, ids)
            log(f"cpu baseline {cpu}")
        except Exception as e:                                   # noqa: BLE001
            log(f"cpu baseline failed: {e}")

    # the same workload with the sign-code pre-filter at its frontier point;
    # reported beside the headline, which is the Index.search path (no codes knob)
    with_codes = None
    if cfg["metric"] == "ip" and not a.no_codes:
        from swann_amd import codes as C
        cd, al, mu = C.build_codes(index.X)
        J, L, Bud, ceps, margin = CODES_POINT
        cs = Searcher(index, Q, k, dict(cfg, branches=J, queue=L, budget=Bud))
        cs.codes = (cd, al, mu, margin)
        cs.step(ceps)
        torch.cuda.synchronize()
        times = []
        for _ in range(3):
            t1 = time.perf_counter()
            ids_c, _, st_c = cs.step(ceps)
            torch.cuda.synchronize()
            times.append(time.perf_counter() - t1)
        with_codes = dict(branches=J, queue=L, budget=Bud, stop_eps=ceps, margin=margin,
                          recall_at_10=round(recall(ids_c, truth, k), 4),
                          qps=round(nq / float(np.median(times)), 1),
                          rows_read_per_query=round(float(st_c.dist_evals.sum()) / nq, 1),
                          path="engine search with codes=(codes, alpha, mu, margin) "
                               "(swann/_engine.py:281-317, local_search.cu:205-243)")
        log(f"with codes {with_codes}")
        del cs, cd, al, mu

    # the build target's own shape, C5 (1M x 1024 fp32 l2 mixture), built beside
    # the headline: the candidate sweep's MFMA fraction is quoted on it
    build_c5 = None
    if a.config == "c3" and not a.no_c5_build:
        c5 = dict(CONFIGS["c5"])
        n5 = a.n or c5["n"]
        X5, _ = generate(c5, n5, 1, dev)
        torch.cuda.synchronize()
        _, b5_s, st5 = timed_build(X5, c5)
        build_c5 = {"workload": f"C5: n={n5:,} x d={c5['d']} fp32 l2 (gmm), D={c5['D']}, "
                                f"C={c5['cand']}, alpha=1.2",
                    "build_s": round(b5_s, 2), "build_s_per_1M_rows": round(b5_s * 1e6 / n5, 2),
                    "build_stages_s": st5, "build_roofline": build_roofline(n5, c5["d"], st5, mpeak)}
        log(f"c5 build {build_c5}")
        del X5
        torch.cuda.empty_cache()

    # configs C2 and C4 at their own shapes, beside the headline
    c2 = c4 = None
    if a.config == "c3" and not a.no_c2:
        c2 = c2_rows(dev, a.n or CONFIGS["c2"]["n"], a.nq or CONFIGS["c2"]["nq"])
    if a.config == "c3" and not a.no_c4:
        rows4, b4_s, w4 = c4_rows(dev, a.n // 2 or CONFIGS["c4"]["n"], CONFIGS["c4"]["nq"],
                                  reps_scale=0.5)
        c4 = dict(workload=w4, build_s=round(b4_s, 2), rows=rows4)

    out = {
        "metric": "QPS at recall@10=0.95 (1 GPU) + achieved HBM GB/s fraction; build s/1M rows",
        "value": round(qps, 1), "unit": "queries/s", "n_gpus": 1, "steps": a.steps,
        "warmup": a.warmup, "ms_per_step": round(ms_step, 3), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (generated on the GPU from fixed seeds; graph built by this "
                "library's exact sweep, prune and reverse)",
        "config": {"workload": f"{a.config.upper()}: n={n:,} x d={cfg['d']} {cfg['dtype']} "
                               f"{cfg['metric']} ({cfg['gen']}), {nq:,} fp32 queries, D={cfg['D']}, "
                               f"k={k}, team={cfg['team']}",
                   "branches": cfg["branches"], "queue": cfg["queue"], "budget": cfg["budget"],
                   "stop_eps": eps, "corpus_dtype": cfg["dtype"]},
        "recall_at_10": round(rec, 4),
        "recall_target_met": rec >= TARGET_RECALL,
        "eps_sweep": sweep,
        "phase_ms": ph_mean,
        "build_s": round(build_s, 2),
        "build_s_per_1M_rows": round(build_s * 1e6 / n, 2),
        "build_stages_s": stages,
        "build_roofline": build_roofline(n, cfg["d"], stages, mpeak),
        "roofline": {"bound": "hbm", "achieved": round(achieved / 1e9, 1),
                     "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK, 4), "traffic": traffic,
                     "kernel": "advance_kernel",
                     "bytes_per_launch": adv_bytes, "launch_ms": round(adv_s * 1e3, 3),
                     "claims": layout},
        "cpu_baseline": cpu,
        "with_codes": with_codes,
        "build_c5": build_c5,
        "c2": c2,
        "c4": c4,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
