"""CPU oracle for the SWANN search and build path -- TEST INFRASTRUCTURE ONLY.

This package is the checker. Only `tests/`, `__graft_entry__.smoke()` and the
`cpu_baseline` leg of `bench.py` may import it. The product (`swann_amd`)
never imports, links or calls anything here, and fails loudly when its own HIP
library is missing.

The arithmetic lives in `swann_oracle.c` (plain C, fp32 with
-ffp-contract=off); this module is a numpy front end over it through ctypes.
Each function names the reference file:line it restates.

Parity pins (see tests/test_oracle.py): the distance against closed forms and
order-sensitive hand cases; the branch walk against golden vectors written from
the reference's own `_refcpu.py` (tests/golden/make_golden.py) and against
brute force on a complete graph; merge, select and the sweep against brute
force; prune and reverse against golden vectors from the reference's CPU-torch
build stages and the DiskANN rule's invariants.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
SRC = HERE / "swann_oracle.c"
LIB = HERE / "_build" / "libswann_oracle.so"

METRIC_IP, METRIC_L2 = 0, 1
POLICY_BEST, POLICY_ROUND_ROBIN = 0, 1
# when a branch's step reads the shared bound (so_search_query)
SCHEDULES = {"serial": 0, "rounds": 1, "rounds2": 2}
NCTR = 10
F32, F16 = 0, 1

_lib = None


def build(force: bool = False) -> Path:
    """Compile the C restatement with gcc into oracle/_build/."""
    if LIB.exists() and not force and LIB.stat().st_mtime >= SRC.stat().st_mtime:
        return LIB
    LIB.parent.mkdir(parents=True, exist_ok=True)
    tmp = LIB.with_suffix(f".so.tmp{os.getpid()}")
    cmd = ["gcc", "-O2", "-std=c11", "-fPIC", "-shared", "-fopenmp",
           "-ffp-contract=off", "-fno-fast-math", "-o", str(tmp), str(SRC), "-lm"]
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    return LIB


def lib():
    global _lib
    if _lib is None:
        build()
        _lib = ctypes.CDLL(str(LIB))
        _declare(_lib)
    return _lib


P = ctypes.c_void_p
I = ctypes.c_int
I64 = ctypes.c_int64
F = ctypes.c_float


def _declare(L):
    L.so_team_distance.restype = F
    L.so_team_distance.argtypes = [P, P, I, I64, I, I, I]
    L.so_init_branch.restype = None
    L.so_init_branch.argtypes = [P, I, I, P, P, I, I, I, I, I, P, P, P, P, P, P]
    L.so_advance_branch.restype = None
    L.so_advance_branch.argtypes = [P, I, I, P, I, P, P, P, P, P, I, P, I, P,
                                    I, I, I, I, I, I, F, I, I, F, P, I, P, P, F]
    L.so_merge.restype = None
    L.so_merge.argtypes = [P, P, I64, I, I, I, P, P]
    L.so_search_query.restype = None
    L.so_search_query.argtypes = [P, I, I, P, I, P, P, I, I, I, I, I, I, I, I, F, I,
                                  I, I, I, I, F, P, P, P, P, P, P, P, P, P, P, I, P, P, F, I]
    L.so_search_batch.restype = None
    L.so_search_batch.argtypes = [P, I, I, P, I, P, I64, P, I, I, I, I, I, I, I, I,
                                  F, I, I, I, I, I, P, P, P, I, I]
    L.so_topk_rows.restype = None
    L.so_topk_rows.argtypes = [P, I64, P, I64, I, I, I, I64, P, P, I]
    L.so_robust_prune.restype = None
    L.so_robust_prune.argtypes = [P, I64, I, I, P, P, I, I, F, P, P, P, I]
    L.so_add_reverse.restype = None
    L.so_add_reverse.argtypes = [P, I64, I, I, P, I, F, I, P, P, I]
    L.so_code_sums.restype = None
    L.so_code_sums.argtypes = [P, P, I, P, P]
    L.so_code_ip.restype = F
    L.so_code_ip.argtypes = [P, P, F, F, F, I, I, I]
    L.so_build_codes.restype = None
    L.so_build_codes.argtypes = [P, I64, I, P, P, P, P]
    L.so_candidates_from_graph.restype = None
    L.so_candidates_from_graph.argtypes = [P, I64, I, I, P, I, I, P, P, I]
    L.so_mutual_rank.restype = None
    L.so_mutual_rank.argtypes = [P, I64, I, I, P]
    L.so_fill_degree.restype = None
    L.so_fill_degree.argtypes = [P, I64, I, P, I, I, I, P]
    L.so_enforce_min_in.restype = I
    L.so_enforce_min_in.argtypes = [P, I64, I, P, I, I, I]
    L.so_half_to_float_export.restype = F
    L.so_half_to_float_export.argtypes = [ctypes.c_uint16]


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p) if a is not None else None


def _corpus(X):
    X = np.ascontiguousarray(X)
    if X.dtype == np.float16:
        return X, F16
    return np.ascontiguousarray(X, dtype=np.float32), F32


def _ts(x, n=1):
    return max(n, int(x))


# -- distance ------------------------------------------------------------
def team_distance(q, X, row, metric=METRIC_IP, team=32):
    """One distance in the kernel's order (local_search.cu:185-203,
    _refcpu.py:21-48); `X` is the corpus and `row` the node id."""
    X, dt = _corpus(X)
    q = np.ascontiguousarray(q, dtype=np.float32)
    return np.float32(lib().so_team_distance(_p(q), _p(X), dt, int(row), X.shape[1],
                                             int(metric), int(team)))


# -- one branch ----------------------------------------------------------
class Branch:
    """One branch's state in the kernel's layout: ids/dist/expanded/lineage [L],
    visited [H], counters [10]."""

    def __init__(self, L, H):
        self.ids = np.full(L, -1, np.int32)
        self.dist = np.full(L, np.finfo(np.float32).max, np.float32)
        self.expanded = np.ones(L, np.uint8)
        self.lineage = np.zeros(L, np.uint8)
        self.visited = np.zeros(max(1, H), np.int32)
        self.counters = np.zeros(NCTR, np.int32)

    @property
    def queue(self):
        """Real entries as (id, dist, expanded, lineage), like _refcpu."""
        return [(int(i), np.float32(d), bool(e), int(l))
                for i, d, e, l in zip(self.ids, self.dist, self.expanded, self.lineage)
                if i >= 0]


def visited_size(B, D):
    """_engine.py:73-77"""
    n = 1
    while n < 2 * (1 + B * D):
        n <<= 1
    return n


def init_branch(X, q, seeds, L=16, H=None, B=16, D=32, metric=METRIC_IP, team=32):
    """local_search.cu:271-351 for one branch; `seeds` is a list of V ids."""
    X, dt = _corpus(X)
    q = np.ascontiguousarray(q, dtype=np.float32)
    seeds = np.ascontiguousarray(np.atleast_1d(np.asarray(seeds, dtype=np.int32)))
    H = visited_size(B, D) if H is None else int(H)
    br = Branch(L, H)
    lib().so_init_branch(_p(X), dt, X.shape[1], _p(q), _p(seeds), len(seeds), L, H,
                         int(metric), int(team), _p(br.ids), _p(br.dist),
                         _p(br.expanded), _p(br.lineage), _p(br.visited), _p(br.counters))
    br.V = len(seeds)
    return br


def _codes(codes):
    """(codes [n, cwords] int32, alpha [n] fp32, mu [dim] fp32, margin) or None."""
    if codes is None:
        return None, 0, None, None, 0.0, ()
    cd, al, mu, margin = codes
    cd = np.ascontiguousarray(cd, dtype=np.int32)
    al = np.ascontiguousarray(al, dtype=np.float32)
    mu = np.ascontiguousarray(mu, dtype=np.float32)
    return _p(cd), cd.shape[1], _p(al), _p(mu), float(margin), (cd, al, mu)


def advance_branch(X, G, q, br, delta, B, metric=METRIC_IP, team=32,
                   policy=POLICY_BEST, stop_eps=-1.0, kstop=10, stall_patience=0,
                   crowd_frac=0.0, codes=None):
    """local_search.cu:451-683 for one branch, in place.  `codes` is the
    sign-code filter's (codes, alpha, mu, margin), as the reference's
    `advance` takes it (_engine.py:281-317)."""
    X, dt = _corpus(X)
    G = np.ascontiguousarray(G, dtype=np.int32)
    q = np.ascontiguousarray(q, dtype=np.float32)
    cp, cw, ap, mp, mg, _keep = _codes(codes)
    L = len(br.ids)
    lib().so_advance_branch(_p(X), dt, X.shape[1], _p(G), G.shape[1], _p(q),
                            _p(br.ids), _p(br.dist), _p(br.expanded), _p(br.lineage), L,
                            _p(br.visited), len(br.visited), _p(br.counters),
                            int(metric), int(team), int(delta), int(B), int(policy),
                            int(br.V), float(stop_eps), int(kstop), int(stall_patience),
                            float(crowd_frac), cp, cw, ap, mp, mg)
    return br


def run(X, G, q, seeds, L=16, B=16, metric=METRIC_IP, team=32, policy=POLICY_BEST,
        stop_eps=-1.0, kstop=10, H=None):
    """init + one full-budget advance (_refcpu.py:146-151)."""
    G = np.ascontiguousarray(G, dtype=np.int32)
    br = init_branch(X, q, seeds, L=L, H=H, B=B, D=G.shape[1], metric=metric, team=team)
    return advance_branch(X, G, q, br, B, B, metric=metric, team=team, policy=policy,
                          stop_eps=stop_eps, kstop=kstop)


# -- a query's branches in one serial schedule ---------------------------
def cache_size(J, B, D, share=4.0, cap=1 << 20):
    """_engine.py:186-198"""
    want = 2 * (1 + J * (1 + B * D) / share)
    n = 1
    while n < int(want):
        n <<= 1
    return min(n, cap)


def search_query(X, G, q, seeds, L=16, B=16, metric=METRIC_IP, team=32,
                 policy=POLICY_BEST, stop_eps=-1.0, kstop=10, H=None, Hc=0,
                 bound=False, exclusive=False, stall_patience=0, crowd_frac=0.0,
                 codes=None, schedule="serial", claim_bits=False):
    """All J branches of one query, stepped in turn (every step atomic).
    seeds: [J] or [J, V].  Returns a dict of [J, ...] arrays.

    claim_bits: exclusive claims kept as one bit per corpus row instead of
    the Hc-slot table (Hc is then ignored); the table at a size where no
    probe fails decides every claim the same way.

    schedule "serial": a step reads the bound as the steps before it left it;
    "rounds": every step of round s reads the bound as it was when the round
    began (a concurrent launch's shape: a query's branches start together)."""
    X, dt = _corpus(X)
    cp, cw, ap, mp, mg, _keep = _codes(codes)
    Hc = _claim_arg(X, Hc, exclusive, claim_bits, codes)
    G = np.ascontiguousarray(G, dtype=np.int32)
    q = np.ascontiguousarray(q, dtype=np.float32)
    seeds = np.asarray(seeds, dtype=np.int32)
    if seeds.ndim == 1:
        seeds = seeds[:, None]
    seeds = np.ascontiguousarray(seeds)
    J, V = seeds.shape
    H = visited_size(B, G.shape[1]) if H is None else int(H)
    ids = np.empty((J, L), np.int32); dist = np.empty((J, L), np.float32)
    expd = np.empty((J, L), np.uint8); lin = np.empty((J, L), np.uint8)
    vis = np.empty((J, H), np.int32); ctr = np.empty((J, NCTR), np.int32)
    cid = np.empty(max(1, Hc, (-Hc + 31) // 32), np.int32)
    cdd = np.empty(max(1, Hc), np.float32)
    bnd = np.empty(1, np.float32)
    lib().so_search_query(_p(X), dt, X.shape[1], _p(G), G.shape[1], _p(q), _p(seeds), J, V,
                          L, B, H, int(metric), int(team), int(policy), float(stop_eps),
                          int(kstop), int(Hc), int(bool(bound)), int(bool(exclusive)),
                          int(stall_patience), float(crowd_frac),
                          _p(ids), _p(dist), _p(expd), _p(lin), _p(vis), _p(ctr),
                          _p(cid), _p(cdd), _p(bnd), cp, cw, ap, mp, mg, SCHEDULES[schedule])
    return dict(ids=ids, dist=dist, expanded=expd, lineage=lin, visited=vis,
                counters=ctr, cache_id=cid[:Hc] if Hc >= 0 else cid[:(-Hc + 31) // 32],
                cache_d=cdd[:max(Hc, 0)], bound=bnd[0])


def search_batch(X, G, Q, seeds, k=10, L=16, B=16, metric=METRIC_IP, team=32,
                 policy=POLICY_BEST, stop_eps=-1.0, H=None, Hc=0, bound=False,
                 exclusive=False, nthreads=0, counters=False, schedule="serial",
                 claim_bits=False):
    """search_query + merge for every query (OpenMP over queries).
    seeds: [nq, J] or [nq, J, V]."""
    X, dt = _corpus(X)
    Hc = _claim_arg(X, Hc, exclusive, claim_bits, None)
    G = np.ascontiguousarray(G, dtype=np.int32)
    Q = np.ascontiguousarray(Q, dtype=np.float32)
    seeds = np.asarray(seeds, dtype=np.int32)
    if seeds.ndim == 2:
        seeds = seeds[:, :, None]
    seeds = np.ascontiguousarray(seeds)
    nq, J, V = seeds.shape
    H = visited_size(B, G.shape[1]) if H is None else int(H)
    oi = np.empty((nq, k), np.int32); od = np.empty((nq, k), np.float32)
    oc = np.empty((nq, J, NCTR), np.int32) if counters else None
    lib().so_search_batch(_p(X), dt, X.shape[1], _p(G), G.shape[1], _p(Q), nq, _p(seeds),
                          J, V, L, B, H, int(metric), int(team), int(policy),
                          float(stop_eps), int(k), int(Hc), int(bool(bound)),
                          int(bool(exclusive)), int(k), _p(oi), _p(od), _p(oc),
                          int(nthreads), SCHEDULES[schedule])
    return (oi, od, oc) if counters else (oi, od)


def _claim_arg(X, Hc, exclusive, claim_bits, codes):
    """The C entry points' Hc: the table's slots, or minus the number of
    claim bits (a power of two >= n and >= 32, as the GPU sizes them)."""
    if not claim_bits:
        return int(Hc)
    if not exclusive or codes is not None:
        raise ValueError("claim bits stand for exclusive claims without sign codes")
    nb = 32
    while nb < X.shape[0]:
        nb <<= 1
    return -nb


# -- sign codes ----------------------------------------------------------
def code_sums(q, mu):
    """(<q, mu>, sum(q)) in the fixed 64-partial order the kernel uses."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    mu = np.ascontiguousarray(mu, dtype=np.float32)
    a = np.zeros(1, np.float32); b = np.zeros(1, np.float32)
    lib().so_code_sums(_p(q), _p(mu), len(q), _p(a), _p(b))
    return a[0], b[0]


def code_ip(q, code_row, alpha, mu, team=16):
    """The code's IP-distance estimate, local_search.cu:222-243."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    code_row = np.ascontiguousarray(code_row, dtype=np.int32)
    qmu, qsum = code_sums(q, mu)
    return np.float32(lib().so_code_ip(_p(q), _p(code_row), float(alpha), float(qmu),
                                       float(qsum), len(q), len(code_row), int(team)))


def build_codes(X, mu=None):
    """Sign codes around the corpus mean: (codes [n, ceil(d/32)] int32,
    alpha [n] fp32, mu [d] fp32)."""
    X = np.ascontiguousarray(X, dtype=np.float32)
    n, d = X.shape
    cw = (d + 31) // 32
    codes = np.empty((n, cw), np.int32); alpha = np.empty(n, np.float32)
    mu_out = np.empty(d, np.float32)
    mu_in = None if mu is None else np.ascontiguousarray(mu, dtype=np.float32)
    lib().so_build_codes(_p(X), n, d, _p(mu_in), _p(codes), _p(alpha), _p(mu_out))
    return codes, alpha, mu_out


# -- merge ---------------------------------------------------------------
def merge(bids, bdist, k):
    """local_search.cu:863-919: per query, first k distinct ids by (d, id)."""
    bids = np.ascontiguousarray(bids, dtype=np.int32)
    bdist = np.ascontiguousarray(bdist, dtype=np.float32)
    Q, V, kk = bids.shape
    oi = np.empty((Q, k), np.int32); od = np.empty((Q, k), np.float32)
    lib().so_merge(_p(bids), _p(bdist), Q, V, kk, int(k), _p(oi), _p(od))
    return oi, od


# -- selection and build -------------------------------------------------
def topk_rows(A, Y, C, metric=METRIC_IP, self_offset=-1, nthreads=0):
    A = np.ascontiguousarray(A, dtype=np.float32)
    Y = np.ascontiguousarray(Y, dtype=np.float32)
    idx = np.empty((A.shape[0], C), np.int32); dst = np.empty((A.shape[0], C), np.float32)
    lib().so_topk_rows(_p(A), A.shape[0], _p(Y), Y.shape[0], A.shape[1], int(metric), int(C),
                       int(self_offset), _p(idx), _p(dst), int(nthreads))
    return idx, dst


def select_nearest(Q, Vp, E, metric=METRIC_IP, nthreads=0):
    """_select.py:93-128: the E nearest catalogue rows, ascending."""
    return topk_rows(Q, Vp, min(E, len(Vp)), metric, -1, nthreads)


def knn_candidates(X, C, metric=METRIC_IP, nthreads=0):
    """build.py:28-43: exact top-C per row, self excluded."""
    return topk_rows(X, X, C, metric, 0, nthreads)


def robust_prune(X, cand, cdist, deg, alpha=1.2, metric=METRIC_IP, nthreads=0,
                 deg_per_node=None, protect=None):
    """build.py:46-91.  With `deg_per_node` the row width is its maximum and
    node u keeps at most deg_per_node[u]; `protect` [n, C] bool exempts a
    candidate from the detour test."""
    X = np.ascontiguousarray(X, dtype=np.float32)
    cand = np.ascontiguousarray(cand, dtype=np.int32)
    cdist = np.ascontiguousarray(cdist, dtype=np.float32)
    dpn = None if deg_per_node is None else np.ascontiguousarray(deg_per_node, dtype=np.int32)
    width = int(deg) if dpn is None else int(dpn.max())
    prot = None if protect is None else np.ascontiguousarray(protect, dtype=np.uint8)
    out = np.empty((X.shape[0], width), np.int32)
    lib().so_robust_prune(_p(X), X.shape[0], X.shape[1], int(metric), _p(cand), _p(cdist),
                          cand.shape[1], width, float(alpha), _p(dpn), _p(prot), _p(out),
                          int(nthreads))
    return out


def add_reverse(X, G, deg, alpha=1.2, max_in=64, metric=METRIC_IP, nthreads=0,
                deg_per_node=None):
    """build.py:94-150; with `deg_per_node` the width is its maximum (G must
    have that many columns) and node u keeps at most deg_per_node[u]."""
    X = np.ascontiguousarray(X, dtype=np.float32)
    G = np.ascontiguousarray(G, dtype=np.int32)
    dpn = None if deg_per_node is None else np.ascontiguousarray(deg_per_node, dtype=np.int32)
    width = int(deg) if dpn is None else int(dpn.max())
    assert G.shape[1] == width
    out = np.empty((X.shape[0], width), np.int32)
    lib().so_add_reverse(_p(X), X.shape[0], X.shape[1], int(metric), _p(G), width,
                         float(alpha), int(max_in), _p(dpn), _p(out), int(nthreads))
    return out


def build_graph(X, metric=METRIC_IP, degree=96, candidates=128, alpha=1.2, nthreads=0):
    """build.py:153-171: sweep, prune, reverse."""
    X = np.ascontiguousarray(X, dtype=np.float32)
    cand, cdist = knn_candidates(X, candidates, metric, nthreads)
    G = robust_prune(X, cand, cdist, degree, alpha, metric, nthreads)
    return add_reverse(X, G, degree, alpha, 64, metric, nthreads)


# -- the offline builder's extras (offline/build_graph.py) ----------------
FILL_RULES = {"near": 0, "far": 1, "bridge": 2}


def candidates_from_graph(X, Gc, C, metric=METRIC_IP, nthreads=0):
    """build_graph.py:63-91"""
    X = np.ascontiguousarray(X, dtype=np.float32)
    Gc = np.ascontiguousarray(Gc, dtype=np.int32)
    C = min(int(C), Gc.shape[1])
    idx = np.empty((X.shape[0], C), np.int32); dst = np.empty((X.shape[0], C), np.float32)
    lib().so_candidates_from_graph(_p(X), X.shape[0], X.shape[1], int(metric), _p(Gc),
                                   Gc.shape[1], C, _p(idx), _p(dst), int(nthreads))
    return idx, dst


def mutual_rank(cand, M):
    """build_graph.py:93-131"""
    cand = np.ascontiguousarray(cand, dtype=np.int32)
    out = np.empty(cand.shape, np.uint8)
    lib().so_mutual_rank(_p(cand), cand.shape[0], cand.shape[1], int(M), _p(out))
    return out.astype(bool)


def fill_degree(G, cand, rule="bridge", chunk=1024):
    """build_graph.py:132-200"""
    G = np.ascontiguousarray(G, dtype=np.int32)
    cand = np.ascontiguousarray(cand, dtype=np.int32)
    out = np.empty_like(G)
    lib().so_fill_degree(_p(G), G.shape[0], G.shape[1], _p(cand), cand.shape[1],
                         FILL_RULES[rule], int(chunk), _p(out))
    return out


def enforce_min_in(G, cand, min_in, rounds=4):
    """build_graph.py:203-294; returns a new graph."""
    G = np.array(G, dtype=np.int32, order="C", copy=True)
    cand = np.ascontiguousarray(cand, dtype=np.int32)
    lib().so_enforce_min_in(_p(G), G.shape[0], G.shape[1], _p(cand), cand.shape[1],
                            int(min_in), int(rounds))
    return G
