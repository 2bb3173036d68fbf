"""The search engine: explicit entries, a resumable state, exact distances.

The same semantics as the reference engine (swann/_engine.py), driven through
the gfx950 library's C ABI instead of a JIT-built CUDA extension:

  queue      best-L over everything evaluated so far, sorted by (distance, id),
             with the `expanded` flag carried along by every merge.
  stop       budget spent, or no retained candidate left unexpanded.
  budget     node expansions, counted per branch; distance evaluations are a
             separate counter.
  resume     advance(a) then advance(b) == advance(a+b).

All state is allocated here with torch on the corpus's GPU and mutated in
place by the kernels; nothing on the search path allocates inside the
library, so a search can be captured in a hipGraph.  Launches go on torch's
current stream.  There is no CPU path: a missing library or GPU raises.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _lib
from ._lib import call, ptr, stream_of

POLICY_BEST = 0          # expand the nearest unexpanded candidate, always
POLICY_ROUND_ROBIN = 1   # give each seed lineage its turn

METRIC_IP = 0   # distance = 1 - dot. Vectors must be L2-normalised.
METRIC_L2 = 1   # distance = ||q - x||^2
NCTR = 10       # expansions, distance evals, hash failures, exhausted, cache hits,
                # cache slots claimed, stalled, crowded, kept candidates, expansions counted

_DTYPES = {torch.float32: 0, torch.float16: 1}


def next_pow2(x: int) -> int:
    n = 1
    while n < x:
        n <<= 1
    return n


def visited_size(B: int, D: int) -> int:
    """Load factor <= 0.5 when every expansion inserts D new nodes, plus the
    seed (swann/_engine.py:73-77)."""
    return next_pow2(2 * (1 + B * D))


def cache_size(J, B, D, share=4.0, cap=1 << 20):
    """Slots for the per-query shared table (swann/_engine.py:186-198): sized
    for the overlap the branches actually have, `share`, capped at 2^20."""
    want = 2 * (1 + J * (1 + B * D) / share)
    return min(next_pow2(int(want)), cap)


@dataclass
class SearchState:
    """Everything a branch needs to be stopped and resumed (swann/_engine.py:80-183)."""
    ids: torch.Tensor        # int32  [Q, J, L]  -1 = empty slot
    dist: torch.Tensor       # float32[Q, J, L]
    expanded: torch.Tensor   # uint8  [Q, J, L]
    lineage: torch.Tensor    # uint8  [Q, J, L]
    visited: torch.Tensor    # int32  [Q, J, H]
    counters: torch.Tensor   # int32  [Q, J, NCTR]
    B: int
    metric: int
    team_size: int
    V: int = 1
    policy: int = POLICY_BEST
    stop_eps: float = -1.0
    stall_patience: int = 0
    crowd_frac: float = 0.0
    kstop: int = 10
    cache_id: torch.Tensor = None
    cache_d: torch.Tensor = None
    bound: torch.Tensor = None
    exclusive: bool = False

    @property
    def shape(self):
        return tuple(self.ids.shape)

    @property
    def expansions(self) -> torch.Tensor:
        return self.counters[..., 0]

    @property
    def dist_evals(self) -> torch.Tensor:
        return self.counters[..., 1]

    @property
    def hash_failures(self) -> torch.Tensor:
        return self.counters[..., 2]

    @property
    def exhausted(self) -> torch.Tensor:
        return self.counters[..., 3]

    @property
    def stalled(self) -> torch.Tensor:
        return self.counters[..., 6]

    @property
    def crowded(self) -> torch.Tensor:
        return self.counters[..., 7]

    @property
    def fanout(self):
        return self.counters[..., 8], self.counters[..., 9]

    @property
    def cache_hits(self) -> torch.Tensor:
        return self.counters[..., 4]

    def check(self):
        """Raise if the visited table overflowed (synchronises)."""
        nf = int(self.hash_failures.sum())
        if nf:
            raise RuntimeError(
                f"visited table overflowed on {int((self.hash_failures > 0).sum())} branches "
                f"({nf} failed inserts): raise max_expansions used for sizing, or the table size")

    def overflow(self) -> torch.Tensor:
        """The overflow count as a device scalar, computed by one kernel with
        no host synchronisation (capturable)."""
        out = torch.empty((), dtype=torch.int32, device=self.counters.device)
        nb = self.counters.numel() // NCTR
        call("swann_overflow_async", ptr(self.counters), nb, ctypes_ptr(out),
             stream_of(self.counters.device))
        return out

    def clone(self) -> "SearchState":
        c = lambda t: None if t is None else t.clone()  # noqa: E731
        return SearchState(ids=c(self.ids), dist=c(self.dist), expanded=c(self.expanded),
                           lineage=c(self.lineage), visited=c(self.visited),
                           counters=c(self.counters), B=self.B, metric=self.metric,
                           team_size=self.team_size, V=self.V, policy=self.policy,
                           stop_eps=self.stop_eps, stall_patience=self.stall_patience,
                           crowd_frac=self.crowd_frac, kstop=self.kstop,
                           cache_id=c(self.cache_id), cache_d=c(self.cache_d),
                           bound=c(self.bound), exclusive=self.exclusive)


def ctypes_ptr(t):
    import ctypes
    return ctypes.c_void_p(t.data_ptr())


# Whether `search` checks, synchronously, that no visited table overflowed.
_OVERFLOW_GUARD = True


def overflow_guard(on: bool) -> bool:
    """Turn the per-search overflow check on or off. Returns the old setting."""
    global _OVERFLOW_GUARD
    was, _OVERFLOW_GUARD = _OVERFLOW_GUARD, bool(on)
    return was


def _check_corpus(X, Qv):
    if not (X.is_cuda and X.dtype in _DTYPES and X.is_contiguous() and X.dim() == 2):
        raise RuntimeError("X: contiguous cuda float32 or float16 [n, dim]")
    if not (Qv.is_cuda and Qv.dtype == torch.float32 and Qv.is_contiguous() and Qv.dim() == 2):
        raise RuntimeError("Q: contiguous cuda float32 [Q, dim]")
    if Qv.shape[1] != X.shape[1]:
        raise RuntimeError(f"Q has dimension {Qv.shape[1]}, X has {X.shape[1]}")


def init_states(X, Qv, seeds, L=16, B=16, D=None, metric=METRIC_IP, team_size=32,
                policy=POLICY_BEST, stop_eps=-1.0, kstop=10, shared_cache=False,
                shared_bound=False, exclusive=False, stall_patience=0, crowd_frac=0.0,
                elide_visited=False, cache_slots=None) -> SearchState:
    """One state per (query, branch); swann/_engine.py:219-278.

    `seeds` is int32 [Q, J] (one entry per branch) or [Q, J, V] (V entries
    sharing one branch).  -1 is an empty slot."""
    _check_corpus(X, Qv)
    seeds = seeds.to(device=X.device, dtype=torch.int32).contiguous()
    if seeds.dim() == 2:
        seeds = seeds.unsqueeze(-1)
    Q, J, V = seeds.shape
    if Q != Qv.shape[0]:
        raise RuntimeError(f"seeds cover {Q} queries, Q has {Qv.shape[0]}")
    if D is None:
        raise ValueError("D (the graph out-degree) is required: it sizes the visited table")
    elide = bool(elide_visited and exclusive and shared_cache and J > 1 and V == 1)
    H = 1 if elide else visited_size(B, D)
    dev = X.device
    st = SearchState(
        ids=torch.empty((Q, J, L), dtype=torch.int32, device=dev),
        dist=torch.empty((Q, J, L), dtype=torch.float32, device=dev),
        expanded=torch.empty((Q, J, L), dtype=torch.uint8, device=dev),
        lineage=torch.empty((Q, J, L), dtype=torch.uint8, device=dev),
        visited=torch.empty((Q, J, H), dtype=torch.int32, device=dev),
        counters=torch.empty((Q, J, NCTR), dtype=torch.int32, device=dev),
        B=B, metric=metric, team_size=team_size, V=V, policy=policy,
        stop_eps=float(stop_eps), kstop=int(kstop), stall_patience=int(stall_patience),
        crowd_frac=float(crowd_frac))
    if shared_cache and J > 1:
        # cache_slots (a power of two) replaces the closed-form size
        Hc = int(cache_slots) if cache_slots else cache_size(J, B, D)
        if Hc & (Hc - 1):
            raise ValueError(f"cache_slots must be a power of two, got {Hc}")
        # one allocation of (id, d) pairs: a claim and the distance later
        # stored into it share a cache line; cache_id / cache_d are views
        tab = torch.empty((Q, Hc, 2), dtype=torch.int32, device=dev)
        st.cache_id = tab[..., 0]
        st.cache_d = tab.view(torch.float32)[..., 1]
    else:
        st.cache_id = torch.empty((0, 0), dtype=torch.int32, device=dev)
        st.cache_d = torch.empty((0, 0), dtype=torch.float32, device=dev)
    st.exclusive = bool(exclusive and shared_cache and J > 1)
    st.bound = (torch.empty((Q,), dtype=torch.float32, device=dev)
                if (shared_bound and J > 1) else torch.empty((0,), dtype=torch.float32, device=dev))
    Hc = st.cache_id.shape[1] if st.cache_id.numel() else 0
    with torch.cuda.device(dev):
        call("swann_init_states", ptr(X), _DTYPES[X.dtype], X.shape[0], X.shape[1],
             ptr(Qv), Q, ptr(seeds), J, V, ptr(st.ids), ptr(st.dist), ptr(st.expanded),
             ptr(st.lineage), L, ptr(st.visited), H, ptr(st.counters), int(metric),
             int(team_size), ptr(st.cache_id), ptr(st.cache_d), Hc, ptr(st.bound),
             stream_of(dev))
    return st


def advance(X, G, Qv, state: SearchState, delta_expansions: int, active=None,
            codes=None) -> SearchState:
    """Advance every branch by up to delta more expansions, in place;
    swann/_engine.py:281-317.  `active` (int32 flattened q*J+j) restricts the
    launch to those branches.

    `codes` is an optional (codes, alpha, mu, margin), as `load_codes` or
    `swann_amd.codes.build_codes` give it: each neighbour that would be scored
    is first estimated from its sign code and its row is read only when the
    estimate leaves it within `margin` of the step's stop line.  It changes
    which distances are computed, so it is off unless asked for; a skip adds 1
    to `exhausted` (counter 3), exactly as the reference counts it."""
    if not (G.is_cuda and G.dtype == torch.int32 and G.is_contiguous() and G.dim() == 2):
        raise RuntimeError("G: contiguous cuda int32 [n, D]")
    _check_corpus(X, Qv)
    cd = al = cm = None
    cw, mg = 0, 0.0
    if codes is not None:
        cd, al, cm, mg = codes
        if not (cd.is_cuda and cd.dtype == torch.int32 and cd.is_contiguous() and cd.dim() == 2):
            raise RuntimeError("codes: contiguous cuda int32 [n, words]")
        if not (al.is_cuda and al.dtype == torch.float32 and al.is_contiguous()
                and cm.is_cuda and cm.dtype == torch.float32 and cm.is_contiguous()):
            raise RuntimeError("alpha and mu: contiguous cuda float32")
        if al.numel() != cd.shape[0] or cd.shape[0] != X.shape[0] or cm.numel() != X.shape[1]:
            raise RuntimeError("codes, alpha and mu must agree with the corpus")
        cw = cd.shape[1]
    Q, J, L = state.ids.shape
    H = state.visited.shape[-1]
    Hc = state.cache_id.shape[1] if state.cache_id is not None and state.cache_id.numel() else 0
    nact = 0
    if active is not None:
        active = active.to(device=X.device, dtype=torch.int32).contiguous()
        nact = active.numel()
        if nact == 0:
            return state
    dev = X.device
    with torch.cuda.device(dev):
        call("swann_advance", ptr(X), _DTYPES[X.dtype], X.shape[0], X.shape[1], ptr(G),
             G.shape[1], ptr(Qv), Q, J, ptr(state.ids), ptr(state.dist), ptr(state.expanded),
             ptr(state.lineage), L, ptr(state.visited), H, ptr(state.counters),
             int(state.metric), int(state.team_size), int(delta_expansions), int(state.B),
             int(state.policy), int(state.V), float(state.stop_eps), int(state.kstop),
             ptr(state.cache_id) if Hc else None, ptr(state.cache_d) if Hc else None, Hc,
             ptr(state.bound), int(bool(state.exclusive)), int(state.stall_patience),
             float(state.crowd_frac), ptr(active) if nact else None, nact,
             ptr(cd) if cw else None, cw, ptr(al) if cw else None, ptr(cm) if cw else None,
             float(mg), stream_of(dev))
    return state


def load_codes(data, name=None, margin=0.20, device="cuda"):
    """The sign code, its per-node scale and the corpus mean, as `advance`
    wants them (swann/_engine.py:320-337): codes_<name>.npy, alpha_<name>.npy
    and mu_<name>.npy under `data`; `name` defaults from manifest.json's
    metric ("1bit" for ip).  `margin` is in the corpus's distance units."""
    import json
    from pathlib import Path
    import numpy as np
    d = Path(data)
    if name is None:
        man = json.loads((d / "manifest.json").read_text())
        name = "1bit" if man["metric"].startswith("ip") else "int8"
    cd = torch.from_numpy(np.load(d / f"codes_{name}.npy")).to(device)
    al = torch.from_numpy(np.load(d / f"alpha_{name}.npy")).to(device)
    cm = torch.from_numpy(np.load(d / f"mu_{name}.npy")).to(device)
    return cd.contiguous(), al.contiguous(), cm.contiguous(), margin


def branch_topk(state: SearchState, k: int):
    """Per-branch best-k, straight off the sorted queue (swann/_engine.py:340-355)."""
    kk = min(k, state.ids.shape[-1])
    return state.ids[..., :kk].clone(), state.dist[..., :kk].clone()


def merge_branches(ids: torch.Tensor, dist: torch.Tensor, k: int, fused: bool = True):
    """Branch results -> one top-k per query, duplicates removed by id
    (swann/_engine.py:358-374).  The fused path is one kernel; the tensor path
    serves shapes the kernel refuses (more than 8192 candidates per query)."""
    if fused and ids.is_cuda and ids.dim() == 3 and ids.shape[1] * ids.shape[2] <= 8192:
        ids = ids.contiguous().to(torch.int32)
        dist = dist.contiguous().float()
        Q, V, kk = ids.shape
        oi = torch.empty((Q, k), dtype=torch.int32, device=ids.device)
        od = torch.empty((Q, k), dtype=torch.float32, device=ids.device)
        with torch.cuda.device(ids.device):
            call("swann_merge_branches", ptr(ids), ptr(dist), Q, V, kk, int(k), ptr(oi), ptr(od),
                 stream_of(ids.device))
        return oi, od
    return _merge_branches_tensor(ids, dist, k)


def _merge_branches_tensor(ids: torch.Tensor, dist: torch.Tensor, k: int):
    """The merge as tensor operations (swann/_engine.py:377-402)."""
    Q = ids.shape[0]
    flat_i = ids.reshape(Q, -1).to(torch.int64)
    flat_d = dist.reshape(Q, -1).clone()
    flat_d[flat_i < 0] = float("inf")
    order = torch.argsort(flat_i, dim=1, stable=True)
    sd = torch.gather(flat_d, 1, order)
    si = torch.gather(flat_i, 1, order)
    dup = torch.zeros_like(si, dtype=torch.bool)
    dup[:, 1:] = (si[:, 1:] == si[:, :-1]) & (si[:, 1:] >= 0)
    sd = sd.masked_fill(dup, float("inf"))
    si = si.masked_fill(dup, -1)
    kk = min(k, sd.shape[1])
    best_d, pos = torch.topk(sd, kk, dim=1, largest=False, sorted=True)
    best_i = torch.gather(si, 1, pos)
    best_i = best_i.masked_fill(torch.isinf(best_d), -1)
    return best_i.to(torch.int32), best_d


def advance_chunked(X, G, Qv, state: SearchState, total: int, chunk: int, codes=None) -> int:
    """Advance in chunks over the branches still running (swann/_engine.py:405-425).
    Returns the number of launches."""
    launches, spent = 0, 0
    while spent < total:
        alive = ((state.exhausted == 0) &
                 (state.expansions < state.B)).reshape(-1).nonzero().squeeze(1)
        if alive.numel() == 0:
            break
        step = min(chunk, total - spent)
        advance(X, G, Qv, state, step, active=alive.to(torch.int32).contiguous(), codes=codes)
        spent += step
        launches += 1
    return launches


def search(X, G, Qv, seeds, k=10, L=16, B=16, metric=METRIC_IP, team_size=32,
           policy=POLICY_BEST, stop_eps=-1.0, shared_cache=False, shared_bound=False,
           exclusive=False, stall_patience=0, crowd_frac=0.0, elide_visited=False, chunk=0,
           codes=None, check=None, cache_slots=None):
    """init -> advance(budget) -> per-branch best-k -> merged top-k
    (swann/_engine.py:428-447).  `check` overrides the global overflow guard:
    True checks synchronously, False skips it."""
    st = init_states(X, Qv, seeds, L=L, B=B, D=G.shape[1], metric=metric, team_size=team_size,
                     policy=policy, stop_eps=stop_eps, kstop=k, shared_cache=shared_cache,
                     shared_bound=shared_bound, exclusive=exclusive,
                     stall_patience=stall_patience, crowd_frac=crowd_frac,
                     elide_visited=elide_visited, cache_slots=cache_slots)
    if chunk:
        advance_chunked(X, G, Qv, st, B, chunk, codes=codes)
    else:
        advance(X, G, Qv, st, B, codes=codes)
    if _OVERFLOW_GUARD if check is None else check:
        st.check()
    bi, bd = branch_topk(st, k)
    ids, dist = merge_branches(bi, bd, k)
    return ids, dist, st


def library_version() -> str:
    return _lib.lib().swann_version().decode()
