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
    table_slots: int = 0     # Hc: table slots, or claim bits, a query (0 = no table)

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
                           bound=c(self.bound), exclusive=self.exclusive,
                           table_slots=self.table_slots)


def ctypes_ptr(t):
    import ctypes
    return ctypes.c_void_p(t.data_ptr())


# `search` and `Index.search` read the branches' failed-insert counters after
# every search and raise if any is nonzero.  A caller whose table sizes are
# known to fit can switch that off and read `state.overflow()` when it likes.
_OVERFLOW_GUARD = True


def overflow_guard(on: bool) -> bool:
    """Enable or disable the overflow check made after every search; the
    previous setting is returned (swann/_engine.py:203-216)."""
    global _OVERFLOW_GUARD
    previous = _OVERFLOW_GUARD
    _OVERFLOW_GUARD = bool(on)
    return previous


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
                elide_visited=False, cache_slots=None, claim_bits=False) -> SearchState:
    """One state per (query, branch); swann/_engine.py:219-278.

    `seeds` is int32 [Q, J] (one entry per branch) or [Q, J, V] (V entries
    sharing one branch).  -1 is an empty slot.

    `claim_bits` replaces the shared table with one claim bit per corpus row
    (exclusive claims only, and no sign codes in `advance`): under exclusive
    claims a row found in the table is never a candidate again, so its cached
    distance is never used, and the bit decides the same.  It takes n / 8
    bytes a query instead of the table's 8 bytes a slot."""
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
    if claim_bits and not (exclusive and shared_cache and J > 1):
        raise ValueError("claim_bits needs exclusive claims over a shared table (J > 1)")
    if claim_bits:
        Hc = next_pow2(max(X.shape[0], 32))
        st.cache_id = torch.empty((Q, Hc // 32), dtype=torch.int32, device=dev)
        st.cache_d = torch.empty((0, 0), dtype=torch.float32, device=dev)
        st.table_slots = Hc
    elif shared_cache and J > 1:
        # cache_slots (a power of two) replaces the closed-form size
        Hc = int(cache_slots) if cache_slots else cache_size(J, B, D)
        if Hc & (Hc - 1):
            raise ValueError(f"cache_slots must be a power of two, got {Hc}")
        # one allocation of (id, d) pairs: a claim and the distance later
        # stored into it share a cache line; cache_id / cache_d are views
        tab = torch.empty((Q, Hc, 2), dtype=torch.int32, device=dev)
        st.cache_id = tab[..., 0]
        st.cache_d = tab.view(torch.float32)[..., 1]
        st.table_slots = Hc
    else:
        st.cache_id = torch.empty((0, 0), dtype=torch.int32, device=dev)
        st.cache_d = torch.empty((0, 0), dtype=torch.float32, device=dev)
    st.exclusive = bool(exclusive and shared_cache and J > 1)
    st.bound = (torch.empty((Q,), dtype=torch.float32, device=dev)
                if (shared_bound and J > 1) else torch.empty((0,), dtype=torch.float32, device=dev))
    Hc = st.table_slots
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
    Hc = state.table_slots
    if not Hc and state.cache_id is not None and state.cache_id.numel() \
            and state.cache_d is not None and state.cache_d.numel():
        Hc = state.cache_id.shape[1]        # a state assembled by hand: the table's width
    if Hc and codes is not None and (state.cache_d is None or state.cache_d.numel() == 0):
        raise ValueError("sign codes need the shared table: init_states(claim_bits=False)")
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


_CODE_FILES = ("codes", "alpha", "mu")


def load_codes(data, name=None, margin=0.20, device="cuda"):
    """`(codes, alpha, mu, margin)` for `advance(codes=...)`, read from
    codes_<name>.npy, alpha_<name>.npy and mu_<name>.npy in the corpus
    directory `data` (swann/_engine.py:320-337).  Without `name`, the corpus's
    manifest.json decides: "1bit" for an ip metric, "int8" otherwise.
    `margin` is in the corpus's distance units."""
    import json
    from pathlib import Path
    import numpy as np
    root = Path(data)
    if name is None:
        metric = json.loads((root / "manifest.json").read_text())["metric"]
        name = "1bit" if metric.startswith("ip") else "int8"
    codes, alpha, mu = (
        torch.as_tensor(np.ascontiguousarray(np.load(root / f"{stem}_{name}.npy",
                                                     allow_pickle=False)), device=device)
        for stem in _CODE_FILES)
    return codes, alpha, mu, margin


def branch_topk(state: SearchState, k: int):
    """Per-branch best-k, straight off the sorted queue (swann/_engine.py:340-355)."""
    kk = min(k, state.ids.shape[-1])
    return state.ids[..., :kk].clone(), state.dist[..., :kk].clone()


def merge_branches(ids: torch.Tensor, dist: torch.Tensor, k: int, fused: bool = True):
    """Branch results [Q, V, kk] -> one top-k per query in (distance, id) order,
    duplicates removed by id (swann/_engine.py:358-374).  One kernel serves
    every shape (a successor walk over (distance, id) keys, no V*kk limit);
    `fused` is accepted for the reference's signature and changes nothing."""
    if not (ids.is_cuda and dist.is_cuda) or ids.dim() != 3 or tuple(dist.shape) != tuple(ids.shape):
        raise RuntimeError("merge_branches: ids and dist must be cuda tensors of shape [Q, V, kk]")
    ids = ids.contiguous().to(torch.int32)
    dist = dist.contiguous().float()
    Q, V, kk = ids.shape
    oi = torch.empty((Q, k), dtype=torch.int32, device=ids.device)
    od = torch.empty((Q, k), dtype=torch.float32, device=ids.device)
    with torch.cuda.device(ids.device):
        call("swann_merge_branches", ptr(ids), ptr(dist), Q, V, kk, int(k), ptr(oi), ptr(od),
             stream_of(ids.device))
    return oi, od


def merge_state(state: SearchState, k: int):
    """branch_topk then merge_branches in one launch (swann/_engine.py:340-374):
    the merge reads each branch's first min(k, L) slots straight from the
    state's sorted queues, so no [Q, J, kk] copy is made.  Same output as
    merge_branches(*branch_topk(state, k), k)."""
    Q, J, L = state.ids.shape
    kk = min(k, L)
    if not (1 <= k <= J * kk):
        raise RuntimeError(f"merge_state: k must be in 1..{J * kk}, got {k}")
    if not (state.ids.is_cuda and state.dist.is_cuda and state.ids.dtype == torch.int32
            and state.dist.dtype == torch.float32 and tuple(state.dist.shape) == (Q, J, L)):
        raise RuntimeError("merge_state: the queues must be cuda int32 ids and float32 "
                           "distances of one shape [Q, J, L]")
    if not (state.ids.is_contiguous() and state.dist.is_contiguous()):
        raise RuntimeError("merge_state: the state's queues must be contiguous")
    oi = torch.empty((Q, k), dtype=torch.int32, device=state.ids.device)
    od = torch.empty((Q, k), dtype=torch.float32, device=state.ids.device)
    with torch.cuda.device(state.ids.device):
        call("swann_merge_branches_strided", ptr(state.ids), ptr(state.dist), Q, J, kk, L,
             int(k), ptr(oi), ptr(od), stream_of(state.ids.device))
    return oi, od


def _live_branches(state: SearchState) -> torch.Tensor:
    """Flattened indices q*J + j (int32, on the state's device) of the branches
    that still have an unexpanded candidate and budget left."""
    done = state.exhausted.ne(0) | state.expansions.ge(state.B)
    return torch.nonzero(done.logical_not().flatten()).flatten().to(torch.int32)


def advance_chunked(X, G, Qv, state: SearchState, total: int, chunk: int, codes=None) -> int:
    """Spend up to `total` expansions per branch in launches of `chunk`, each
    over only the branches still live, so a finished branch gives its slot on
    the GPU to one that is not (swann/_engine.py:405-425).  Stops early once
    no branch is live; returns the number of launches."""
    if chunk < 1:
        raise ValueError(f"chunk must be >= 1, got {chunk}")
    launches = 0
    for start in range(0, total, chunk):
        live = _live_branches(state)
        if live.numel() == 0:
            break
        advance(X, G, Qv, state, min(chunk, total - start), active=live, codes=codes)
        launches += 1
    return launches


def search(X, G, Qv, seeds, k=10, L=16, B=16, metric=METRIC_IP, team_size=32,
           policy=POLICY_BEST, stop_eps=-1.0, shared_cache=False, shared_bound=False,
           exclusive=False, stall_patience=0, crowd_frac=0.0, elide_visited=False, chunk=0,
           codes=None, check=None, cache_slots=None, claim_bits=False):
    """init -> advance(budget) -> merged top-k of the branches' best k, read
    from their queues in place (swann/_engine.py:428-447).  `check` overrides
    the global overflow guard: True checks synchronously, False skips it."""
    st = init_states(X, Qv, seeds, L=L, B=B, D=G.shape[1], metric=metric, team_size=team_size,
                     policy=policy, stop_eps=stop_eps, kstop=k, shared_cache=shared_cache,
                     shared_bound=shared_bound, exclusive=exclusive,
                     stall_patience=stall_patience, crowd_frac=crowd_frac,
                     elide_visited=elide_visited, cache_slots=cache_slots,
                     claim_bits=claim_bits)
    if chunk:
        advance_chunked(X, G, Qv, st, B, chunk, codes=codes)
    else:
        advance(X, G, Qv, st, B, codes=codes)
    if _OVERFLOW_GUARD if check is None else check:
        st.check()
    ids, dist = merge_state(st, k)
    return ids, dist, st


def library_version() -> str:
    return _lib.lib().swann_version().decode()
