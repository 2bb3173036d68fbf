"""The public interface: build an index over vectors, then search it
(swann/index.py).

    import swann                  # or: import swann_amd as swann
    index = swann.Index.build(X, metric="ip")      # X: (n, d) float32 or float16
    ids, dist = index.search(Q, k=10)

Same classes, signatures, knobs and file format as the reference.  Two
deliberate differences: there is no 65535-query cap (the kernels run on a
1-D grid), and the overflow check no longer costs its own host
synchronisation: it is computed on the device with the search and read after
the results' own copy back.

For small batches, where launch overhead is a large part of the latency,
`Index.capture(batch)` records the whole search once as a HIP graph and
replays it (`CapturedSearch`).
"""
from __future__ import annotations

import json
from dataclasses import dataclass
from pathlib import Path

import numpy as np
import torch

from . import _engine as E
from . import _select as S

METRICS = {"ip": E.METRIC_IP, "l2": E.METRIC_L2}


@dataclass
class SearchConfig:
    """Knobs, with the reference's defaults (swann/index.py:26-45).

    branches  trajectories one query is split into (workgroups per query).
    queue     width of each branch's candidate queue.
    budget    cap on expansions per branch; `stop_eps` usually binds first.
    stop_eps  stop a branch once its best candidate is worse than the query's
              current k-th answer by this fraction; negative disables it.
    team      lanes cooperating on one distance (4, 8, 16, 32 or 64).
    """
    branches: int = 32
    queue: int = 12
    budget: int = 64
    stop_eps: float = 0.05
    team: int = 16
    k: int = 10


class Index:
    """A proximity graph plus the vectors it indexes, resident on one GPU."""

    def __init__(self, vectors: torch.Tensor, graph: torch.Tensor, metric: str = "ip",
                 catalogue: torch.Tensor | None = None, catalogue_size: int = 4096,
                 seed: int = 0):
        if vectors.device.type != "cuda":
            raise ValueError("vectors must already be on the GPU")
        if vectors.dtype not in (torch.float32, torch.float16):
            raise ValueError("vectors must be float32 or float16")
        if metric not in METRICS:
            raise ValueError(f"metric must be one of {sorted(METRICS)}")
        self.X = vectors.contiguous()
        self.G = graph.to(device=self.X.device, dtype=torch.int32).contiguous()
        if self.G.dim() != 2 or self.G.shape[0] != self.X.shape[0]:
            raise ValueError(f"graph must be [n, degree] with n = {self.X.shape[0]}")
        self.metric = metric
        self._m = METRICS[metric]
        if catalogue is None:
            n = self.X.shape[0]
            rng = np.random.default_rng(seed)
            pick = np.sort(rng.permutation(n)[:min(catalogue_size, n)])
            catalogue = torch.from_numpy(pick.astype(np.int64)).to(self.X.device)
        self.catalogue = catalogue.to(device=self.X.device, dtype=torch.int64)
        self._cat = S.pool_vectors(self.X, self.catalogue)
        self._cat_ids = self.catalogue.to(torch.int32)     # seeds are int32 row ids
        self._flag = None

    # -- construction ----------------------------------------------------
    @classmethod
    def build(cls, vectors, metric: str = "ip", degree: int = 96, candidates: int = 128,
              alpha: float = 1.2, **kw) -> "Index":
        """Build a graph over `vectors` on the GPU (sweep, prune, reverse)."""
        from .build import build_graph
        X = _on_gpu(vectors)
        G = build_graph(X, metric=metric, degree=degree, candidates=candidates, alpha=alpha)
        return cls(X, G, metric=metric, **kw)

    # -- search ----------------------------------------------------------
    def search_async(self, queries, k: int = 10, config: SearchConfig | None = None,
                     **overrides):
        """Launch a search and return device tensors (ids, dist, state,
        overflow) without synchronising; `overflow` is a device scalar."""
        cfg = config or SearchConfig(k=k)
        for key, value in overrides.items():
            if not hasattr(cfg, key):
                raise TypeError(f"unknown search option {key!r}")
            setattr(cfg, key, value)
        Q = _on_gpu(queries).float().contiguous()
        return self._search_device(Q, k, cfg)

    def _search_device(self, Q: torch.Tensor, k: int, cfg: SearchConfig):
        """select -> seeds -> init -> advance -> merge -> overflow,
        all stream-ordered device work with no host synchronisation (so it can
        be captured)."""
        entries = S.select_nearest_i32(Q, self._cat, cfg.branches, metric=self._m)
        seeds = torch.index_select(self._cat_ids, 0, entries.view(-1)).view(entries.shape)
        bits, slots = self._claims(Q.shape[0], cfg)
        ids, dist, st = E.search(
            self.X, self.G, Q, seeds, k=k, L=cfg.queue, B=cfg.budget, metric=self._m,
            team_size=cfg.team, stop_eps=cfg.stop_eps, shared_cache=True, shared_bound=True,
            exclusive=True, elide_visited=True, check=False,
            cache_slots=None if bits else slots, claim_bits=bits)
        return ids, dist, st, st.overflow()

    def _claims(self, nq: int, cfg: SearchConfig) -> tuple[bool, int]:
        """How the branches of a query share their claims: (True, bits) for
        one claim bit per corpus row, (False, slots) for the reference's
        per-query table of (id, d) pairs (swann/_engine.py:186-198).  Under
        exclusive claims a row found in the table is never a candidate again,
        so the bits decide the same as a table whose probes never fail, in
        n / 8 bytes a query, cleared and probed in L2 rather than HBM (at C3:
        128 KiB a query against the table's 4 MiB, init 2 ms instead of 9,
        the same advance time at 64 branches and 6% less at 32).  Bits are
        taken when the batch's fit a quarter of the free device memory.

        Otherwise the table: the reference sizes it for a quarter of the rows
        the branches could score; a table that full runs long probe chains, so
        this takes up to four times that (the closed form with share 1, capped
        at 2^20 slots), halved until the batch's tables fit a quarter of the
        free device memory, and never below the reference's size.  Decided
        once per (batch, branches, budget), so repeated and captured searches
        keep one layout."""
        key = (nq, cfg.branches, cfg.budget)
        got = self._layouts.get(key) if hasattr(self, "_layouts") else None
        if got is None:
            free, _ = torch.cuda.mem_get_info(self.X.device)
            nbits = E.next_pow2(max(self.X.shape[0], 32))
            got = ((True, nbits) if nq * nbits // 8 <= free // 4 else
                   (False, self._table_size(nq, cfg, free)))
            if not hasattr(self, "_layouts"):
                self._layouts = {}
            self._layouts[key] = got
        return got

    def _table_size(self, nq: int, cfg, free: int | None = None) -> int:
        """Slots of each query's (id, d) table (the layout the sign-code
        filter needs, and the fallback of `_claims`)."""
        if free is None:
            free, _ = torch.cuda.mem_get_info(self.X.device)
        D = self.G.shape[1]
        base = E.cache_size(cfg.branches, cfg.budget, D)
        hc = E.cache_size(cfg.branches, cfg.budget, D, share=1.0)
        while hc > base and nq * hc * 8 > free // 4:
            hc //= 2
        return max(hc, base)

    def capture(self, batch: int, k: int = 10, config: SearchConfig | None = None,
                **overrides) -> "CapturedSearch":
        """A search of exactly `batch` queries recorded as one HIP graph; see
        `CapturedSearch`.  The knobs are fixed at capture time."""
        cfg = config or SearchConfig(k=k)
        for key, value in overrides.items():
            if not hasattr(cfg, key):
                raise TypeError(f"unknown search option {key!r}")
            setattr(cfg, key, value)
        return CapturedSearch(self, int(batch), k, cfg)

    def search(self, queries, k: int = 10, config: SearchConfig | None = None, **overrides):
        """Return (ids, distances), each (nq, k), as numpy arrays
        (swann/index.py:86-110)."""
        ids, dist, st, over = self.search_async(queries, k=k, config=config, **overrides)
        if self._flag is None:
            self._flag = torch.empty((), dtype=torch.int32, pin_memory=True)
        flag = self._flag
        if E._OVERFLOW_GUARD:
            flag.copy_(over, non_blocking=True)
        ids_h, dist_h = ids.cpu().numpy(), dist.cpu().numpy()     # synchronises
        if E._OVERFLOW_GUARD and int(flag):
            raise RuntimeError(f"visited table overflowed ({int(flag)} failed inserts)")
        return ids_h, dist_h

    # -- persistence -----------------------------------------------------
    def save(self, path) -> None:
        """Write graph.npy, catalogue.npy and index.json (swann/index.py:113-122)."""
        path = Path(path)
        path.mkdir(parents=True, exist_ok=True)
        np.save(path / "graph.npy", self.G.cpu().numpy())
        np.save(path / "catalogue.npy", self.catalogue.cpu().numpy())
        (path / "index.json").write_text(json.dumps(
            {"metric": self.metric, "n": int(self.X.shape[0]), "d": int(self.X.shape[1]),
             "degree": int(self.G.shape[1])}, indent=2))

    @classmethod
    def load(cls, path, vectors) -> "Index":
        path = Path(path)
        meta = json.loads((path / "index.json").read_text())
        G = torch.from_numpy(np.load(path / "graph.npy", allow_pickle=False)).cuda()
        cat = torch.from_numpy(np.load(path / "catalogue.npy", allow_pickle=False)).cuda()
        return cls(_on_gpu(vectors), G, metric=meta["metric"], catalogue=cat)

    def __repr__(self) -> str:
        n, d = self.X.shape
        return (f"Index(n={n:,}, d={d}, degree={self.G.shape[1]}, "
                f"metric={self.metric!r}, dtype={self.X.dtype})")


def _on_gpu(a) -> torch.Tensor:
    """`a` -- a numpy array, a nested list or a tensor on any device -- as a
    contiguous tensor on the GPU (the current device unless it is already on
    one)."""
    if isinstance(a, torch.Tensor):
        return (a if a.is_cuda else a.to("cuda")).contiguous()
    return torch.as_tensor(np.ascontiguousarray(a), device="cuda")


class CapturedSearch:
    """One search of a fixed batch size, recorded once as a HIP graph
    (`torch.cuda.CUDAGraph`) and replayed.

    Every kernel of the search (selection GEMM and top-k, seed gather, branch
    init, advance, merge of the branches' best k, overflow count) is one node; the
    state, table, workspace and outputs live in the graph's private memory
    pool and are reused by every replay.  The overflow guard is not applied:
    `overflow` is a device scalar the caller may read when it likes.  Nothing
    in the captured work clears memory with a memset node; every clear is a
    kernel.

        cs = index.capture(8, k=10, branches=32)
        ids, dist = cs.run(Q8)          # device tensors, valid until the next run
    """

    def __init__(self, index: Index, batch: int, k: int, cfg: SearchConfig, warmup: int = 2):
        if batch < 1:
            raise ValueError("batch must be >= 1")
        dev = index.X.device
        self.index, self.batch, self.k, self.cfg = index, batch, k, cfg
        self.queries = torch.zeros((batch, index.X.shape[1]), dtype=torch.float32, device=dev)
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            for _ in range(warmup):
                index._search_device(self.queries, k, cfg)
        torch.cuda.current_stream(dev).wait_stream(side)
        torch.cuda.synchronize(dev)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.ids, self.dist, self.state, self.overflow = index._search_device(
                self.queries, k, cfg)

    def run(self, queries) -> tuple[torch.Tensor, torch.Tensor]:
        """Copy `queries` (batch x d) into the graph's input and replay it on
        the current stream.  Returns the graph's (ids, dist) device tensors,
        overwritten by the next run."""
        q = _on_gpu(queries)
        if q.shape != self.queries.shape:
            raise ValueError(f"captured for queries of shape {tuple(self.queries.shape)}, "
                             f"got {tuple(q.shape)}")
        self.queries.copy_(q, non_blocking=True)
        self.graph.replay()
        return self.ids, self.dist
