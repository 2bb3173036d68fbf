"""The offline graph builder: candidates, prune, reverse, and the extras that
spend degree where the search needs it (offline/build_graph.py).

    python -m swann_amd.offline --data DIR [--D 64] [--cand 128] [--fill bridge]
        [--cand-graph G_other.npy] [--pool-boost 16] [--mutual 8] [--min-in 8] ...

Reads DIR/manifest.json and DIR/X.npy, writes DIR/<out> (int32 [n, D]),
DIR/<out stem>_deg.npy and DIR/<out stem>.json, as the reference does.  Every
stage runs on the GPU library; the functions keep the reference's names and
arguments:

  candidates_from_graph  build_graph.py:63-91
  mutual_rank            build_graph.py:93-131
  fill_degree            build_graph.py:132-200
  enforce_min_in         build_graph.py:203-294
  pool_degrees           the --pool-boost rule of build_graph.py:339-346
"""
from __future__ import annotations

import argparse
import json
import time
from pathlib import Path

import numpy as np
import torch

from . import build as B
from ._lib import call, lib, ptr, stream_of

_DT = {torch.float32: 0, torch.float16: 1}
_RULES = {"near": 0, "far": 1, "bridge": 2}


def _metric(m):
    return {"ip": 0, "l2": 1}[m] if isinstance(m, str) else int(m)


@torch.no_grad()
def candidates_from_graph(Xg, Gc, C, metric="ip", chunk=1024):
    """Candidates from an existing graph with exact distances: the first C
    entries of each row, -1 and self at 3.4e38, ascending (ties keep their
    column order).  Returns (idx int32 [n, C], dist fp32 [n, C])."""
    del chunk
    Xg = B._rows(Xg)
    Gc = Gc.to(device=Xg.device, dtype=torch.int32).contiguous()
    n = Xg.shape[0]
    C = min(int(C), Gc.shape[1])
    idx = torch.empty((n, C), dtype=torch.int32, device=Xg.device)
    dst = torch.empty((n, C), dtype=torch.float32, device=Xg.device)
    with torch.cuda.device(Xg.device):
        call("swann_candidates_from_graph", ptr(Xg), _DT[Xg.dtype], n, Xg.shape[1],
             _metric(metric), ptr(Gc), Gc.shape[1], C, ptr(idx), ptr(dst), stream_of(Xg.device))
    return idx, dst


@torch.no_grad()
def mutual_rank(cand, M, chunk=2048):
    """bool [n, C]: entry (u, j) is set when j < M and u is among the first M
    candidates of cand[u, j] -- the pair is mutual within rank M."""
    del chunk
    cand = cand.to(torch.int32).contiguous()
    n, C = cand.shape
    out = torch.empty((n, C), dtype=torch.bool, device=cand.device)
    with torch.cuda.device(cand.device):
        call("swann_mutual_rank", ptr(cand), n, C, int(M), ptr(out), stream_of(cand.device))
    return out


@torch.no_grad()
def fill_degree(G, cand, rule="bridge", chunk=1024, deg_two=None):
    """Spend the slots the prune left empty on candidates it refused: the
    nearest ("near"), the farthest ("far"), or the nearest with no two-hop
    path back through the kept graph ("bridge").  Chunks of `chunk` nodes in
    order, each seeing the earlier chunks' fills.  Returns a new graph."""
    del deg_two
    if rule not in _RULES:
        raise ValueError(f"rule must be one of {sorted(_RULES)}")
    G = G.to(torch.int32).contiguous()
    cand = cand.to(device=G.device, dtype=torch.int32).contiguous()
    n, W = G.shape
    out = torch.empty_like(G)
    ws = torch.empty((int(lib().swann_fill_workspace_size(n, W, int(chunk))),), dtype=torch.uint8,
                     device=G.device)
    with torch.cuda.device(G.device):
        call("swann_fill_degree", ptr(G), n, W, ptr(cand), cand.shape[1], _RULES[rule],
             int(chunk), ptr(out), ptr(ws), stream_of(G.device))
    return out


@torch.no_grad()
def enforce_min_in(Xg, G, cand, min_in, metric="ip", rounds=4):
    """A floor on every node's in-degree at a fixed edge count, in place on G
    (returned).  A weak node is offered, column by column of its candidate
    list, to that candidate, which drops its farthest edge whose head stays
    above the floor; several offers to one target in a column go to the
    lowest node id (the reference's choice there follows an unstable sort)."""
    del Xg, metric
    if not G.is_contiguous() or G.dtype != torch.int32:
        raise ValueError("G must be a contiguous int32 tensor (it is updated in place)")
    cand = cand.to(device=G.device, dtype=torch.int32).contiguous()
    n, W = G.shape
    ws = torch.empty((int(lib().swann_min_in_workspace_size(n)),), dtype=torch.uint8,
                     device=G.device)
    with torch.cuda.device(G.device):
        call("swann_enforce_min_in", ptr(G), n, W, ptr(cand), cand.shape[1], int(min_in),
             int(rounds), ptr(ws), stream_of(G.device))
    return G


def pool_degrees(n, D, pool, boost, cand, device="cuda"):
    """Per-node degrees for --pool-boost: D everywhere, min(D + boost,
    min(cand, 128)) on the entry-pool nodes."""
    dpn = torch.full((n,), D, dtype=torch.int32, device=device)
    pi = torch.as_tensor(np.asarray(pool, dtype=np.int64), device=device)
    dpn[pi] = min(D + boost, min(cand, 128))
    return dpn


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--data", type=Path, required=True)
    ap.add_argument("--D", type=int, default=64, help="target graph out-degree")
    ap.add_argument("--cand", type=int, default=128)
    ap.add_argument("--fill", default=None, choices=["near", "far", "bridge"])
    ap.add_argument("--cand-graph", default=None,
                    help="take candidates from this graph inside --data instead of the sweep")
    ap.add_argument("--pool-boost", type=int, default=0)
    ap.add_argument("--pool-name", default="random4k")
    ap.add_argument("--mutual", type=int, default=0)
    ap.add_argument("--min-in", type=int, default=0)
    ap.add_argument("--min-in-rounds", type=int, default=6)
    ap.add_argument("--alpha", type=float, default=1.2)
    ap.add_argument("--metric", default=None, choices=["ip", "l2"])
    ap.add_argument("--out", default="G_ours.npy")
    a = ap.parse_args(argv)

    man = json.loads((a.data / "manifest.json").read_text())
    metric = a.metric or ("ip" if man["metric"].startswith("ip") else "l2")
    X = np.load(a.data / "X.npy")
    Xg = torch.from_numpy(X).cuda()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    if a.cand_graph:
        Gc = torch.from_numpy(np.load(a.data / a.cand_graph)).cuda()
        cand, cdist = candidates_from_graph(Xg, Gc, a.cand, metric=metric)
        del Gc
    else:
        cand, cdist = B.knn_candidates(Xg, a.cand, metric=metric)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    dpn = None
    if a.pool_boost:
        pool = np.load(a.data / "pools" / f"pool_{a.pool_name}.npy")
        dpn = pool_degrees(Xg.shape[0], a.D, pool, a.pool_boost, a.cand)
    prot = mutual_rank(cand, a.mutual) if a.mutual else None
    G = B.robust_prune(Xg, cand, cdist, a.D, alpha=a.alpha, deg_per_node=dpn, metric=metric,
                       protect=prot)
    torch.cuda.synchronize()
    t2 = time.perf_counter()
    G = B.add_reverse(Xg, G, a.D, alpha=a.alpha, deg_per_node=dpn, metric=metric)
    if a.min_in:
        G = enforce_min_in(Xg, G, cand, a.min_in, metric=metric, rounds=a.min_in_rounds)
    if a.fill:
        G = fill_degree(G, cand, rule=a.fill)
    torch.cuda.synchronize()
    t3 = time.perf_counter()
    Gc = G.cpu().numpy().astype(np.int32)
    filled = (Gc >= 0).sum(1)
    stages = {"candidates": t1 - t0, "prune": t2 - t1, "reverse+extras": t3 - t2}
    print("[build] " + ", ".join(f"{k} {v:.2f} s" for k, v in stages.items()) +
          f" (total {t3 - t0:.2f} s)")
    print(f"[build] out-degree range {filled.min()}..{filled.max()}, "
          f"median {int(np.median(filled))}")
    np.save(a.data / a.out, Gc)
    np.save(a.data / (Path(a.out).stem + "_deg.npy"), filled.astype(np.int32))
    (a.data / (Path(a.out).stem + ".json")).write_text(json.dumps(
        dict(deg=a.D, cand=a.cand, candidates=("graph" if a.cand_graph else "exact"),
             alpha=a.alpha, metric=metric, candidate_graph=a.cand_graph,
             pool_boost=a.pool_boost, min_in=a.min_in, mutual=a.mutual, fill=a.fill,
             seconds=round(t3 - t0, 2),
             stage_seconds=dict(candidates=round(t1 - t0, 2), prune=round(t2 - t1, 2),
                                reverse=round(t3 - t2, 2))), indent=2))
    print(f"[build] graph saved to {a.data / a.out}")


if __name__ == "__main__":
    main()
