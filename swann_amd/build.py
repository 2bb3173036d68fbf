"""Graph construction: exact candidates, then a prune that keeps detours short
(swann/build.py).

The three stages keep the reference's signatures and run as gfx950 kernels:
`knn_candidates` is a fused distance-tile sweep with per-row top-C selection
(the n^2 scores never reach HBM), `robust_prune` builds each node's candidate
Gram in LDS and applies the sequential alpha rule, and `add_reverse` offers
every edge back to its target through a count / scan / scatter pass and
re-prunes.  Inputs and outputs live on the GPU.
"""
from __future__ import annotations

import torch

from ._lib import call, lib, ptr, stream_of

_METRICS = {"ip": 0, "l2": 1}


def _m(metric) -> int:
    if isinstance(metric, str):
        if metric not in _METRICS:
            raise ValueError(f"metric must be one of {sorted(_METRICS)}")
        return _METRICS[metric]
    return int(metric)


_DT = {torch.float32: 0, torch.float16: 1}


def _rows(X):
    """The corpus as the kernels read it: fp16 stays fp16 (its exact upcast is
    the reference's X.float()), anything else becomes fp32."""
    if not X.is_cuda:
        raise RuntimeError("the build runs on the GPU: move the vectors to cuda first")
    if X.dtype not in _DT:
        X = X.float()
    return X.contiguous()


@torch.no_grad()
def knn_candidates(Xg, C, chunk=4096, metric="ip"):
    """Exact top-C neighbours by the corpus's metric, self excluded
    (swann/build.py:28-43).  Returns (int32 [n, C], float32 [n, C]), ascending."""
    del chunk
    Xg = _rows(Xg)
    n, d = Xg.shape
    idx = torch.empty((n, C), dtype=torch.int32, device=Xg.device)
    dst = torch.empty((n, C), dtype=torch.float32, device=Xg.device)
    ws = torch.empty(int(lib().swann_sweep_workspace_size(n, d, _DT[Xg.dtype], C)),
                     dtype=torch.uint8, device=Xg.device)
    with torch.cuda.device(Xg.device):
        call("swann_build_sweep", ptr(Xg), _DT[Xg.dtype], n, d, _m(metric), int(C), ptr(idx),
             ptr(dst), ptr(ws), stream_of(Xg.device))
    return idx, dst


@torch.no_grad()
def robust_prune(Xg, cand, cdist, deg, alpha=1.2, chunk=4096, deg_per_node=None, metric="ip",
                 protect=None):
    """Keep a candidate only when no nearer kept neighbour detours to it
    (swann/build.py:46-91).  Returns int32 [n, width], -1 padded, where width
    is `deg`, or max(deg_per_node) when per-node degrees are given (node u then
    keeps at most deg_per_node[u]).  `protect` [n, C] bool exempts a
    candidate from the detour test (a mutual pair survives it)."""
    del chunk
    Xg = _rows(Xg)
    cand = cand.to(device=Xg.device, dtype=torch.int32).contiguous()
    cdist = cdist.to(device=Xg.device, dtype=torch.float32).contiguous()
    n, C = cand.shape
    width = int(deg)
    dpn = None
    if deg_per_node is not None:
        dpn = deg_per_node.to(device=Xg.device, dtype=torch.int32).contiguous()
        if dpn.shape != (n,):
            raise ValueError("deg_per_node must have one entry per node")
        width = int(dpn.max())
    prot = None
    if protect is not None:
        prot = protect.to(device=Xg.device, dtype=torch.bool).contiguous()
        if prot.shape != (n, C):
            raise ValueError("protect must be [n, C] like the candidates")
    out = torch.empty((n, width), dtype=torch.int32, device=Xg.device)
    wsb = int(lib().swann_prune_workspace_size(n, Xg.shape[1], _DT[Xg.dtype]))
    ws = torch.empty(wsb, dtype=torch.uint8, device=Xg.device) if wsb else None
    with torch.cuda.device(Xg.device):
        call("swann_build_prune", ptr(Xg), _DT[Xg.dtype], n, Xg.shape[1], _m(metric), ptr(cand),
             ptr(cdist), int(C), width, float(alpha), ptr(dpn), ptr(prot), ptr(out), ptr(ws),
             stream_of(Xg.device))
    return out


@torch.no_grad()
def add_reverse(Xg, G, deg, chunk=2048, alpha=1.2, max_in=64, deg_per_node=None, metric="ip"):
    """Offer every edge back to its target, then re-prune the union per node
    (swann/build.py:94-150).  With `deg_per_node` the width is its maximum and
    node u keeps at most deg_per_node[u]."""
    del chunk
    Xg = _rows(Xg)
    G = G.to(device=Xg.device, dtype=torch.int32).contiguous()
    n, d = Xg.shape
    width = int(deg)
    dpn = None
    if deg_per_node is not None:
        dpn = deg_per_node.to(device=Xg.device, dtype=torch.int32).contiguous()
        width = int(dpn.max())
    if G.shape[1] != width:
        raise ValueError(f"G has {G.shape[1]} columns, the row width is {width}")
    out = torch.empty((n, width), dtype=torch.int32, device=Xg.device)
    ws = torch.empty(int(lib().swann_reverse_workspace_size(n, width, max_in)),
                     dtype=torch.uint8, device=Xg.device)
    with torch.cuda.device(Xg.device):
        call("swann_build_reverse", ptr(Xg), _DT[Xg.dtype], n, d, _m(metric), ptr(G), width,
             float(alpha), int(max_in), ptr(dpn), ptr(out), ptr(ws), stream_of(Xg.device))
    return out


@torch.no_grad()
def build_graph(X, metric: str = "ip", degree: int = 96, candidates: int = 128,
                alpha: float = 1.2):
    """Return an (n, degree) int32 neighbour table on the GPU (swann/build.py:153-171)."""
    if X.device.type != "cuda":
        X = X.cuda()
    Xg = _rows(X)
    cand, cdist = knn_candidates(Xg, candidates, metric=metric)
    G = robust_prune(Xg, cand, cdist, degree, alpha=alpha, metric=metric)
    G = add_reverse(Xg, G, degree, alpha=alpha, metric=metric)
    return G.to(torch.int32).contiguous()
