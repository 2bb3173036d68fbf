"""Seed selection: the E nearest catalogue entries per query (swann/_select.py).

`select_nearest` runs on the GPU library: one distance GEMM over the
catalogue written to a workspace, then a per-row top-E kernel.  fp32 only:
gfx950 has no tf32, and the selected entries are exact up to ties.
"""
from __future__ import annotations

import torch

from ._engine import METRIC_IP, METRIC_L2  # noqa: F401
from ._lib import call, ptr, stream_of


def pool_vectors(Xg, pool_t):
    """The catalogue as its own fp32 matrix, held for the life of the index
    (swann/_select.py:54-61)."""
    return Xg[pool_t.long()].float().contiguous()


def select_nearest(Qg, Vp, E, metric=METRIC_IP, precision="fp32", slice_P=8192, workspace=None):
    """The E nearest rows of Vp per query, ascending; int64 [n, min(E, P)]
    (swann/_select.py:93-128).  `precision` and `slice_P` are accepted for
    interface compatibility; the GPU kernel is fp32 and unsliced."""
    del precision, slice_P
    return select_nearest_i32(Qg, Vp, E, metric, workspace).long()


def select_nearest_i32(Qg, Vp, E, metric=METRIC_IP, workspace=None):
    """select_nearest's entries as the kernel writes them, int32 [n, min(E, P)]
    (the search maps them to seeds without a widening copy)."""
    if not (Qg.is_cuda and Vp.is_cuda):
        raise RuntimeError("select_nearest: queries and catalogue must be on the GPU")
    Qg = Qg.float().contiguous()
    Vp = Vp.float().contiguous()
    n, P = Qg.shape[0], Vp.shape[0]
    E = min(int(E), P)
    out = torch.empty((n, E), dtype=torch.int32, device=Qg.device)
    if n == 0:
        return out
    need = int(_ws_size(n, P))
    if workspace is None or workspace.numel() < need:
        workspace = torch.empty(need, dtype=torch.uint8, device=Qg.device)
    with torch.cuda.device(Qg.device):
        call("swann_select_nearest", ptr(Qg), n, Qg.shape[1], ptr(Vp), P, E, int(metric),
             ptr(out), None, ptr(workspace), stream_of(Qg.device))
    return out


def _ws_size(n, P):
    from ._lib import lib
    return lib().swann_select_workspace_size(n, P)
