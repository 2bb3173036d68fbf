"""The reference-side binding documented for a reference maintainer (the
ctypes `ext()` block of the repository's integration notes, replacing the
reference's JIT extension, swann/_engine.py:42-63) --
executed as written (only the library's path is filled in) and driven with the
reference's own calling convention: state tensors allocated by the caller,
empty tensors for disabled features (swann/_engine.py:251-306).  Its results
must equal swann_amd._engine's, bit for bit, on a deterministic configuration
(no claims, no bound)."""
import re
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

from conftest import ROOT, gaussian
from test_oracle_helpers import knn_graph

pytestmark = pytest.mark.gpu

E = pytest.importorskip("swann_amd._engine")
from swann_amd import _lib  # noqa: E402


def note(*a):
    print("[case]", *a, flush=True)
    sys.stdout.flush()


def load_shim():
    text = (ROOT / "INTEGRATION.md").read_text()
    block = re.search(r"```python\n(# swann/_engine.py — replacement for ext\(\).*?)```", text,
                      re.S)
    assert block, "INTEGRATION.md no longer holds the ext() shim"
    code = block.group(1).replace('ctypes.CDLL("libswann_amd.so")',
                                  f'ctypes.CDLL({str(_lib.LIB_PATH)!r})')
    ns = {}
    exec(compile(code, "INTEGRATION.md:ext()", "exec"), ns)
    return ns["ext"]()


def empty(dtype):
    return torch.empty(0, dtype=dtype, device="cuda")


@pytest.mark.parametrize("dtype,metric,cache", [("f32", 0, False), ("f16", 0, True),
                                                ("f32", 1, True)])
def test_reference_binding_equals_the_engine(dtype, metric, cache):
    note("shim", dtype, metric, cache)
    ext = load_shim()
    X = gaussian(3000, 64, 41, metric == 0)
    G = knn_graph(X, 24, metric)
    if dtype == "f16":
        X = X.astype(np.float16)
    Q = gaussian(12, 64, 42, metric == 0)
    seeds = np.random.default_rng(43).integers(0, 3000, (12, 6)).astype(np.int32)
    Xg = torch.from_numpy(X).cuda()
    Gg = torch.from_numpy(G).cuda()
    Qg = torch.from_numpy(Q).cuda()
    Sg = torch.from_numpy(seeds).cuda()
    nq, J, L, B, team, k = 12, 6, 16, 20, 16, 10
    H = E.visited_size(B, G.shape[1])
    Hc = E.cache_size(J, B, G.shape[1]) if cache else 0

    # the reference's allocation (swann/_engine.py:251-274), then ext() calls
    dev = "cuda"
    ids = torch.empty((nq, J, L), dtype=torch.int32, device=dev)
    dist = torch.empty((nq, J, L), dtype=torch.float32, device=dev)
    expd = torch.empty((nq, J, L), dtype=torch.uint8, device=dev)
    lin = torch.empty((nq, J, L), dtype=torch.uint8, device=dev)
    visited = torch.empty((nq, J, H), dtype=torch.int32, device=dev)
    counters = torch.empty((nq, J, E.NCTR), dtype=torch.int32, device=dev)
    cache_id = (torch.empty((nq, Hc), dtype=torch.int32, device=dev) if cache
                else empty(torch.int32).reshape(0, 0))
    cache_d = (torch.empty((nq, Hc), dtype=torch.float32, device=dev) if cache
               else empty(torch.float32).reshape(0, 0))
    bound = empty(torch.float32)
    ext.init_states(Xg, Qg, Sg, ids, dist, expd, lin, visited, counters, metric, team,
                    cache_id, cache_d, bound)
    ext.advance(Xg, Gg, Qg, ids, dist, expd, lin, visited, counters, metric, team, B, B,
                E.POLICY_BEST, 1, 0.05, k, cache_id, cache_d, bound, False, 0, 0.0,
                empty(torch.int32), empty(torch.int32), empty(torch.float32),
                empty(torch.float32), 0.2)
    mi, md = ext.merge_branches(ids[..., :k].contiguous(), dist[..., :k].contiguous(), k)

    st = E.init_states(Xg, Qg, Sg, L=L, B=B, D=G.shape[1], metric=metric, team_size=team,
                       stop_eps=0.05, kstop=k, shared_cache=cache, cache_slots=Hc or None)
    E.advance(Xg, Gg, Qg, st, B)
    bi, bd = E.branch_topk(st, k)
    wi, wd = E.merge_branches(bi, bd, k)
    torch.cuda.synchronize()
    assert torch.equal(ids, st.ids) and torch.equal(expd, st.expanded)
    assert torch.equal(lin, st.lineage)
    assert dist.cpu().numpy().tobytes() == st.dist.cpu().numpy().tobytes()
    # with a shared table, which branch scores a node first is the schedule's
    # choice: evaluations (1), hits (4) and claims (5) move between branches
    # run to run, evaluations + hits per branch do not
    fixed = [0, 2, 3, 6, 7, 8, 9] + ([] if cache else [1, 4, 5])
    assert torch.equal(counters[..., fixed], st.counters[..., fixed])
    assert torch.equal(counters[..., 1] + counters[..., 4], st.counters[..., 1] + st.counters[..., 4])
    assert torch.equal(mi, wi)
    assert md.cpu().numpy().tobytes() == wd.cpu().numpy().tobytes()
    assert int(counters[..., 1].sum()) > nq * J          # the search did expand
