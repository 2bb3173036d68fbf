"""The built graph against a reference-built one beyond C1 (swann/build.py:
153-171): a C5-shaped corpus at 20,000 x 1024 fp32 l2 (centres N(0,1), 20
of them so a cluster holds 1,000 rows as in C5's 1M over 1,000; per-cluster
std 0.3), built on the GPU (fp16 MFMA screen + exact fp32 re-rank, MFMA
prune, reverse) and by the oracle's restatement of the reference's three
stages (fp64 dot products).  Both graphs are searched by the same GPU search
with the same seeds and knobs; recall@10 must agree within 0.005 either way,
with independent branches (deterministic) and in the production mode."""
import os
import sys

import numpy as np
import pytest
import torch

import oracle as O

pytestmark = pytest.mark.gpu

swann = pytest.importorskip("swann_amd")
from swann_amd import _engine as E  # noqa: E402
from swann_amd import _select as S  # noqa: E402
from swann_amd.build import build_graph  # noqa: E402

N, DIM, C, DEG, NQ = 20_000, 1024, 128, 64, 1000


def note(*a):
    print("[case]", *a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def graphs():
    rng = np.random.default_rng(55)
    centres = rng.standard_normal((N // 1000, DIM)).astype(np.float32)

    def draw(m):
        return np.ascontiguousarray(
            (centres[rng.integers(0, len(centres), m)] +
             0.3 * rng.standard_normal((m, DIM))).astype(np.float32))
    X, Q = draw(N), draw(NQ)
    Xg = torch.from_numpy(X).cuda()
    G_gpu = build_graph(Xg, metric="l2", degree=DEG, candidates=C, alpha=1.2)
    cores = len(os.sched_getaffinity(0))
    note(f"oracle build_graph on {cores} cores")
    G_ref = O.build_graph(X, metric=O.METRIC_L2, degree=DEG, candidates=C, alpha=1.2,
                          nthreads=cores)
    d = ((X.astype(np.float64) ** 2).sum(1)[None, :] - 2.0 * Q.astype(np.float64) @
         X.astype(np.float64).T)
    truth = np.argsort(d, axis=1, kind="stable")[:, :10]
    return dict(X=X, Q=Q, Xg=Xg, Qg=torch.from_numpy(Q).cuda(), G_gpu=G_gpu,
                G_ref=torch.from_numpy(np.ascontiguousarray(G_ref, dtype=np.int32)).cuda(),
                truth=truth)


def test_gpu_built_graph_searches_like_the_reference_built_one(graphs):
    X, Xg, Qg, truth = graphs["X"], graphs["Xg"], graphs["Qg"], graphs["truth"]
    Gg, Gr = graphs["G_gpu"], graphs["G_ref"]
    same_rows = float((Gg == Gr).all(dim=1).float().mean())
    same_sets = np.mean([len(set(a) & set(b)) / max(1, len(set(b) - {-1}))
                         for a, b in zip(Gg.cpu().tolist()[:2000], Gr.cpu().tolist()[:2000])])
    note("identical rows", same_rows, "edge-set agreement (2,000 rows)", same_sets)
    index = swann.Index(Xg, Gg, metric="l2")

    def rec(ids):
        ids = ids.cpu().numpy() if torch.is_tensor(ids) else ids
        return float(np.mean([len(set(a) & set(b)) / 10 for a, b in zip(ids.tolist(),
                                                                        truth.tolist())]))
    for J, L, Bud, eps in ((32, 12, 64, 0.05), (4, 12, 16, 0.02)):
        seeds = index.catalogue[S.select_nearest(Qg, index._cat, J, metric=1)].to(torch.int32)
        for prod in (False, True):
            r = {}
            for tag, G in (("gpu-built", Gg), ("reference-built", Gr)):
                ids, _, _ = E.search(Xg, G, Qg, seeds, k=10, L=L, B=Bud, metric=1, team_size=16,
                                     stop_eps=eps, shared_cache=prod, shared_bound=prod,
                                     exclusive=prod, elide_visited=prod, check=False)
                r[tag] = rec(ids)
            note(f"J={J} L={L} B={Bud} eps={eps} production={prod}: {r}")
            assert abs(r["gpu-built"] - r["reference-built"]) <= 0.005
