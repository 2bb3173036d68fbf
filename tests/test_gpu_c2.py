"""Config C2 at its full size on one GPU: 1M x 960 fp32 rows from a
1,000-centre Gaussian mixture (centres N(0,1), per-cluster std 0.3),
unnormalised, metric l2; graph D=64 from a C=128 sweep; k=10, 32 branches,
queue 12, budget 64.  Checked through size-independent properties: sampled
candidate lists against an fp64 brute force over the whole corpus, the
search's distances against fp64 recomputation, no repeated ids, and recall@10
within 0.005 of the oracle's rounds schedule on the same seeds and table size
(the reference's own sizing, swann/_engine.py:186-198) at each stop_eps of
the config's sweep."""
import os
import sys

import numpy as np
import pytest
import torch

import oracle as O
from test_oracle_helpers import describe_rows, untied_rows

pytestmark = pytest.mark.gpu

swann = pytest.importorskip("swann_amd")
from swann_amd import _engine as E  # noqa: E402
from swann_amd import _select as S  # noqa: E402
from swann_amd import build as B  # noqa: E402

N, DIM, C, DEG, NQ = 1_000_000, 960, 128, 64, 1000


def note(*a):
    print("[case]", *a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def c2():
    g = torch.Generator(device="cuda")
    g.manual_seed(22)
    centres = torch.randn((1000, DIM), generator=g, device="cuda")

    def draw(m):
        lab = torch.randint(0, 1000, (m,), generator=g, device="cuda")
        return centres[lab] + 0.3 * torch.randn((m, DIM), generator=g, device="cuda")
    X, Q = draw(N), draw(NQ)
    note("c2 full size: sweep")
    cand, cdist = B.knn_candidates(X, C, metric="l2")
    note("c2 full size: prune + reverse")
    G = B.add_reverse(X, B.robust_prune(X, cand, cdist, DEG, alpha=1.2, metric="l2"), DEG,
                      alpha=1.2, metric="l2")
    xn = (X * X).sum(1)
    truth = torch.topk(xn[None, :] - 2.0 * Q @ X.T, 10, dim=1, largest=False).indices
    torch.cuda.synchronize()
    return dict(X=X, Q=Q, cand=cand, cdist=cdist, G=G, truth=truth.cpu().numpy())


def test_c2_candidates_are_exact_on_sampled_rows(c2):
    X, cand, cdist = c2["X"], c2["cand"], c2["cdist"]
    rows = torch.from_numpy(np.random.default_rng(4).choice(N, 128, replace=False)).cuda()
    A = X[rows].double()
    an = (A * A).sum(1, keepdim=True)
    best_d, best_i = None, None
    for s in range(0, N, 100_000):
        Y = X[s:s + 100_000].double()
        d = an - 2.0 * A @ Y.T + (Y * Y).sum(1)[None, :]
        cols = torch.arange(s, min(N, s + 100_000), device="cuda")
        d[rows[:, None] == cols[None, :]] = 3.4e38             # self, as build.py:39
        v, i = torch.topk(d, C, dim=1, largest=False)
        if best_d is None:
            best_d, best_i = v, i + s
        else:
            dd, ii = torch.cat([best_d, v], 1), torch.cat([best_i, i + s], 1)
            best_d, j = torch.topk(dd, C, dim=1, largest=False)
            best_i = torch.gather(ii, 1, j)
    got = cand[rows].long()
    xb = X[got.reshape(-1)].double().reshape(128, C, DIM)
    exact = ((xb - A[:, None, :]) ** 2).sum(-1)
    g_, w_ = got.cpu().numpy(), best_i.cpu().numpy()
    bad = untied_rows(g_, w_, best_d.cpu().numpy(), exact.cpu().numpy(), atol=0, rtol=2e-5)
    note("c2 sampled candidate rows differing", int((g_ != w_).any(1).sum()), "beyond ties", bad)
    assert bad == [], describe_rows(bad, g_, w_, best_d.cpu().numpy(), exact.cpu().numpy())
    assert torch.allclose(cdist[rows].double(), exact, rtol=2e-5, atol=0)
    cd = cdist.cpu().numpy()
    assert (np.diff(cd, axis=1) >= 0).all()
    Gc = c2["G"].cpu().numpy()
    assert Gc.shape == (N, DEG) and ((Gc >= -1) & (Gc < N)).all()
    assert not (Gc == np.arange(N)[:, None]).any()


@pytest.mark.parametrize("eps", [0.02, 0.05, 0.1, 0.2])
def test_c2_search_matches_the_oracle_rounds_schedule(c2, eps):
    X, Q, G, truth = c2["X"], c2["Q"], c2["G"], c2["truth"]
    index = swann.Index(X, G, metric="l2")
    J, L, Bud = 32, 12, 64
    seeds = index.catalogue[S.select_nearest(Q, index._cat, J, metric=1)].to(torch.int32)
    Hc = E.cache_size(J, Bud, DEG)

    def rec(ids):
        return float(np.mean([len(set(a) & set(b)) / 10 for a, b in zip(ids.tolist(),
                                                                        truth.tolist())]))
    ids, dist, _ = E.search(X, G, Q, seeds, k=10, L=L, B=Bud, metric=1, team_size=16,
                            stop_eps=eps, shared_cache=True, shared_bound=True, exclusive=True,
                            elide_visited=True, check=False, cache_slots=Hc)
    ids_h = ids.cpu().numpy()
    oi, _ = O.search_batch(X.cpu().numpy(), G.cpu().numpy(), Q.cpu().numpy(),
                           seeds.cpu().numpy(), k=10, L=L, B=Bud, metric=1, team=16,
                           stop_eps=eps, H=1, Hc=Hc, bound=True, exclusive=True,
                           nthreads=len(os.sched_getaffinity(0)), schedule="rounds")
    r_gpu, r_oracle = rec(ids_h), rec(oi)
    note("c2 recall eps", eps, "gpu", r_gpu, "oracle rounds", r_oracle)
    assert abs(r_gpu - r_oracle) <= 0.005
    assert r_gpu >= 0.95
    assert (ids_h >= 0).all() and all(len(set(r)) == 10 for r in ids_h.tolist())
    exact = ((X[ids.long().reshape(-1)].double().reshape(NQ, 10, DIM) -
              Q.double()[:, None, :]) ** 2).sum(-1)
    assert torch.allclose(dist.double(), exact, rtol=1e-5, atol=0)
    # Index.search (its larger table) lands on the same recall
    ids2, _ = index.search(Q, k=10, branches=J, queue=L, budget=Bud, stop_eps=eps, team=16)
    note("c2 recall eps", eps, "Index.search", rec(ids2))
    assert abs(rec(ids2) - r_oracle) <= 0.005
