"""Config C3 at its full size on one GPU (1M x 1536 fp16, inner product, D=64,
C=128), checked through properties that do not depend on the size: the
candidate lists of sampled rows against a brute-force product of those rows
with the whole corpus, the prune of sampled nodes against the oracle on the
rows it reads, the final graph's invariants, and the search's answers
against exact recomputation and exact ground truth."""
import sys

import numpy as np
import pytest
import torch

import oracle as O
from test_oracle_helpers import describe_rows, prune_margins, untied_rows

pytestmark = pytest.mark.gpu

swann = pytest.importorskip("swann_amd")
from swann_amd import build as B  # noqa: E402

N, DIM, RANK, C, DEG = 1_000_000, 1536, 256, 128, 64


def note(*a):
    print("[case]", *a, flush=True)
    sys.stdout.flush()


def lowrank(m, W, g):
    """x = z W / 16 + 0.1 e, rows normalised (the C3 generator's shape)."""
    z = torch.randn((m, RANK), generator=g, device="cuda")
    x = z @ W / 16.0 + 0.1 * torch.randn((m, DIM), generator=g, device="cuda")
    return x / x.norm(dim=1, keepdim=True)


@pytest.fixture(scope="module")
def c3():
    g = torch.Generator(device="cuda")
    g.manual_seed(33)
    W = torch.randn((RANK, DIM), generator=g, device="cuda")
    X16 = lowrank(N, W, g).half()
    Q = lowrank(1000, W, g)
    Q2 = lowrank(1000, W, g)                        # 1,000 more, for the stated-knob sweep
    note("c3 full size: sweep")
    cand, cdist = B.knn_candidates(X16, C, metric="ip")
    note("c3 full size: prune")
    Gp = B.robust_prune(X16, cand, cdist, DEG, alpha=1.2, metric="ip")
    note("c3 full size: reverse")
    G = B.add_reverse(X16, Gp, DEG, alpha=1.2, metric="ip")
    torch.cuda.synchronize()
    return dict(X16=X16, Q=Q, Q2=Q2, cand=cand, cdist=cdist, Gp=Gp, G=G)


def test_candidate_lists_are_exact_on_sampled_rows(c3):
    """The lists of 256 sampled rows equal a brute-force fp64 top-C over the
    whole corpus up to ties within 1e-5 (the bound the returned distances
    are held to: fp16 products are exact, 1,536-term fp32 sums are not), and
    carry distances equal to an fp64 recomputation to 1e-5."""
    X16, cand, cdist = c3["X16"], c3["cand"], c3["cdist"]
    rows = torch.from_numpy(np.random.default_rng(1).choice(N, 256, replace=False)).cuda()
    A = X16[rows].double()
    best_d, best_i = None, None
    for s in range(0, N, 100_000):                  # brute force in fp64
        d = 1.0 - A @ X16[s:s + 100_000].double().T
        cols = torch.arange(s, min(N, s + 100_000), device="cuda")
        d[rows[:, None] == cols[None, :]] = 3.4e38          # self, as build.py:39
        v, i = torch.topk(d, C, dim=1, largest=False)
        i = i + s
        if best_d is None:
            best_d, best_i = v, i
        else:
            dd, ii = torch.cat([best_d, v], 1), torch.cat([best_i, i], 1)
            best_d, j = torch.topk(dd, C, dim=1, largest=False)
            best_i = torch.gather(ii, 1, j)
    got = cand[rows].long()
    xb = X16[got.reshape(-1)].double().reshape(256, C, DIM)
    exact = 1.0 - (xb @ A[:, :, None])[..., 0]
    g_, w_ = got.cpu().numpy(), best_i.cpu().numpy()
    bad = untied_rows(g_, w_, best_d.cpu().numpy(), exact.cpu().numpy(), atol=1e-5, rtol=0)
    note("sampled candidate rows differing", int((g_ != w_).any(1).sum()), "beyond ties", bad)
    assert bad == [], describe_rows(bad, g_, w_, best_d.cpu().numpy(), exact.cpu().numpy())
    # returned distances against an fp64 recomputation from the stored rows
    assert torch.allclose(cdist[rows].double(), exact, rtol=0, atol=1e-5)
    # invariants of every row
    cc, cd = cand.cpu().numpy(), cdist.cpu().numpy()
    assert ((cc >= 0) & (cc < N)).all()
    assert not (cc == np.arange(N)[:, None]).any()
    assert (np.diff(cd, axis=1) >= 0).all()


def test_prune_of_sampled_nodes_matches_oracle(c3):
    """The oracle prunes each sampled node on the corpus rows it reads (the
    node and its candidates), with the sweep's own lists and distances: the
    rows are identical, except where a detour test lies within 2e-5 of its
    threshold (fp32 Gram sums against the oracle's double ones)."""
    X16, cand, cdist, Gp = c3["X16"], c3["cand"], c3["cdist"], c3["Gp"]
    nodes = np.random.default_rng(2).choice(N, 48, replace=False)
    same, bad = 0, []
    for u in nodes:
        ids = np.concatenate([[u], cand[u].cpu().numpy()]).astype(np.int64)
        Xs = X16[torch.from_numpy(ids).cuda()].float().cpu().numpy()
        cs = np.full((len(ids), C), -1, np.int32)
        ds = np.full((len(ids), C), np.inf, np.float32)
        cs[0] = np.arange(1, C + 1, dtype=np.int32)
        ds[0] = cdist[u].cpu().numpy()
        row = O.robust_prune(Xs, cs, ds, DEG, 1.2, O.METRIC_IP, nthreads=8)[0]
        want = np.where(row >= 0, ids[np.clip(row, 0, None)], -1)
        got = Gp[u].cpu().numpy()
        if np.array_equal(want, got):
            same += 1
            continue
        m = prune_margins(Xs, cs, ds, [0], DEG, 1.2, 0)[0]
        if m > 2e-5:
            bad.append((int(u), float(m)))
    note("sampled prune rows equal to the oracle", same, "of", len(nodes), "beyond near-ties", bad)
    assert bad == []


def test_final_graph_invariants(c3):
    G = c3["G"].cpu().numpy()
    assert G.shape == (N, DEG) and G.dtype == np.int32
    assert ((G >= -1) & (G < N)).all()
    assert not (G == np.arange(N)[:, None]).any()
    live = G >= 0
    srt = np.sort(np.where(live, G, -1 - np.arange(DEG)[None, :]), axis=1)
    assert (np.diff(srt, axis=1) != 0).all()          # no id twice in a row
    deg = live.sum(1)
    note("out-degree min/mean", int(deg.min()), float(deg.mean()))
    assert deg.min() >= 1


def test_search_answers_are_exact_and_recall_meets_the_target(c3):
    X16, Q, G = c3["X16"], c3["Q"], c3["G"]
    index = swann.Index(X16, G, metric="ip")
    ids, dist = index.search(Q, k=10, branches=64, queue=48, budget=64, stop_eps=0.2, team=16)
    ids_t = torch.from_numpy(ids.astype(np.int64)).cuda()
    assert (ids >= 0).all()
    assert all(len(set(r)) == 10 for r in ids.tolist())
    exact = 1.0 - (X16[ids_t.reshape(-1)].double().reshape(1000, 10, DIM)
                   @ Q.double()[:, :, None])[..., 0]
    assert torch.allclose(torch.from_numpy(dist).cuda().double(), exact, rtol=0, atol=1e-5)
    truth = torch.topk(Q @ X16.float().T, 10, dim=1).indices.cpu().numpy()
    r = np.mean([len(set(a) & set(b)) / 10 for a, b in zip(ids.tolist(), truth.tolist())])
    note("full-size C3 recall@10", r)
    assert r >= 0.95


def test_c3_headline_knobs_match_the_oracle_rounds_schedule(c3):
    """The production search -- claims, bound, no visited table
    (swann/index.py:105-109) -- at the bench's operating point (64 branches,
    queue 44, budget 64, stop_eps 0.3) on 1,000 queries, against the oracle's
    rounds schedule (each round's steps read the bound the round began with,
    claims land at once) on the same seeds.  Claims kept three ways: the
    reference's table size (swann/_engine.py:186-198) and a 4x larger table,
    each against the oracle at the reference's size, and claim bits (what
    Index.search takes) against the oracle's claim bits.  Recall@10 within
    0.005, distances equal to an fp64 recomputation, no id twice in an
    answer."""
    import os
    from swann_amd import _engine as E
    from swann_amd import _select as S
    X16, Q, G = c3["X16"], c3["Q"], c3["G"]
    index = swann.Index(X16, G, metric="ip")
    J, L, Bud, eps = 64, 44, 64, 0.3
    seeds = index.catalogue[S.select_nearest(Q, index._cat, J, metric=0)].to(torch.int32)
    base = E.cache_size(J, Bud, DEG)
    big = E.cache_size(J, Bud, DEG, share=1.0)
    truth = torch.topk(Q @ X16.float().T, 10, dim=1).indices.cpu().numpy()

    def rec(ids):
        return float(np.mean([len(set(a) & set(b)) / 10 for a, b in zip(ids.tolist(),
                                                                        truth.tolist())]))
    cores = len(os.sched_getaffinity(0))
    Xh, Gh, Qh, Sh = X16.cpu().numpy(), G.cpu().numpy(), Q.cpu().numpy(), seeds.cpu().numpy()
    r_oracle = {}
    for bits in (False, True):
        note(f"c3 headline: oracle rounds schedule on {cores} cores, claim bits {bits}")
        oi, _ = O.search_batch(Xh, Gh, Qh, Sh, k=10, L=L, B=Bud, metric=0, team=16,
                               stop_eps=eps, H=1, Hc=base, bound=True, exclusive=True,
                               nthreads=cores, schedule="rounds", claim_bits=bits)
        r_oracle[bits] = rec(oi)
    for bits, hc in ((False, base), (False, big), (True, None)):
        ids, dist, _ = E.search(X16, G, Q, seeds, k=10, L=L, B=Bud, metric=0, team_size=16,
                                stop_eps=eps, shared_cache=True, shared_bound=True,
                                exclusive=True, elide_visited=True, check=False, cache_slots=hc,
                                claim_bits=bits)
        ids_h = ids.cpu().numpy()
        r_gpu = rec(ids_h)
        note("c3 headline recall: gpu", r_gpu, "table", hc, "bits", bits,
             "oracle rounds", r_oracle[bits])
        assert abs(r_gpu - r_oracle[bits]) <= 0.005
        assert (ids_h >= 0).all() and all(len(set(r)) == 10 for r in ids_h.tolist())
        exact = 1.0 - (X16[ids.long().reshape(-1)].double().reshape(-1, 10, DIM)
                       @ Q.double()[:, :, None])[..., 0]
        assert torch.allclose(dist.double(), exact, rtol=0, atol=1e-5)
    assert index._claims(Q.shape[0], swann.SearchConfig(branches=J, budget=Bud))[0]
    ids, _ = index.search(Q, k=10, branches=J, queue=L, budget=Bud, stop_eps=eps, team=16)
    r_index = rec(ids)
    note("c3 headline recall: Index.search", r_index)
    assert abs(r_index - r_oracle[True]) <= 0.005


@pytest.mark.parametrize("eps", [0.02, 0.05, 0.1, 0.2])
def test_c3_stated_knobs_match_the_oracle_schedules(c3, eps):
    """C3 at the knobs the config states (32 branches, team 16) with the
    reference's queue 12 and budget 64 (swann/index.py:40-45), over the
    stop_eps sweep, 2,000 queries, Index.search (claim bits) against the
    oracle with claim bits on the same seeds.

    The shared bound is racy: a step reads it at some point after other
    branches' steps lowered it (local_search.cu:466-469, :655-658), so
    where a tight stop_eps lets it end branches early the recall depends on
    how stale the bound a step reads is.  Two legal schedules bracket the
    concurrent launch: every step of round s reading the bound as round s
    began ("rounds") and as round s - 1 began ("rounds2"); the GPU's recall
    must lie between them, widened by 0.005 -- within 0.005 of both where
    they agree.  At eps 0.02, where they differ most, the bound's part is
    separated out: with the bound off (claims kept) the GPU and the oracle
    must agree within 0.005.  Distances equal an fp64 recomputation, no id
    twice."""
    import os
    from swann_amd import _engine as E
    from swann_amd import _select as S
    X16, G = c3["X16"], c3["G"]
    Q = torch.cat([c3["Q"], c3["Q2"]])
    index = swann.Index(X16, G, metric="ip")
    J, L, Bud = 32, 12, 64
    seeds = index.catalogue[S.select_nearest(Q, index._cat, J, metric=0)].to(torch.int32)
    truth = torch.topk(Q @ X16.float().T, 10, dim=1).indices.cpu().numpy()

    def rec(ids):
        return float(np.mean([len(set(a) & set(b)) / 10 for a, b in zip(ids.tolist(),
                                                                        truth.tolist())]))
    Xh, Gh, Qh, Sh = X16.cpu().numpy(), G.cpu().numpy(), Q.cpu().numpy(), seeds.cpu().numpy()
    cores = len(os.sched_getaffinity(0))

    def oracle(schedule, bound=True):
        oi, _ = O.search_batch(Xh, Gh, Qh, Sh, k=10, L=L, B=Bud, metric=0, team=16,
                               stop_eps=eps, H=1, Hc=None, bound=bound, exclusive=True,
                               nthreads=cores, schedule=schedule, claim_bits=True)
        return rec(oi)
    r1, r2 = oracle("rounds"), oracle("rounds2")
    ids, dist = index.search(Q, k=10, branches=J, queue=L, budget=Bud, stop_eps=eps, team=16)
    r_gpu = rec(ids)
    note("c3 stated knobs eps", eps, "queries", Q.shape[0], "Index.search", r_gpu,
         "oracle rounds", r1, "rounds2", r2)
    assert min(r1, r2) - 0.005 <= r_gpu <= max(r1, r2) + 0.005
    if eps == 0.02:
        r_off = oracle("rounds", bound=False)
        ids_off, _, _ = E.search(X16, G, Q, seeds, k=10, L=L, B=Bud, metric=0, team_size=16,
                                 stop_eps=eps, shared_cache=True, shared_bound=False,
                                 exclusive=True, elide_visited=True, check=False,
                                 claim_bits=True)
        r_gpu_off = rec(ids_off.cpu().numpy())
        note("c3 stated knobs eps", eps, "bound off: gpu", r_gpu_off, "oracle", r_off)
        assert abs(r_gpu_off - r_off) <= 0.005
    assert (ids >= 0).all() and all(len(set(r)) == 10 for r in ids.tolist())
    ids_t = torch.from_numpy(ids.astype(np.int64)).cuda()
    exact = 1.0 - (X16[ids_t.reshape(-1)].double().reshape(-1, 10, DIM)
                   @ Q.double()[:, :, None])[..., 0]
    assert torch.allclose(torch.from_numpy(dist).cuda().double(), exact, rtol=0, atol=1e-5)


# ---------------------------------------------------------------------------
# Config C5: the build target, 1M x 1024 fp32 L2 (a 1000-centre mixture)

D5 = 1024


def gmm(m, centres, g):
    lab = torch.randint(0, centres.shape[0], (m,), generator=g, device="cuda")
    return centres[lab] + 0.3 * torch.randn((m, D5), generator=g, device="cuda")


@pytest.fixture(scope="module")
def c5():
    g = torch.Generator(device="cuda")
    g.manual_seed(55)
    centres = torch.randn((1000, D5), generator=g, device="cuda")
    X = gmm(N, centres, g)
    Q = gmm(1000, centres, g)
    note("c5 full size: sweep")
    cand, cdist = B.knn_candidates(X, C, metric="l2")
    note("c5 full size: prune + reverse")
    G = B.add_reverse(X, B.robust_prune(X, cand, cdist, DEG, alpha=1.2, metric="l2"), DEG,
                      alpha=1.2, metric="l2")
    torch.cuda.synchronize()
    return dict(X=X, Q=Q, cand=cand, cdist=cdist, G=G)


def test_c5_candidates_are_exact_on_sampled_rows(c5):
    """fp32 rows go through the fp16 screen and the exact fp32 re-rank: the
    lists of sampled rows equal a brute-force fp64 top-C up to near-ties and
    carry distances equal to an fp64 recomputation to fp32 rounding."""
    X, cand, cdist = c5["X"], c5["cand"], c5["cdist"]
    rows = torch.from_numpy(np.random.default_rng(3).choice(N, 128, replace=False)).cuda()
    A = X[rows].double()
    an = (A * A).sum(1, keepdim=True)
    best_d, best_i = None, None
    for s in range(0, N, 100_000):
        Y = X[s:s + 100_000].double()
        d = an - 2.0 * A @ Y.T + (Y * Y).sum(1)[None, :]
        cols = torch.arange(s, min(N, s + 100_000), device="cuda")
        d[rows[:, None] == cols[None, :]] = 3.4e38
        v, i = torch.topk(d, C, dim=1, largest=False)
        if best_d is None:
            best_d, best_i = v, i + s
        else:
            dd, ii = torch.cat([best_d, v], 1), torch.cat([best_i, i + s], 1)
            best_d, j = torch.topk(dd, C, dim=1, largest=False)
            best_i = torch.gather(ii, 1, j)
    got = cand[rows].long()
    xb = X[got.reshape(-1)].double().reshape(128, C, D5)
    exact = ((xb - A[:, None, :]) ** 2).sum(-1)
    g_, w_ = got.cpu().numpy(), best_i.cpu().numpy()
    bad = untied_rows(g_, w_, best_d.cpu().numpy(), exact.cpu().numpy(), atol=0, rtol=2e-5)
    note("c5 sampled candidate rows differing", int((g_ != w_).any(1).sum()), "beyond ties", bad)
    assert bad == [], describe_rows(bad, g_, w_, best_d.cpu().numpy(), exact.cpu().numpy())
    assert torch.allclose(cdist[rows].double(), exact, rtol=2e-5, atol=0)
    cc, cd = cand.cpu().numpy(), cdist.cpu().numpy()
    assert ((cc >= 0) & (cc < N)).all()
    assert not (cc == np.arange(N)[:, None]).any()
    assert (np.diff(cd, axis=1) >= 0).all()


def test_c5_graph_and_search(c5):
    """The C5 graph's invariants, and a search over it at the config's knobs
    (32 branches, stop_eps 0.05, queue 12, budget 64): distances equal to an
    fp64 recomputation, recall@10 within 0.005 of the oracle's rounds
    schedule on the same seeds."""
    X, Q, G = c5["X"], c5["Q"], c5["G"]
    Gc = G.cpu().numpy()
    assert Gc.shape == (N, DEG) and ((Gc >= -1) & (Gc < N)).all()
    assert not (Gc == np.arange(N)[:, None]).any()
    index = swann.Index(X, G, metric="l2")
    ids, dist = index.search(Q, k=10, branches=32, queue=12, budget=64, stop_eps=0.05, team=16)
    assert (ids >= 0).all() and all(len(set(r)) == 10 for r in ids.tolist())
    ids_t = torch.from_numpy(ids.astype(np.int64)).cuda()
    exact = ((X[ids_t.reshape(-1)].double().reshape(1000, 10, D5) - Q.double()[:, None, :]) ** 2
             ).sum(-1)
    assert torch.allclose(torch.from_numpy(dist).cuda().double(), exact, rtol=1e-5, atol=0)
    xn = (X * X).sum(1)
    truth = torch.topk(xn[None, :] - 2.0 * Q @ X.T, 10, dim=1, largest=False).indices
    truth = truth.cpu().tolist()

    def rec(a):
        return float(np.mean([len(set(x) & set(y)) / 10 for x, y in zip(a.tolist(), truth)]))
    # the oracle's rounds schedule with claim bits on the same seeds
    import os
    from swann_amd import _select as S
    seeds = index.catalogue[S.select_nearest(Q, index._cat, 32, metric=1)].to(torch.int32)
    oi, _ = O.search_batch(X.cpu().numpy(), Gc, Q.cpu().numpy(), seeds.cpu().numpy(), k=10,
                           L=12, B=64, metric=1, team=16, stop_eps=0.05, H=1, Hc=None,
                           bound=True, exclusive=True, nthreads=len(os.sched_getaffinity(0)),
                           schedule="rounds", claim_bits=True)
    r, r_oracle = rec(ids), rec(oi)
    note("full-size C5 recall@10: Index.search", r, "oracle rounds", r_oracle)
    assert abs(r - r_oracle) <= 0.005


@pytest.fixture(scope="module")
def c3_small():
    """A C3-shaped corpus (20,000 x 1536 fp16, rank-256 low-rank plus noise,
    rows normalised, ip) built by Index.build on the GPU and by the oracle's
    restatement of build.py (sweep, prune, reverse on the fp32 values of the
    same fp16 rows), with 1,000 queries and their exact top 10."""
    import os
    n = 20_000
    g = torch.Generator(device="cuda")
    g.manual_seed(2033)
    W = torch.randn((RANK, DIM), generator=g, device="cuda")
    X16 = lowrank(n, W, g).half()
    Q = lowrank(1000, W, g)
    note("c3-shaped graph parity: GPU build")
    ix_gpu = swann.Index.build(X16, metric="ip", degree=DEG, candidates=C)
    note("c3-shaped graph parity: oracle build")
    G_or = O.build_graph(X16.float().cpu().numpy(), metric=O.METRIC_IP, degree=DEG,
                         candidates=C, alpha=1.2, nthreads=len(os.sched_getaffinity(0)))
    ix_or = swann.Index(X16, torch.from_numpy(np.ascontiguousarray(G_or, dtype=np.int32)).cuda(),
                        metric="ip")
    truth = torch.topk(Q @ X16.float().T, 10, dim=1).indices.cpu().tolist()
    return dict(ix_gpu=ix_gpu, ix_or=ix_or, G_or=G_or, Q=Q, truth=truth)


@pytest.mark.parametrize("knobs", [(8, 12, 32, 0.02), (32, 12, 64, 0.1)])
def test_c3_shaped_graph_built_both_ways_gives_the_same_recall(c3_small, knobs):
    """Both builds of the C3-shaped corpus searched by Index.search with the
    same catalogue and knobs: recall@10 against exact ground truth agrees
    within 0.005 either way (build.py:153-171, index.py:40-45)."""
    J, L, Bud, eps = knobs
    ix_gpu, ix_or, Q, truth = c3_small["ix_gpu"], c3_small["ix_or"], c3_small["Q"], c3_small["truth"]
    assert torch.equal(ix_gpu.catalogue, ix_or.catalogue)

    def rec(a):
        return float(np.mean([len(set(x) & set(y)) / 10 for x, y in zip(a.tolist(), truth)]))
    rs = []
    for ix in (ix_gpu, ix_or):
        ids, _ = ix.search(Q, k=10, branches=J, queue=L, budget=Bud, stop_eps=eps, team=16)
        rs.append(rec(ids))
    edges = int((ix_gpu.G >= 0).sum()), int((c3_small["G_or"] >= 0).sum())
    note("c3-shaped graph parity", knobs, "recall@10 gpu-built / oracle-built", rs, "edges", edges)
    assert abs(rs[0] - rs[1]) <= 0.005
