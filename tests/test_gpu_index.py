"""The public interface on the GPU, end to end (the reference's
tests/test_index.py), plus seed selection and the build stages against the
oracle and the reference's golden build vectors."""
import sys

import numpy as np
import pytest
import torch

import oracle as O
from conftest import ROOT, deg96_corpus, gaussian, golden, regen
from test_oracle_helpers import (describe_rows, exact_topk, recall, untied_graph_rows,
                                 untied_prune_rows, untied_rows)

pytestmark = pytest.mark.gpu

swann = pytest.importorskip("swann_amd")
from swann_amd import _select as S  # noqa: E402
from swann_amd import build as B  # noqa: E402


def note(*a):
    print("[case]", *a, flush=True)
    sys.stdout.flush()


def same_lists(tag, cand, cdist, oc, od, atol, rtol):
    """The GPU's candidate lists equal the oracle's up to ties: within each
    run of oracle distances closer than the distance tolerance (atol + rtol
    |d|, the bound the same test holds the GPU distances to) the ids may come
    in another order, and at the cut another tied row may take the place."""
    cand = cand.cpu().numpy() if torch.is_tensor(cand) else cand
    cdist = cdist.cpu().numpy() if torch.is_tensor(cdist) else cdist
    bad = untied_rows(cand, oc, od, cdist, atol=atol, rtol=rtol)
    note(tag, "rows differing", int((cand != oc).any(1).sum()), "beyond ties", len(bad),
         describe_rows(bad, cand, oc, od, cdist))
    assert bad == [], describe_rows(bad, cand, oc, od, cdist)


def corpus(n=8000, d=128, nq=200, seed=0, normalise=True):
    rng = np.random.default_rng(seed)
    X = rng.standard_normal((n, d), dtype=np.float32)
    Q = rng.standard_normal((nq, d), dtype=np.float32)
    if normalise:
        X /= np.linalg.norm(X, axis=1, keepdims=True)
        Q /= np.linalg.norm(Q, axis=1, keepdims=True)
    return X, Q


@pytest.mark.parametrize("metric", ["ip", "l2"])
def test_recall_is_high(metric):
    note("recall", metric)
    X, Q = corpus(normalise=(metric == "ip"))
    index = swann.Index.build(X, metric=metric, degree=48, candidates=64)
    ids, dist = index.search(Q, k=10)
    assert ids.shape == (Q.shape[0], 10) and dist.shape == ids.shape
    r = recall(ids, exact_topk(X, Q, 10, 0 if metric == "ip" else 1), 10)
    note("recall", metric, r)
    assert r > 0.90


def test_more_branches_do_not_lose_recall():
    X, Q = corpus()
    index = swann.Index.build(X, degree=48, candidates=64)
    truth = exact_topk(X, Q, 10)
    few = recall(index.search(Q, k=10, branches=8)[0], truth, 10)
    many = recall(index.search(Q, k=10, branches=64)[0], truth, 10)
    assert many >= few - 1e-9


def test_round_trip(tmp_path):
    X, Q = corpus()
    index = swann.Index.build(X, degree=48, candidates=64)
    before, _ = index.search(Q, k=10)
    index.save(tmp_path / "ix")
    again = swann.Index.load(tmp_path / "ix", X)
    assert torch.equal(again.G, index.G) and torch.equal(again.catalogue, index.catalogue)
    after, _ = again.search(Q, k=10)
    # claims and the bound are racy: the answers agree, up to rare reorders,
    # and find the same share of the true neighbours
    assert (before == after).mean() > 0.99
    truth = exact_topk(X, Q, 10)
    assert abs(recall(before, truth, 10) - recall(after, truth, 10)) <= 0.005


def test_batch_beyond_65535_is_served():
    """The reference refuses more than 65535 queries; the 1-D grid does not."""
    X, _ = corpus(n=2000)
    index = swann.Index.build(X, degree=32, candidates=48)
    Q = np.ascontiguousarray(np.repeat(X[:700], 100, axis=0))       # 70,000 queries
    ids, dist = index.search(Q, k=10, branches=2)
    assert ids.shape == (70000, 10)
    assert (ids[:, 0] == np.repeat(np.arange(700), 100)).mean() > 0.95


@pytest.mark.parametrize("branches", [40, 100])
def test_nan_query_finds_nothing_and_leaves_the_batch_alone(branches):
    """A query that is NaN throughout: its catalogue distances cannot be
    ranked, yet its seeds are distinct catalogue rows (the selection's sorts
    rank NaN after every number, and a branch count that is not a power of
    two pads them), each seed scores NaN and is dropped, so its answer is
    empty, (-1, +inf); the other queries' answers stay valid, with their
    recall."""
    X, Q = corpus(n=4000, nq=64)
    index = swann.Index.build(X, degree=32, candidates=48)
    truth = exact_topk(X, Q, 10)
    base = recall(index.search(Q, k=10, branches=branches)[0], truth, 10)
    Qn = Q.copy()
    Qn[5] = np.nan
    ids, dist = index.search(Qn, k=10, branches=branches)
    note("nan query", branches, "recall without/with", base)
    assert (ids[5] == -1).all() and np.isinf(dist[5]).all()
    keep = np.arange(len(Q)) != 5
    assert ((ids[keep] >= 0) & (ids[keep] < len(X))).all()
    assert np.isfinite(dist[keep]).all()
    r = recall(ids[keep], truth[keep], 10)
    note("nan query", branches, base, r)
    assert r > 0.85 and abs(r - base) <= 0.05


def test_unknown_option_is_a_type_error():
    X, Q = corpus(n=1000)
    index = swann.Index.build(X, degree=16, candidates=32)
    with pytest.raises(TypeError):
        index.search(Q, k=10, banches=4)


def test_fp16_corpus_distances_within_tolerance():
    """fp16 corpus, fp32 queries: returned distances equal exact fp32
    recomputation on the fp16 values to 2e-3."""
    X, Q = corpus(n=6000)
    X16 = X.astype(np.float16)
    index = swann.Index(torch.from_numpy(X16).cuda(),
                        B.build_graph(torch.from_numpy(X).cuda(), degree=32, candidates=64),
                        metric="ip")
    ids, dist = index.search(Q, k=10)
    Xf = X16.astype(np.float64)
    for q in range(0, Q.shape[0], 7):
        for i, dv in zip(ids[q], dist[q]):
            if i >= 0:
                assert abs(dv - (1.0 - Q[q].astype(np.float64) @ Xf[i])) < 2e-3


def test_select_matches_oracle():
    g = golden("refcpu_c1.npz")
    X = regen(10000, 128, 0, True, g["X_sha"])
    cat = g["catalogue"].astype(np.int64)
    Vp = torch.from_numpy(X[cat]).cuda()
    for metric in (0, 1):
        idx = S.select_nearest(torch.from_numpy(g["Q"]).cuda(), Vp, 8, metric=metric)
        want, _ = O.select_nearest(g["Q"], X[cat], 8, metric, nthreads=8)
        got = idx.cpu().numpy()
        Q64, V64 = g["Q"].astype(np.float64), X[cat].astype(np.float64)
        if metric == 0:
            dist = lambda e: 1.0 - np.einsum("qd,qkd->qk", Q64, V64[e])  # noqa: E731
        else:
            dist = lambda e: ((V64[e] - Q64[:, None, :]) ** 2).sum(-1)  # noqa: E731
        bad = untied_rows(got, want, dist(want), dist(got))
        note("select", metric, "rows beyond ties", bad)
        assert bad == []
        if metric == 0:
            ref = g["seeds"].astype(np.int64)
            pos = np.searchsorted(cat, ref)
            assert untied_rows(got, pos, dist(pos), dist(got)) == []


@pytest.mark.parametrize("tag,metric", [("ip", 0), ("l2", 1)])
def test_build_stages_match_reference(tag, metric):
    """The three stages against the reference's CPU-torch build.py
    (tests/golden/refbuild_small.npz): the sweep equal up to ties within
    1e-6, the prune identical, the reverse pass equal up to the order of
    tied neighbours."""
    g = golden("refbuild_small.npz")
    X = torch.from_numpy(g[f"{tag}_X"]).cuda()
    m = "ip" if metric == 0 else "l2"
    cand, cdist = B.knn_candidates(X, 32, metric=m)
    rc = g[f"{tag}_cand"].astype(np.int32); rd = g[f"{tag}_cdist"]
    bad = untied_rows(cand.cpu().numpy(), rc, rd, cdist.cpu().numpy())
    note("sweep", tag, "untied rows", bad)
    assert bad == []
    assert np.allclose(cdist.cpu().numpy(), rd, atol=3e-5, rtol=1e-5)
    Gp = B.robust_prune(X, torch.from_numpy(rc).cuda(), torch.from_numpy(rd).cuda(), 16,
                        alpha=1.2, metric=m).cpu().numpy()
    assert np.array_equal(Gp, g[f"{tag}_Gp"].astype(np.int32))
    Gf = B.add_reverse(X, torch.from_numpy(g[f"{tag}_Gp"].astype(np.int32)).cuda(), 16,
                       alpha=1.2, metric=m).cpu().numpy()
    bad = untied_graph_rows(Gf, g[f"{tag}_Gf"].astype(np.int32), g[f"{tag}_X"], metric)
    note("reverse", tag, "untied rows", bad)
    assert bad == []


@pytest.mark.parametrize("tag,metric", [("ip", 0), ("l2", 1)])
def test_build_at_default_degree_matches_reference(tag, metric):
    """Index.build with the reference API's defaults (candidates 128, degree
    96, alpha 1.2; index.py:76, build.py:153-171), where add_reverse cuts
    its 160-wide union to 128 (build.py:138-148), against the reference's
    CPU-torch stages (tests/golden/refbuild_deg96.npz) stage by stage, and
    the whole build against the oracle's prune and reverse of the GPU's own
    candidate lists, row for row."""
    g = golden("refbuild_deg96.npz")
    X = deg96_corpus(tag, g)
    Xg = torch.from_numpy(X).cuda()
    m = "ip" if metric == 0 else "l2"
    note("deg96", tag)
    rc = g[f"{tag}_cand"].astype(np.int32); rd = g[f"{tag}_cdist"]
    cand, cdist = B.knn_candidates(Xg, 128, metric=m)
    cand, cdist = cand.cpu().numpy(), cdist.cpu().numpy()
    bad = untied_rows(cand, rc, rd, cdist)
    note("deg96 sweep untied rows", bad)
    assert bad == []
    want_p = g[f"{tag}_Gp"].astype(np.int32)
    Gp = B.robust_prune(Xg, torch.from_numpy(rc).cuda(), torch.from_numpy(rd).cuda(), 96,
                        alpha=1.2, metric=m).cpu().numpy()
    note("deg96 prune rows differing", int((Gp != want_p).any(1).sum()))
    assert np.array_equal(Gp, want_p)
    want_f = g[f"{tag}_Gf"].astype(np.int32)
    Gf = B.add_reverse(Xg, torch.from_numpy(want_p).cuda(), 96, alpha=1.2, metric=m).cpu().numpy()
    bad = untied_graph_rows(Gf, want_f, X, metric)
    note("deg96 reverse untied rows", bad)
    assert bad == []
    index = swann.Index.build(Xg, metric=m)
    G = index.G.cpu().numpy()
    assert G.shape == (X.shape[0], 96)
    Op = O.robust_prune(X, cand, cdist, 96, 1.2, metric, nthreads=8)
    Of = O.add_reverse(X, Op, 96, 1.2, 64, metric, nthreads=8)
    bad = untied_graph_rows(G, Of, X, metric)
    note("deg96 Index.build vs oracle untied rows", bad)
    assert bad == []


@pytest.mark.parametrize("tag,metric", [("adv_l2", 1), ("adv_ip", 0)])
def test_reverse_cut_and_in_edge_order_match_reference(tag, metric):
    """add_reverse at degree 96 on the hand-made graph whose node 0 keeps
    1 + 32 neighbours only through the cut to 128 and the ascending-source
    in-edges (tests/golden/refbuild_deg96.npz): every row as the reference."""
    g = golden("refbuild_deg96.npz")
    X = g[f"{tag}_X"]
    want = g[f"{tag}_Gf"].astype(np.int32)
    Gf = B.add_reverse(torch.from_numpy(X).cuda(),
                       torch.from_numpy(g[f"{tag}_G"].astype(np.int32)).cuda(), 96, alpha=1.2,
                       metric="ip" if metric == 0 else "l2").cpu().numpy()
    assert (Gf[0] >= 0).sum() == 33
    assert untied_graph_rows(Gf, want, X, metric) == []


def test_build_matches_oracle_exactly_where_it_can():
    """Against the oracle's restatement on one corpus: the same candidate
    lists, and the prune of identical inputs gives identical rows."""
    X = gaussian(3000, 40, 313, False)
    Xg = torch.from_numpy(X).cuda()
    cand, cdist = B.knn_candidates(Xg, 48, metric="l2")
    oc, od = O.knn_candidates(X, 48, O.METRIC_L2, nthreads=8)
    same_lists("sweep l2 d40", cand, cdist, oc, od, 1e-6, 1e-6)
    Gp = B.robust_prune(Xg, torch.from_numpy(oc).cuda(), torch.from_numpy(od).cuda(), 24,
                        metric="l2").cpu().numpy()
    Op = O.robust_prune(X, oc, od, 24, 1.2, O.METRIC_L2, nthreads=8)
    assert np.array_equal(Gp, Op)


def test_c1_built_graph_recall_matches_reference_graph():
    """The GPU-built C1 graph gives recall within 0.005 of the reference-built
    graph (tests/golden/refcpu_c1.npz) under the same search."""
    from swann_amd import _engine as E
    g = golden("refcpu_c1.npz")
    X = regen(10000, 128, 0, True, g["X_sha"])
    Xg = torch.from_numpy(X).cuda()
    G_gpu = B.build_graph(Xg, metric="ip", degree=32, candidates=64, alpha=1.2)
    G_ref = torch.from_numpy(g["G"].astype(np.int32)).cuda()
    Q = gaussian(2000, 128, 777, True)
    Qg = torch.from_numpy(Q).cuda()
    cat = torch.from_numpy(g["catalogue"].astype(np.int64)).cuda()
    seeds = cat[S.select_nearest(Qg, Xg[cat], 8, metric=0)].to(torch.int32)
    truth = exact_topk(X, Q, 10)
    rs = []
    for G in (G_gpu, G_ref):
        ids, _, _ = E.search(Xg, G, Qg, seeds, k=10, L=12, B=64, metric=0, team_size=16,
                             stop_eps=0.05)
        rs.append(recall(ids.cpu().numpy(), truth, 10))
    note("C1 graph recall gpu-built / reference-built", rs)
    assert abs(rs[0] - rs[1]) <= 0.005


@pytest.mark.parametrize("metric", [0, 1])
@pytest.mark.parametrize("dtype", ["f32", "f16"])
def test_mfma_sweep_matches_oracle(metric, dtype):
    """The MFMA sweep (dim % 8 == 0): fp32 rows through a power-of-two scaled
    fp16 screen of C+32 per row and an exact fp32 re-rank, fp16 rows as exact
    products; ragged n exercises the tile edges."""
    n, d = 3001, 64
    X = gaussian(n, d, 401 + metric, metric == 0)
    if metric == 1:
        X = X * 3.0 + 1.5                       # unnormalised, offset: exercises the row scales
    if dtype == "f16":
        X = X.astype(np.float16)
    Xg = torch.from_numpy(X).cuda()
    m = "ip" if metric == 0 else "l2"
    note("mfma sweep", dtype, m)
    cand, cdist = B.knn_candidates(Xg, 40, metric=m)
    oc, od = O.knn_candidates(X.astype(np.float32), 40, metric, nthreads=8)
    scale = 1.0 if metric == 0 else float(np.abs(od).max())
    same_lists(f"mfma sweep {dtype} {m}", cand, cdist, oc, od, 2e-6 * scale, 2e-5)
    assert np.allclose(cdist.cpu().numpy(), od, rtol=2e-5, atol=2e-6 * scale)
    # self is never a candidate, rows are ascending
    assert not (cand.cpu().numpy() == np.arange(n)[:, None]).any()
    assert (np.diff(cdist.cpu().numpy(), axis=1) >= 0).all()


@pytest.mark.parametrize("switch", [("sweep_waves", 8), ("sweep_regstage", 1),
                                    ("sweep_sym", 1), ("sweep_sym_fcap", 4),
                                    ("sweep_rowscale", 1)])
@pytest.mark.parametrize("metric", [0, 1])
@pytest.mark.parametrize("dtype", ["f32", "f16"])
def test_mfma_sweep_other_layouts_match_oracle(opt, switch, metric, dtype):
    """The direct-load sweep's 8-wave layout (128 x 64 wave tiles), the
    register-staged kernel and the symmetric sweep (each tile scored once for
    both of its panels' rows, in bands of launches), all chosen by
    environment at each call, keep the oracle's lists like the default
    layout; so does the symmetric sweep whose second lists are made to
    overflow (4 entries of room), which must redo the sweep one-sided, and an
    fp32 corpus screened on a row-scaled fp16 plane (the default takes these
    corpora's values into fp16 unscaled).  Each is an option of the library
    (swann_set_option), set for the test."""
    opt(**{switch[0]: switch[1]})
    if switch[0] == "sweep_sym_fcap":
        opt(sweep_sym=1)
    n, d = 3001, 64
    X = gaussian(n, d, 431 + metric, metric == 0)
    if metric == 1:
        X = X * 3.0 + 1.5
    if dtype == "f16":
        X = X.astype(np.float16)
    Xg = torch.from_numpy(X).cuda()
    m = "ip" if metric == 0 else "l2"
    note("mfma sweep layout", switch, dtype, m)
    cand, cdist = B.knn_candidates(Xg, 40, metric=m)
    oc, od = O.knn_candidates(X.astype(np.float32), 40, metric, nthreads=8)
    scale = 1.0 if metric == 0 else float(np.abs(od).max())
    same_lists(f"mfma sweep layout {switch} {dtype} {m}", cand, cdist, oc, od, 2e-6 * scale, 2e-5)
    assert np.allclose(cdist.cpu().numpy(), od, rtol=2e-5, atol=2e-6 * scale)
    assert not (cand.cpu().numpy() == np.arange(n)[:, None]).any()


@pytest.mark.parametrize("metric,spread", [(0, "wide"), (1, "wide"), (1, "tiny"), (1, "some")])
def test_mfma_sweep_picks_the_row_scaled_plane_from_the_range(metric, spread):
    """An fp32 corpus goes to fp16 unscaled only when every row's max |x| lies
    in [2^-4, 2^14]; the sweep measures that range on the GPU (row_range,
    several rows a wave).  A corpus scaled past fp16's range (x 3e5), far
    below it (x 1e-6, subnormal in fp16) or with every 7th row past it must
    go to the row-scaled plane: unscaled, those values overflow to inf or
    keep a few bits, and the lists would not be the oracle's.  dim 64 reads
    rows as 16-byte vectors, dim 66 element by element.  (A tiny corpus under
    ip has every distance within an ulp of 1, ties that fp32 rounding order
    decides, so it runs under l2.)"""
    factor = {"wide": 3e5, "tiny": 1e-6, "some": 3e5}[spread]
    for d in (64, 66):
        n = 3001
        X = gaussian(n, d, 441 + metric + d, metric == 0)
        if metric == 1:
            X = X * 3.0 + 1.5
        if spread == "some":
            X[::7] *= factor
        else:
            X *= factor
        X = np.ascontiguousarray(X.astype(np.float32))
        Xg = torch.from_numpy(X).cuda()
        m = "ip" if metric == 0 else "l2"
        note("mfma sweep plane choice", spread, m, d)
        cand, cdist = B.knn_candidates(Xg, 40, metric=m)
        oc, od = O.knn_candidates(X, 40, metric, nthreads=8)
        assert np.isfinite(cdist.cpu().numpy()).all()
        # rounding of (|a|^2 + |b|^2) - 2 a.b in fp32 scales with the norms
        nrm = (X.astype(np.float64) ** 2).sum(1)
        scale = nrm[:, None] + nrm[oc] if metric == 1 else np.abs(od).max()
        same_lists(f"mfma sweep plane choice {spread} {m} {d}", cand, cdist, oc, od,
                   4e-6 * scale, 2e-5)
        assert np.allclose(cdist.cpu().numpy(), od, rtol=2e-5, atol=4e-6 * scale)


_ORACLE_LISTS = {}


def oracle_lists(X, C, metric, key):
    """The oracle's top-C lists of X, computed once per corpus key."""
    if key not in _ORACLE_LISTS:
        _ORACLE_LISTS[key] = O.knn_candidates(X.astype(np.float32), C, metric, nthreads=16)
    return _ORACLE_LISTS[key]


@pytest.mark.parametrize("d", [64, 256])
@pytest.mark.parametrize("mode", ["order", "seeds", "order-overflow", "order-overflow-16"])
@pytest.mark.parametrize("metric", [0, 1])
@pytest.mark.parametrize("dtype", ["f32", "f16"])
def test_mfma_sweep_seeded_thresholds_keep_the_lists(opt, metric, dtype, mode, d):
    """On clustered rows (n = 20,000 of a 60-cluster mixture) the symmetric
    sweep runs on a locality-ordered copy from seeded thresholds ("order", the
    default), or in the rows' own order from the same seeds
    (option sweep_order 0); with room for only 4 foreign candidates a row,
    every panel overflows and is repaired by the one-sided re-sweep of its
    panel, two column halves for all panels at once ("order-overflow") or
    sixteen column ranges a panel at a time with a per-row merge of the
    sixteen lists ("order-overflow-16", forced by option sweep_repair_max).
    The lists, mapped back to the rows' own ids, must be those of the plain
    sweep (option sweep_noseed) and the oracle's.  d = 256 takes four K
    steps a tile: the staged foreign queue, its drain after the loop and the
    deferred threshold wait run only there."""
    opt(sweep_sym=1)
    if mode == "seeds":
        opt(sweep_order=0)
    n, C = 20000, 24
    rng = np.random.default_rng(451 + metric)
    centres = rng.standard_normal((60, d)).astype(np.float32)
    X = centres[rng.integers(0, 60, n)] + 0.3 * rng.standard_normal((n, d)).astype(np.float32)
    if metric == 0:
        X /= np.linalg.norm(X, axis=1, keepdims=True)
    if dtype == "f16":
        X = X.astype(np.float16)
    X = np.ascontiguousarray(X)
    Xg = torch.from_numpy(X).cuda()
    m = "ip" if metric == 0 else "l2"
    note("mfma sweep seeds", mode, dtype, m, d)
    if mode.startswith("order-overflow"):
        opt(sweep_sym_fcap=4, sweep_repair_max=1000 if mode.endswith("16") else 0)
    cand, cdist = B.knn_candidates(Xg, C, metric=m)
    opt(sweep_sym_fcap=0, sweep_repair_max=4, sweep_noseed=1)
    c0, d0 = B.knn_candidates(Xg, C, metric=m)
    opt(sweep_noseed=0)
    same_lists(f"mfma sweep seeds vs none {mode} {dtype} {m}", cand, cdist, c0.cpu().numpy(),
               d0.cpu().numpy(), 1e-6, 1e-6)
    assert torch.allclose(cdist, d0, rtol=1e-6, atol=1e-6)
    oc, od = oracle_lists(X, C, metric, ("seeded", metric, dtype, d))
    scale = 1.0 if metric == 0 else float(np.abs(od).max())
    same_lists(f"mfma sweep seeds vs oracle {mode} {dtype} {m} {d}", cand, cdist, oc, od,
               2e-6 * scale, 2e-5)
    assert np.allclose(cdist.cpu().numpy(), od, rtol=2e-5, atol=2e-6 * scale)
    assert not (cand.cpu().numpy() == np.arange(n)[:, None]).any()


@pytest.mark.parametrize("k", [15, 30, "noise", "noise10"])
@pytest.mark.parametrize("metric", [0, 1])
@pytest.mark.parametrize("dtype", ["f32", "f16"])
def test_ordered_sweep_prunes_empty_tiles_and_keeps_the_lists(opt, metric, dtype, k):
    """Clusters in the locality order: most tiles pair two clusters, and the
    panels' centres and radii prove them empty, so the ordered sweep scores
    far fewer tiles than the symmetric triangle -- and its lists are still
    those of the unpruned plain sweep and the oracle's.  With 15 clusters of
    2,000 rows each cluster spans about eight row panels; with 30 of 1,000
    the 58 pivots leave a few clusters without a pivot of their own, whose
    rows then share one with another cluster's, so some panels mix two
    clusters and prune only once their rows are split into groups.  With
    "noise10", 15 clusters and 10 rows far from all of them: under l2 the few
    panels holding those bound nothing and go dense (their tiles scored by the
    other panels after the bands, their rows repaired one-sided; under ip the
    normalised outliers are mere directions and some clustered ip panels go
    dense instead); with "noise", 1,500 such rows spread over most panels,
    too many to repair, and the bands keep those panels' tiles as they are.
    Every variant must give the plain sweep's lists."""
    opt(sweep_sym=1)
    from swann_amd import _lib
    n, d, C = 30000, 64, 24
    noisy = {"noise": 1500, "noise10": 10}.get(k, 0)
    rng = np.random.default_rng(461 + metric + (k if not noisy else 99 + noisy))
    kc = 15 if noisy else k
    centres = rng.standard_normal((kc, d)).astype(np.float32)
    X = centres[rng.integers(0, kc, n)] + 0.3 * rng.standard_normal((n, d)).astype(np.float32)
    if noisy:
        X[rng.choice(n, noisy, replace=False)] = 3.0 * rng.standard_normal((noisy, d)).astype(np.float32)
    if metric == 0:
        X /= np.linalg.norm(X, axis=1, keepdims=True)
    X = np.ascontiguousarray(X.astype(np.float16) if dtype == "f16" else X)
    Xg = torch.from_numpy(X).cuda()
    m = "ip" if metric == 0 else "l2"
    note("pruned ordered sweep", dtype, m, k)
    cand, cdist = B.knn_candidates(Xg, C, metric=m)
    nt = (n + 255) // 256
    tiles = int(_lib.lib().swann_sweep_tiles_scored())
    dense = int(_lib.lib().swann_sweep_dense_panels())
    note("pruned ordered sweep tiles scored", tiles, "of", nt * (nt + 1) // 2, "dense", dense)
    if k != "noise":
        assert 0 < tiles < 0.6 * nt * (nt + 1) // 2
    if k == "noise10" and metric == 1:
        assert 0 < dense <= 10          # the outliers' panels, scored after the bands
    if k == "noise":
        assert dense == 0               # too many to repair: left to the bands
    opt(sweep_noseed=1)
    c0, d0 = B.knn_candidates(Xg, C, metric=m)
    assert int(_lib.lib().swann_sweep_tiles_scored()) == nt * (nt + 1) // 2
    same_lists(f"pruned vs plain {dtype} {m} {k}", cand, cdist, c0.cpu().numpy(), d0.cpu().numpy(),
               1e-6, 1e-6)
    oc, od = oracle_lists(X, C, metric, ("pruned", metric, dtype, k))
    scale = 1.0 if metric == 0 else float(np.abs(od).max())
    same_lists(f"pruned vs oracle {dtype} {m} {k}", cand, cdist, oc, od, 2e-6 * scale, 2e-5)
    assert np.allclose(cdist.cpu().numpy(), od, rtol=2e-5, atol=2e-6 * scale)
    assert not (cand.cpu().numpy() == np.arange(n)[:, None]).any()


@pytest.mark.parametrize("d", [64, 256])
@pytest.mark.parametrize("sym", ["0", "1"])
@pytest.mark.parametrize("metric", [0, 1])
@pytest.mark.parametrize("dtype", ["f32", "f16"])
def test_mfma_sweep_with_duplicate_rows_matches_oracle(opt, metric, dtype, sym, d):
    """A larger sweep (n = 12,000: 47 row panels, 47 column tiles, several
    compactions per row) with rows 0..999 duplicated at 6000..6999, so many
    rows hold exact ties, some of them at the C-th place: the lists must be
    the oracle's, and each duplicated row must find its twin -- one-sided
    and symmetric (47 panels, 9 band launches)."""
    opt(sweep_sym=int(sym))
    n, C = 12000, 16
    X = gaussian(n, d, 421 + metric, metric == 0)
    if metric == 1:
        X = X * 2.0 + 0.5
    X[6000:7000] = X[0:1000]
    if dtype == "f16":
        X = X.astype(np.float16)
    Xg = torch.from_numpy(X).cuda()
    m = "ip" if metric == 0 else "l2"
    note("mfma sweep with duplicates", dtype, m, d)
    cand, cdist = B.knn_candidates(Xg, C, metric=m)
    oc, od = oracle_lists(X, C, metric, ("dup", metric, dtype, d))
    cc, cd = cand.cpu().numpy(), cdist.cpu().numpy()
    scale = 1.0 if metric == 0 else float(np.abs(od).max())
    same_lists(f"mfma sweep with duplicates {dtype} {m} sym={sym}", cc, cd, oc, od, 2e-6 * scale,
               2e-5)
    assert np.allclose(cd, od, rtol=2e-5, atol=2e-6 * scale)
    assert ((cc >= 0) & (cc < n)).all()
    assert not (cc == np.arange(n)[:, None]).any()
    assert (np.diff(cd, axis=1) >= 0).all()
    # each duplicated row finds its twin first (distance 0 for l2)
    twin = np.where(np.arange(n) < 1000, np.arange(n) + 6000,
                    np.where((np.arange(n) >= 6000) & (np.arange(n) < 7000), np.arange(n) - 6000, -1))
    rows = np.nonzero(twin >= 0)[0]
    assert (cc[rows] == twin[rows][:, None]).any(axis=1).all()


@pytest.mark.parametrize("metric", [0, 1])
@pytest.mark.parametrize("dtype", ["f32", "f16"])
def test_mfma_sweep_self_is_last_when_candidates_cover_the_corpus(metric, dtype):
    """C = n: every other row is a candidate and self comes last at 3.4e38
    (build.py:39 sets the self score so).  n = 48 is one row panel, so most
    of the sweep's column splits receive no column tile."""
    n, d = 48, 64
    X = gaussian(n, d, 411 + metric, metric == 0)
    if dtype == "f16":
        X = X.astype(np.float16)
    Xg = torch.from_numpy(X).cuda()
    note("mfma sweep C = n", dtype, metric)
    cand, cdist = B.knn_candidates(Xg, n, metric="ip" if metric == 0 else "l2")
    oc, od = O.knn_candidates(X.astype(np.float32), n, metric, nthreads=8)
    c = cand.cpu().numpy()
    assert (c[:, -1] == np.arange(n)).all()
    assert (cdist.cpu().numpy()[:, -1] == np.float32(3.4e38)).all()
    assert (oc[:, -1] == np.arange(n)).all()
    for r in range(n):
        assert sorted(c[r, :-1].tolist()) == sorted(set(range(n)) - {r})
    same_lists(f"mfma sweep C = n {dtype} {metric}", c, cdist.cpu().numpy(), oc, od, 2e-6, 2e-5)


def test_captured_search_replays_exactly():
    """The whole search path under hipGraph capture (selection, seed gather,
    init, advance, top-k, merge, overflow count), in a deterministic
    configuration (no shared table, bound or claims): recorded once, replayed
    with four different batches, with eager work and synchronisations between
    the replays; every replay equals the eager search bit for bit."""
    from swann_amd import _engine as E
    X, Q = corpus(n=4000, d=64, nq=64, seed=4)
    Xg = torch.from_numpy(X).cuda()
    index = swann.Index.build(Xg, degree=32, candidates=48)

    def run(Qb):
        ent = S.select_nearest(Qb, index._cat, 8, metric=0)
        seeds = index.catalogue[ent].to(torch.int32)
        ids, dist, st = E.search(index.X, index.G, Qb, seeds, k=10, L=16, B=24, metric=0,
                                 team_size=16, stop_eps=0.1, check=False)
        return ids, dist, st.overflow()

    static_q = torch.zeros((8, 64), device="cuda")
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        run(static_q)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        gi, gd, go = run(static_q)
    Qg = torch.from_numpy(Q).cuda()
    for rep in range(4):
        note("capture replay", rep)
        Qb = Qg[rep * 8:(rep + 1) * 8].contiguous()
        ei, ed, eo = run(Qb)                       # eager, on the same stream
        torch.cuda.synchronize()
        static_q.copy_(Qb)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(gi, ei) and torch.equal(gd.view(torch.int32), ed.view(torch.int32))
        assert int(go) == int(eo) == 0
        _ = (Qg @ Qg.T).sum().item()               # unrelated eager work between replays


def test_index_capture_matches_eager_search():
    """`Index.capture`: the production configuration (claims, bound -- racy
    by design) replayed on 64 batches agrees with the eager search on the same
    batches (recall within 0.005 over 1,024 queries), and its distances are
    exact."""
    X, Q = corpus(n=6000, d=96, nq=1024, seed=5)
    index = swann.Index.build(X, degree=32, candidates=48)
    cs = index.capture(16, k=10, branches=16, queue=16)
    Xd = X.astype(np.float64)
    truth = exact_topk(X, Q, 10)
    agree, rg, re = [], [], []
    for rep in range(Q.shape[0] // 16):
        sl = slice(rep * 16, (rep + 1) * 16)
        ei, _ = index.search(Q[sl], k=10, branches=16, queue=16)
        gi, gd = cs.run(Q[sl])
        torch.cuda.synchronize()
        gi, gd = gi.cpu().numpy(), gd.cpu().numpy()
        agree.append(np.mean([len(set(a) & set(b)) / 10 for a, b in zip(gi, ei)]))
        rg.append(recall(gi, truth[sl], 10)); re.append(recall(ei, truth[sl], 10))
        assert int(cs.overflow) == 0
        if rep < 4:
            for qi in range(16):
                for i, dv in zip(gi[qi], gd[qi]):
                    if i >= 0:
                        assert abs(dv - (1.0 - Q[rep * 16 + qi].astype(np.float64) @ Xd[i])) < 1e-5
    note("capture set agreement / recall graph / recall eager", np.mean(agree), np.mean(rg),
         np.mean(re))
    assert np.mean(agree) > 0.95
    assert abs(np.mean(rg) - np.mean(re)) <= 0.005       # 1,024 queries in 64 replays
    with pytest.raises(ValueError):
        cs.run(Q[:3])


@pytest.mark.parametrize("nq", [1, 2, 3, 5, 8, 64, 300])
@pytest.mark.parametrize("metric", [0, 1])
def test_select_small_and_large_batches_match_oracle(nq, metric):
    """Selection at every batch shape: the one-pass product for batches of up
    to 8 (16-byte loads, and element loads at d = 70), split-K partials for
    small grids, the radix top-E for rows up to 16384 and the chunked bitonic
    beyond; ties (duplicated catalogue rows) resolve to the lower index, as the oracle's
    (d, index) order.  With two or more queries, query 1 is NaN throughout:
    its distances cannot be ranked, so its E entries come in no stated order,
    but they are E distinct catalogue rows (both survivor sorts swap pairs
    whole), and the other queries' lists are unaffected."""
    rng = np.random.default_rng(100 + nq)
    for P, d, E in ((4096, 256, 32), (5000, 72, 128), (20000, 64, 40), (3000, 70, 16)):
        V = rng.standard_normal((P, d)).astype(np.float32)
        V[P // 2:P // 2 + 50] = V[:50]                     # exact duplicates -> ties
        Q = rng.standard_normal((nq, d)).astype(np.float32)
        Q[0] = V[7]
        if nq >= 2:
            Q[1] = np.nan
        idx = S.select_nearest(torch.from_numpy(Q).cuda(), torch.from_numpy(V).cuda(), E,
                               metric=metric).cpu().numpy()
        assert idx.shape == (nq, E)
        assert ((idx >= 0) & (idx < P)).all()
        assert (np.sort(idx, 1)[:, 1:] != np.sort(idx, 1)[:, :-1]).all()   # distinct
        if nq >= 2:
            keep = np.arange(nq) != 1
            Q, idx = Q[keep], idx[keep]
        want, _ = O.select_nearest(Q, V, E, metric, nthreads=8)
        Q64, V64 = Q.astype(np.float64), V.astype(np.float64)

        def dist(e):
            if metric == 0:
                return 1.0 - np.einsum("qd,qkd->qk", Q64, V64[e])
            return ((V64[e] - Q64[:, None, :]) ** 2).sum(-1)
        wd = dist(want)
        same_lists(f"select {nq} {metric} {P} {d} {E}", idx, dist(idx), want, wd,
                   2e-6 * float(np.abs(wd).max()), 2e-5)
        if metric == 1:
            # q = V[7], which has an exact duplicate at P//2 + 7: a tie at the
            # top, resolved to the lower index
            assert idx[0, 0] == 7 and idx[0, 1] == P // 2 + 7


@pytest.mark.parametrize("nq", [1, 5, 70])
def test_select_tiny_catalogues_match_oracle(nq):
    """Catalogues of 1 to 17 rows (the one-pass product's last workgroup
    mostly past P, the top-E over rows shorter than a wave) and E up to P:
    the same entries as the oracle, up to ties."""
    rng = np.random.default_rng(700 + nq)
    for P, d, E in ((1, 16, 1), (3, 20, 3), (17, 64, 5), (17, 7, 17)):
        V = rng.standard_normal((P, d)).astype(np.float32)
        Q = rng.standard_normal((nq, d)).astype(np.float32)
        for metric in (0, 1):
            idx = S.select_nearest(torch.from_numpy(Q).cuda(), torch.from_numpy(V).cuda(), E,
                                   metric=metric).cpu().numpy()
            want, _ = O.select_nearest(Q, V, E, metric, nthreads=8)
            assert idx.shape == (nq, E)
            Q64, V64 = Q.astype(np.float64), V.astype(np.float64)
            if metric == 0:
                dist = lambda e: 1.0 - np.einsum("qd,qkd->qk", Q64, V64[e])  # noqa: E731
            else:
                dist = lambda e: ((V64[e] - Q64[:, None, :]) ** 2).sum(-1)  # noqa: E731
            wd = dist(want)
            same_lists(f"tiny select {nq} {metric} {P} {d} {E}", idx, dist(idx), want, wd,
                       2e-6 * max(float(np.abs(wd).max()), 1.0), 2e-5)


@pytest.mark.parametrize("tag,metric", [("ip", 0), ("l2", 1)])
def test_prune_per_node_degree_and_protect_match_reference(tag, metric):
    """robust_prune(deg_per_node=, protect=) and add_reverse(deg_per_node=)
    against the reference's CPU-torch build.py (refbuild_extras.npz) and,
    on identical inputs, the oracle."""
    g = golden("refbuild_extras.npz")
    X = regen(800, 24, 23 if tag == "ip" else 24, tag == "ip", g[f"{tag}_X_sha"])
    m = "ip" if metric == 0 else "l2"
    Xg = torch.from_numpy(X).cuda()
    rc = g[f"{tag}_cand"].astype(np.int32); rd = g[f"{tag}_cdist"]
    dpn = g[f"{tag}_dpn"].astype(np.int32); prot = g[f"{tag}_prot"]
    rcg, rdg = torch.from_numpy(rc).cuda(), torch.from_numpy(rd).cuda()
    dpng, protg = torch.from_numpy(dpn).cuda(), torch.from_numpy(prot).cuda()
    for key, kw, okw in (("Gd", dict(deg_per_node=dpng), dict(deg_per_node=dpn)),
                         ("Gm", dict(protect=protg), dict(protect=prot)),
                         ("Gb", dict(deg_per_node=dpng, protect=protg),
                          dict(deg_per_node=dpn, protect=prot))):
        got = B.robust_prune(Xg, rcg, rdg, 12, alpha=1.2, metric=m, **kw).cpu().numpy()
        want = g[f"{tag}_{key}"].astype(np.int32)
        assert got.shape == want.shape
        ora = O.robust_prune(X, rc, rd, 12, 1.2, metric, nthreads=8, **okw)
        note("prune extras", tag, key, int((got != want).any(1).sum()),
             int((got != ora).any(1).sum()))
        assert np.array_equal(got, want), key
        assert np.array_equal(got, ora), key
    Rd = B.add_reverse(Xg, torch.from_numpy(g[f"{tag}_Gd"].astype(np.int32)).cuda(), 12,
                       alpha=1.2, deg_per_node=dpng, metric=m).cpu().numpy()
    bad = untied_graph_rows(Rd, g[f"{tag}_Rd"].astype(np.int32), X, metric)
    note("reverse dpn", tag, bad)
    assert bad == []


@pytest.mark.parametrize("C", [48, 100])
@pytest.mark.parametrize("dtype", ["f16", "f32", "f32-fp32gram"])
@pytest.mark.parametrize("metric", [0, 1])
def test_prune_mfma_gram_matches_simt_and_oracle(metric, dtype, C, opt):
    """The prune's Gram on MFMA -- fp16 rows: exact products, fp32 sums
    (32x32x16 f16); fp32 rows: split fp16 planes (hi.hi + (hi.lo + lo.hi) /
    2^11 on 32x32x16 f16), or with option prune_f32 fp32 products and sums
    (32x32x2 f32); nodes grouped by shared candidates -- keeps
    the same rows as the fp32 SIMT Gram (option prune_simt) and the oracle
    (double dots) up to near-ties.  d = 80 leaves a ragged last K group for
    fp16; C = 48 fills two of the four 32-row blocks (three of the ten Gram
    tiles), C = 100 all four with a ragged last (every tile, every wave);
    per-node caps and protect ride along."""
    if dtype == "f32-fp32gram":
        opt(prune_f32=1)
    X = gaussian(3000, 80, 71 + metric, metric == 0)
    if metric == 1:
        X = X * 2.0 + 0.5
    X16 = X.astype(np.float16) if dtype == "f16" else X.astype(np.float32)
    m = "ip" if metric == 0 else "l2"
    Xg = torch.from_numpy(X16).cuda()
    cand, cdist = B.knn_candidates(Xg, C, metric=m)
    rng = np.random.default_rng(8)
    dpn = np.where(rng.random(3000) < 0.2, 32, 20).astype(np.int32)
    prot = rng.random((3000, C)) < 0.1
    kw = dict(alpha=1.2, metric=m, deg_per_node=torch.from_numpy(dpn).cuda(),
              protect=torch.from_numpy(prot).cuda())
    g_mfma = B.robust_prune(Xg, cand, cdist, 24, **kw).cpu().numpy()
    opt(prune_simt=1)
    g_simt = B.robust_prune(Xg, cand, cdist, 24, **kw).cpu().numpy()
    ora = O.robust_prune(X16.astype(np.float32), cand.cpu().numpy(), cdist.cpu().numpy(), 24,
                         1.2, metric, nthreads=8, deg_per_node=dpn, protect=prot)
    Xo, cn, cdn = X16.astype(np.float32), cand.cpu().numpy(), cdist.cpu().numpy()
    kw = dict(alpha=1.2, metric=metric, deg_per_node=dpn, protect=prot)
    a = untied_prune_rows(g_mfma, g_simt, Xo, cn, cdn, 24, **kw)
    b = untied_prune_rows(g_mfma, ora, Xo, cn, cdn, 24, **kw)
    note("prune mfma vs simt / oracle: rows differing", int((g_mfma != g_simt).any(1).sum()),
         int((g_mfma != ora).any(1).sum()), "beyond near-ties", a, b)
    assert a == [] and b == []


def test_many_branches_keep_recall_in_every_layout(opt):
    """128 claiming branches a query on a 100,000 x 512 low-rank corpus.  With
    1024 threads a branch one XCD holds only 32 branches at once; placing a
    query's 128 branches on one XCD made them run in rounds, the late ones
    finding the nodes claimed and the bound tightened, and recall@10 fell
    from 0.98 to 0.86.  Every layout stays within 0.07 of the one-wave one,
    whose 128 branches fit on one XCD."""
    n, d, r, nq = 100_000, 512, 128, 64
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(4007)
    W = torch.randn((r, d), generator=g, device=dev)

    def draw(m):
        x = (torch.randn((m, r), generator=g, device=dev) @ W / r ** 0.5
             + 0.1 * torch.randn((m, d), generator=g, device=dev))
        return x / x.norm(dim=1, keepdim=True)
    X32, Q = draw(n), draw(nq)
    truth = torch.topk(Q @ X32.T, 10, dim=1).indices.cpu().numpy()
    X = X32.half()
    del X32
    G = B.build_graph(X, metric="ip", degree=32, candidates=64)
    ix = swann.Index(X, G, metric="ip")
    rec = {}
    for blk in ("64", "256", "1024"):
        opt(search_block=int(blk))
        ids = ix.search(Q, k=10, branches=128, queue=12, team=32)[0]
        rec[blk] = recall(ids, truth, 10)
    note("128 branches recall by layout", rec)
    assert rec["64"] > 0.9
    assert min(rec["256"], rec["1024"]) >= rec["64"] - 0.07


def test_claims_fall_back_to_the_table_when_bits_do_not_fit(monkeypatch):
    """Index.search shares claims as one bit per row while the batch's bits
    fit a quarter of the free device memory, else as the reference's (id, d)
    table; both layouts decide claims alike, so recall agrees within 0.01 on
    the same seeds, and a layout is kept per (batch, branches, budget)."""
    X, Q = corpus(nq=400, seed=5)
    index = swann.Index.build(X, degree=48, candidates=64)
    truth = exact_topk(X, Q, 10)
    cfg = swann.SearchConfig(branches=32, budget=48)
    assert index._claims(Q.shape[0], cfg) == (True, 8192)
    r_bits = recall(index.search(Q, k=10, branches=32, budget=48)[0], truth, 10)
    small = swann.Index(index.X, index.G, metric="ip", catalogue=index.catalogue)
    monkeypatch.setattr(torch.cuda, "mem_get_info", lambda *a, **k: (4 * 400 * 8192 // 8 - 4,
                                                                      1 << 40))
    bits, slots = small._claims(Q.shape[0], cfg)
    assert not bits and slots == swann._engine.cache_size(32, 48, 48)
    ids, _, st, _ = small.search_async(Q, k=10, branches=32, budget=48)
    assert st.cache_d.numel() > 0 and st.table_slots == slots
    r_table = recall(ids.cpu().numpy(), truth, 10)
    note("claims layouts: bits", r_bits, "table", r_table)
    assert abs(r_bits - r_table) <= 0.01
    monkeypatch.undo()
    assert small._claims(Q.shape[0], cfg) == (False, slots)      # kept once decided


def test_mfma_probe_reports_a_rate_below_the_published_peak():
    """The measurement probe's FLOP count is its launch's MFMA work
    (blocks x 4 waves x iters x 4 MFMAs x 2*32*32*16), and the rate it gives
    is positive and below the published dense fp16 peak."""
    sys.path.insert(0, str(ROOT))
    import bench
    from swann_amd import _lib
    assert _lib.lib().swann_mfma_probe_flop(10, 3) == 3 * 4 * 10 * 4 * 2 * 32 * 32 * 16
    rate = bench.mfma_probe(torch.device("cuda:0"), seconds=0.05)
    note("mfma probe TFLOP/s", rate / 1e12)
    assert 0.2e15 < rate < bench.MFMA_F16_PEAK
