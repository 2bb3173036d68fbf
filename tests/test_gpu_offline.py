"""The offline builder's extras on the GPU (offline/build_graph.py) against the
oracle and the reference's CPU-torch vectors, plus the corpus layout and the
offline command line end to end."""
import json
import sys

import numpy as np
import pytest
import torch

import oracle as O
from test_oracle_helpers import untied_rows
from conftest import gaussian, golden, regen

pytestmark = pytest.mark.gpu

swann = pytest.importorskip("swann_amd")
from swann_amd import build as B  # noqa: E402
from swann_amd import corpus as CO  # noqa: E402
from swann_amd import offline as OF  # noqa: E402


def note(*a):
    print("[case]", *a, flush=True)
    sys.stdout.flush()


@pytest.mark.parametrize("tag,metric", [("ip", 0), ("l2", 1)])
def test_offline_extras_match_reference_and_oracle(tag, metric):
    g = golden("refbuild_extras.npz")
    X = regen(800, 24, 23 if tag == "ip" else 24, tag == "ip", g[f"{tag}_X_sha"])
    m = "ip" if metric == 0 else "l2"
    Xg = torch.from_numpy(X).cuda()
    cand = g[f"{tag}_cand"].astype(np.int32)
    cg = torch.from_numpy(cand).cuda()
    note("offline extras", tag)
    assert np.array_equal(OF.mutual_rank(cg, 8).cpu().numpy(), g[f"{tag}_prot"])
    ci, cd = OF.candidates_from_graph(Xg, torch.from_numpy(g[f"{tag}_R"].astype(np.int32)).cuda(),
                                      12, metric=m)
    wi, wd = g[f"{tag}_cg"].astype(np.int32), g[f"{tag}_cgd"]
    bad = untied_rows(ci.cpu().numpy(), wi, wd, cd.cpu().numpy(), atol=2e-5, rtol=2e-5)
    note("candidates_from_graph", tag, "rows beyond ties", bad)
    assert bad == []
    assert np.allclose(cd.cpu().numpy(), wd, rtol=2e-5, atol=2e-5)
    Gp24 = torch.from_numpy(g[f"{tag}_Gp24"].astype(np.int32)).cuda()
    for rule in ("near", "far", "bridge"):
        f = OF.fill_degree(Gp24, cg, rule=rule).cpu().numpy()
        assert np.array_equal(f, g[f"{tag}_fill_{rule}"].astype(np.int32)), rule
    R = torch.from_numpy(g[f"{tag}_R"].astype(np.int32)).cuda()
    got = OF.enforce_min_in(Xg, R.clone(), cg, 8, metric=m, rounds=4).cpu().numpy()
    want = O.enforce_min_in(g[f"{tag}_R"].astype(np.int32), cand, 8, 4)
    assert np.array_equal(got, want)


def test_fill_chunks_see_earlier_chunks():
    """Chunked fill on a larger graph: the GPU equals the oracle for every
    rule and chunk size (later chunks read the rows earlier chunks filled)."""
    X = gaussian(3000, 32, 91, True)
    Xg = torch.from_numpy(X).cuda()
    cand, cdist = B.knn_candidates(Xg, 40, metric="ip")
    G = B.robust_prune(Xg, cand, cdist, 24, alpha=1.2, metric="ip")
    for rule in ("near", "far", "bridge"):
        for chunk in (1, 100, 1024, 5000):
            got = OF.fill_degree(G, cand, rule=rule, chunk=chunk).cpu().numpy()
            want = O.fill_degree(G.cpu().numpy(), cand.cpu().numpy(), rule, chunk=chunk)
            assert np.array_equal(got, want), (rule, chunk)


def test_min_in_on_a_larger_graph_matches_oracle():
    X = gaussian(4000, 32, 92, False)
    Xg = torch.from_numpy(X).cuda()
    cand, cdist = B.knn_candidates(Xg, 48, metric="l2")
    G = B.build_graph(Xg, metric="l2", degree=16, candidates=48)
    got = OF.enforce_min_in(Xg, G.clone(), cand, 12, metric="l2", rounds=3).cpu().numpy()
    want = O.enforce_min_in(G.cpu().numpy(), cand.cpu().numpy(), 12, 3)
    assert np.array_equal(got, want)
    indeg = np.bincount(got[got >= 0].astype(np.int64), minlength=4000)
    note("min_in below floor", int((indeg < 12).sum()))


@pytest.mark.parametrize("metric", ["ip", "l2"])
def test_corpus_layout_and_offline_cli(tmp_path, metric):
    """write_corpus writes the shared layout with exact ground truth; the
    offline builder reads it and writes G_*.npy, *_deg.npy and *.json; the
    built graph searches well through the public interface."""
    rng = np.random.default_rng(12)
    X = rng.standard_normal((3000, 61)).astype(np.float32)     # padded to 64
    Q = rng.standard_normal((200, 61)).astype(np.float32)
    d = CO.write_corpus(tmp_path / "c", X, Q, metric=metric, k=10, deg=24, seed=0)
    man, Xs, Qs, ids, sim = CO.load_corpus(d, "test")
    assert man["d"] == 64 and man["d_original"] == 61 and Xs.shape == (3000, 64)
    assert Qs.shape == (100, 64) and ids.shape == (100, 10)
    Xf = np.asarray(Xs, dtype=np.float64); Qf = Qs.astype(np.float64)
    if metric == "ip":
        want = np.argsort(-(Qf @ Xf.T), axis=1, kind="stable")[:, :10]
        assert np.allclose(sim, np.take_along_axis(Qf @ Xf.T, ids.astype(np.int64), 1), atol=1e-5)
    else:
        dd = ((Qf[:, None, :] - Xf[None]) ** 2).sum(-1)
        want = np.argsort(dd, axis=1, kind="stable")[:, :10]
    wdist = np.take_along_axis(-(Qf @ Xf.T) if metric == "ip" else dd, want, 1)
    gdist = np.take_along_axis(-(Qf @ Xf.T) if metric == "ip" else dd, ids.astype(np.int64), 1)
    assert untied_rows(ids.astype(np.int64), want, wdist, gdist, atol=1e-5, rtol=1e-5) == []
    CO.write_pool(d, "random4k", np.sort(rng.permutation(3000)[:256]))
    OF.main(["--data", str(d), "--D", "24", "--cand", "48", "--fill", "bridge",
             "--mutual", "8", "--min-in", "6", "--pool-boost", "8", "--out", "G_ours.npy"])
    G = np.load(d / "G_ours.npy")
    meta = json.loads((d / "G_ours.json").read_text())
    assert G.shape == (3000, 32) and G.dtype == np.int32           # width = D + boost
    assert meta["deg"] == 24 and meta["fill"] == "bridge" and meta["pool_boost"] == 8
    assert np.array_equal(np.load(d / "G_ours_deg.npy"), (G >= 0).sum(1))
    # candidates from an existing graph
    OF.main(["--data", str(d), "--D", "24", "--cand", "24", "--cand-graph", "G_knn.npy",
             "--out", "G_cg.npy"])
    index = swann.Index(torch.from_numpy(np.array(Xs, dtype=Xs.dtype, copy=True)).cuda(),
                        torch.from_numpy(np.load(d / "G_cg.npy")).cuda(), metric=metric)
    got, _ = index.search(Qs, k=10, branches=16, queue=24)
    r = np.mean([len(set(a) & set(b)) / 10 for a, b in zip(got, ids)])
    note("corpus search recall", metric, r)
    assert r > 0.9
