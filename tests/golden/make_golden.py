"""Write the golden vectors under tests/golden/ from the reference's own CPU code.

Run in the build container only (it reads /root/reference, which does not
exist on the GPU box):

    python tests/golden/make_golden.py

What is imported from the reference, and why nothing else pins it:
  * swann/_refcpu.py (numpy): the branch walk -- round-robin turns, per-lineage
    retirement, the eps stop rule and the merge -- whose trajectories no closed
    form fixes; plus fp16 distances with vec=8.
  * swann/build.py on CPU tensors: knn_candidates / robust_prune / add_reverse,
    whose torch.topk / argsort tie behaviour only the code itself defines,
    including robust_prune's per-node degrees and protect mask.
  * offline/build_graph.py on CPU tensors: candidates_from_graph,
    mutual_rank, fill_degree and enforce_min_in (the offline builder's
    extras), whose selection orders only the code defines.
  * swann/_select.py select_nearest (fp32, CPU) and
    swann/_engine.py _merge_branches_tensor: the C1 seeds and merged answers.

Inputs are generated here, platform-stably (float64 normalisation, then cast),
and stored or hashed (SHA-256) so a test can tell if its regenerated inputs
drifted. Outputs are stored as small compressed .npz files. The reference's
source is not copied anywhere: only inputs and outputs are written.
"""
from __future__ import annotations

import hashlib
import importlib.util
import multiprocessing as mp
import sys
from pathlib import Path

import numpy as np

REF = Path("/root/reference")
OUT = Path(__file__).resolve().parent

IP, L2 = 0, 1


def _load(name, path, package=None):
    spec = importlib.util.spec_from_file_location(
        name, path, submodule_search_locations=[str(path.parent)] if package else None)
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def ref_offline():
    return _load("ref_offline_build", REF / "offline" / "build_graph.py")


def ref_modules():
    refcpu = _load("ref_refcpu", REF / "swann" / "_refcpu.py")
    build = _load("ref_build", REF / "swann" / "build.py")
    pkg = _load("ref_swann", REF / "swann" / "__init__.py", package=True)
    select = sys.modules["ref_swann._select"] if "ref_swann._select" in sys.modules else \
        importlib.import_module("ref_swann._select")
    engine = sys.modules["ref_swann._engine"]
    return refcpu, build, select, engine, pkg


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def gaussian(n, d, seed, normalise):
    """N(0,1) float32 rows; normalised in float64 and cast once, so the bytes do
    not depend on numpy's float32 SIMD reduction order."""
    X = np.random.default_rng(seed).standard_normal((n, d), dtype=np.float32)
    if normalise:
        X64 = X.astype(np.float64)
        X = (X64 / np.sqrt((X64 * X64).sum(1, keepdims=True))).astype(np.float32)
    return np.ascontiguousarray(X)


def norm_spread(X, sigma, seed):
    """Rows of X scaled by exp(sigma * N(0,1)) in float64, then cast: an
    inner-product corpus whose norms differ, so hubs collect many in-edges."""
    s = np.exp(sigma * np.random.default_rng(seed).standard_normal((X.shape[0], 1)))
    return np.ascontiguousarray((X.astype(np.float64) * s).astype(np.float32))


def knn_graph(X, deg, metric):
    """Exact kNN graph in float64 (the reference toy graph, tests/test_engine.py:24-34)."""
    X64 = X.astype(np.float64)
    if metric == IP:
        sim = X64 @ X64.T
    else:
        sq = (X64 * X64).sum(1)
        sim = -(sq[:, None] - 2 * X64 @ X64.T + sq[None, :])
    np.fill_diagonal(sim, -np.inf)
    return np.ascontiguousarray(np.argsort(-sim, axis=1, kind="stable")[:, :deg].astype(np.int32))


def pack_queue(state, L):
    ids = np.full(L, -1, np.int32); dist = np.full(L, np.nan, np.float32)
    expd = np.zeros(L, np.uint8); lin = np.zeros(L, np.uint8)
    for s, e in enumerate(state["queue"]):
        ids[s], dist[s], expd[s], lin[s] = e[0], np.float32(e[1]), int(e[2]), e[3]
    c = state["counters"]
    return ids, dist, expd, lin, np.array([c["expansions"], c["dist_evals"], c["exhausted"]], np.int32)


# ---------------------------------------------------------------------------
def make_branch(refcpu):
    """tests/test_engine.py:42-78 (teams), :263-288 (multiseed), :291-316 (eps)."""
    out = {}
    for metric, tag in ((IP, "ip"), (L2, "l2")):
        X = gaussian(2000, 64, 0, metric == IP)
        G = knn_graph(X, 32, metric)
        rng = np.random.default_rng(7)
        nq, J, L, B = 5, 3, 16, 12
        Q = gaussian(nq, 64, 1007, metric == IP)
        seeds = rng.integers(0, 2000, size=(nq, J)).astype(np.int32)
        out[f"{tag}_X_sha"] = np.array(sha(X)); out[f"{tag}_G"] = G.astype(np.int16)
        out[f"{tag}_Q"] = Q; out[f"{tag}_seeds"] = seeds
        for team in (4, 8, 16, 32):
            R = [[pack_queue(refcpu.run(X, G, Q[q], int(seeds[q, j]), L=L, B=B,
                                        metric=metric, team=team), L)
                  for j in range(J)] for q in range(nq)]
            for f, name in enumerate(("ids", "dist", "expanded", "lineage", "counters")):
                out[f"{tag}_t{team}_{name}"] = np.array([[R[q][j][f] for j in range(J)]
                                                         for q in range(nq)])
    # several seeds in one branch, both policies (IP toy of seed 53)
    X = gaussian(2000, 64, 53, True); G = knn_graph(X, 32, IP)
    rng = np.random.default_rng(59)
    nq, V, L, B = 4, 6, 32, 20
    Q = gaussian(nq, 64, 1059, True)
    seeds = rng.integers(0, 2000, (nq, V)).astype(np.int32)
    out["ms_X_sha"] = np.array(sha(X)); out["ms_G"] = G.astype(np.int16)
    out["ms_Q"] = Q; out["ms_seeds"] = seeds
    for pol in (0, 1):
        R = [pack_queue(refcpu.run(X, G, Q[q], list(seeds[q]), L=L, B=B, policy=pol), L)
             for q in range(nq)]
        for f, name in enumerate(("ids", "dist", "expanded", "lineage", "counters")):
            out[f"ms_p{pol}_{name}"] = np.array([r[f] for r in R])
    # per-lineage early stop under round robin
    X = gaussian(2000, 64, 71, True); G = knn_graph(X, 32, IP)
    rng = np.random.default_rng(73)
    nq, V, L, B, k = 4, 4, 32, 64, 10
    Q = gaussian(nq, 64, 1073, True)
    seeds = rng.integers(0, 2000, (nq, V)).astype(np.int32)
    out["es_X_sha"] = np.array(sha(X)); out["es_G"] = G.astype(np.int16)
    out["es_Q"] = Q; out["es_seeds"] = seeds
    for e, eps in enumerate((0.0, 0.1, 0.25)):
        R = [pack_queue(refcpu.run(X, G, Q[q], list(seeds[q]), L=L, B=B, policy=1,
                                   stop_eps=eps, kstop=k), L) for q in range(nq)]
        for f, name in enumerate(("ids", "dist", "expanded", "lineage", "counters")):
            out[f"es_e{e}_{name}"] = np.array([r[f] for r in R])
    np.savez_compressed(OUT / "refcpu_branch.npz", **out)
    print("refcpu_branch.npz", sum(v.nbytes for v in out.values()), "bytes raw")


def make_distance(refcpu):
    """Distances alone: odd dimensions (tails), every team, and fp16 with vec=8
    (the kernel's fp16 layout, local_search.cu:131-133, which _refcpu.run never
    passes but team_distance accepts)."""
    rng = np.random.default_rng(101)
    out = {}
    cases = []
    for d in (1, 3, 4, 7, 8, 37, 64, 100, 128, 250, 512):
        for metric in (IP, L2):
            for team in (4, 8, 16, 32):
                q = rng.standard_normal(d).astype(np.float32)
                x = rng.standard_normal(d).astype(np.float32)
                x16 = x.astype(np.float16)
                v32 = refcpu.team_distance(q, x, metric, team, 4)
                v16 = refcpu.team_distance(q, x16.astype(np.float32), metric, team, 8)
                cases.append((d, metric, team, q, x, x16, v32, v16))
    out["n"] = np.array(len(cases))
    for i, (d, metric, team, q, x, x16, v32, v16) in enumerate(cases):
        out[f"c{i}_meta"] = np.array([d, metric, team], np.int32)
        out[f"c{i}_q"] = q; out[f"c{i}_x"] = x; out[f"c{i}_x16"] = x16
        out[f"c{i}_d32"] = np.float32(v32); out[f"c{i}_d16"] = np.float32(v16)
    np.savez_compressed(OUT / "refcpu_distance.npz", **out)
    print("refcpu_distance.npz", len(cases), "cases")


def make_build_small(build):
    """The three build stages on CPU tensors (build.py:28-150)."""
    import torch
    out = {}
    for metric, tag in ((IP, "ip"), (L2, "l2")):
        X = gaussian(1000, 24, 211 + metric, metric == IP)
        Xt = torch.from_numpy(X)
        m = "ip" if metric == IP else "l2"
        cand, cdist = build.knn_candidates(Xt, 32, metric=m)
        Gp = build.robust_prune(Xt, cand, cdist, 16, alpha=1.2, metric=m)
        Gf = build.add_reverse(Xt, Gp, 16, alpha=1.2, metric=m)
        out[f"{tag}_X"] = X
        out[f"{tag}_cand"] = cand.numpy().astype(np.int16)
        out[f"{tag}_cdist"] = cdist.numpy()
        out[f"{tag}_Gp"] = Gp.numpy().astype(np.int16)
        out[f"{tag}_Gf"] = Gf.numpy().astype(np.int16)
    np.savez_compressed(OUT / "refbuild_small.npz", **out)
    print("refbuild_small.npz written")


def reverse_cut_case(metric, n=300, d=100):
    """A hand-made graph on which add_reverse's cut and in-edge order decide
    the result.  Node 0 lists the 96 cluster nodes 1..96, which sit close
    together and block one another in the prune; the 70 far nodes 97..166
    each list node 0, so node 0 has 70 in-sources, of which the first 64 in
    source order join its union; the far nodes lie in orthogonal directions
    and block nothing.  The union is 160 wide: the cut to 128 keeps the
    nearest 32 far nodes, so node 0 ends with 1 + 32 neighbours (1 + 64
    without the cut, others with another in-edge order).  Other rows link
    at random, never to node 0."""
    rng = np.random.default_rng(971 + (metric == "ip"))
    X = np.zeros((n, d), np.float64)
    e = np.eye(d)
    if metric == "l2":
        X[0] = 0.001 * rng.standard_normal(d)
        X[1:97] = e[1] + 0.05 * rng.standard_normal((96, d))
        for k in range(70):
            X[97 + k] = (2.0 + 0.01 * k) * e[2 + k]
        X[167:] = rng.standard_normal((n - 167, d))
    else:
        X[0] = e[0]
        c = (e[0] + e[1]) / np.sqrt(2.0)
        X[1:97] = c + 0.02 * rng.standard_normal((96, d))
        for k in range(70):
            a = 0.3 - 0.002 * k
            X[97 + k] = a * e[0] + np.sqrt(1 - a * a) * e[2 + k]
        X[167:] = rng.standard_normal((n - 167, d))
        X /= np.linalg.norm(X, axis=1, keepdims=True)
    G = np.full((n, 96), -1, np.int32)
    G[0] = np.arange(1, 97)
    for u in range(1, n):
        row = rng.choice(np.arange(1, n), size=40, replace=False)
        row = row[row != u][:39]
        if 97 <= u < 167:
            row = np.r_[0, row[:38]]
        G[u, :len(row)] = row
    return np.ascontiguousarray(X.astype(np.float32)), G


def make_build_deg96(build):
    """The build at the reference API's defaults (build.py:153-171,
    index.py:76): candidates=128, degree=96, alpha=1.2, max_in=64.  The
    reverse pass's union is then 96 + 64 = 160 wide and add_reverse cuts it
    to its 128 nearest before the re-prune (build.py:138-148); both corpora
    are chosen so that cut binds on many rows (l2: 200 of 2,000; ip: 136)."""
    import torch
    out = {}
    cases = (("l2", "l2", gaussian(2000, 128, 961, False)),
             ("ip", "ip", norm_spread(gaussian(2000, 256, 962, True), 0.2, 963)))
    for tag, m, X in cases:
        Xt = torch.from_numpy(X)
        cand, cdist = build.knn_candidates(Xt, 128, metric=m)
        Gp = build.robust_prune(Xt, cand, cdist, 96, alpha=1.2, metric=m)
        Gf = build.add_reverse(Xt, Gp, 96, alpha=1.2, metric=m)
        out.update({f"{tag}_X_sha": np.array(sha(X)), f"{tag}_cand": cand.numpy().astype(np.int16),
                    f"{tag}_cdist": cdist.numpy(), f"{tag}_Gp": Gp.numpy().astype(np.int16),
                    f"{tag}_Gf": Gf.numpy().astype(np.int16)})
    for tag, m in (("adv_l2", "l2"), ("adv_ip", "ip")):
        X, G = reverse_cut_case(m)
        Gf = build.add_reverse(torch.from_numpy(X), torch.from_numpy(G), 96, alpha=1.2, metric=m)
        out.update({f"{tag}_X": X, f"{tag}_G": G.astype(np.int16),
                    f"{tag}_Gf": Gf.numpy().astype(np.int16)})
    np.savez_compressed(OUT / "refbuild_deg96.npz", **out)
    print("refbuild_deg96.npz written")


_C1 = {}


def _c1_run(args):
    q, j = args
    refcpu, X, G, Q, seeds = (_C1[k] for k in ("refcpu", "X", "G", "Q", "seeds"))
    st = refcpu.run(X, G, Q[q], int(seeds[q, j]), L=12, B=64, metric=IP, team=16,
                    stop_eps=0.05, kstop=10)
    return q, j, pack_queue(st, 12)


def make_build_extras(build, offline):
    """Per-node degrees, the protect mask and the offline extras on CPU
    tensors (build.py:46-150, offline/build_graph.py:72-386), n = 800."""
    import contextlib
    import io
    import torch
    out = {}
    for tag, metric in (("ip", "ip"), ("l2", "l2")):
        X = gaussian(800, 24, 23 if tag == "ip" else 24, tag == "ip")
        Xt = torch.from_numpy(X)
        cand, cdist = build.knn_candidates(Xt, 32, metric=metric)
        rng = np.random.default_rng(5)
        dpn = torch.from_numpy(np.where(rng.random(800) < 0.1, 20, 12).astype(np.int32))
        prot = offline.mutual_rank(cand, 8)
        Gp = build.robust_prune(Xt, cand, cdist, 12, alpha=1.2, metric=metric)
        Gd = build.robust_prune(Xt, cand, cdist, 12, alpha=1.2, deg_per_node=dpn, metric=metric)
        Gm = build.robust_prune(Xt, cand, cdist, 12, alpha=1.2, metric=metric, protect=prot)
        Gb = build.robust_prune(Xt, cand, cdist, 12, alpha=1.2, deg_per_node=dpn,
                                metric=metric, protect=prot)
        Rd = build.add_reverse(Xt, Gd, 12, alpha=1.2, deg_per_node=dpn, metric=metric)
        R = build.add_reverse(Xt, Gp, 12, alpha=1.2, metric=metric)
        cg, cgd = offline.candidates_from_graph(Xt, R, 12, metric=metric)
        Gp24 = build.robust_prune(Xt, cand, cdist, 24, alpha=1.2, metric=metric)
        fills = {rule: offline.fill_degree(Gp24, cand, rule=rule).numpy().astype(np.int16)
                 for rule in ("near", "far", "bridge")}
        with contextlib.redirect_stdout(io.StringIO()):
            Gmin = offline.enforce_min_in(Xt, R.clone(), cand, 8, metric=metric, rounds=4)
        out.update({f"{tag}_X_sha": np.array(sha(X)), f"{tag}_cand": cand.numpy().astype(np.int16),
                    f"{tag}_cdist": cdist.numpy(), f"{tag}_dpn": dpn.numpy().astype(np.int16),
                    f"{tag}_prot": prot.numpy(), f"{tag}_Gp": Gp.numpy().astype(np.int16),
                    f"{tag}_Gd": Gd.numpy().astype(np.int16), f"{tag}_Gm": Gm.numpy().astype(np.int16),
                    f"{tag}_Gb": Gb.numpy().astype(np.int16), f"{tag}_R": R.numpy().astype(np.int16),
                    f"{tag}_Rd": Rd.numpy().astype(np.int16),
                    f"{tag}_cg": cg.numpy().astype(np.int16), f"{tag}_cgd": cgd.numpy(),
                    f"{tag}_Gmin": Gmin.numpy().astype(np.int16),
                    f"{tag}_Gp24": Gp24.numpy().astype(np.int16)})
        for rule, g in fills.items():
            out[f"{tag}_fill_{rule}"] = g
    np.savez_compressed(OUT / "refbuild_extras.npz", **out)
    print("refbuild_extras.npz written")


def make_c1(refcpu, build, select, engine):
    """10k x 128 fp32 IP, D=32 cand=64 alpha=1.2, 200
    queries, 8 branches each searched independently by _refcpu (claims off),
    L=12 B=64 eps=0.05 team=16 k=10."""
    import torch
    X = gaussian(10000, 128, 0, True)
    Q = gaussian(200, 128, 1, True)
    Xt = torch.from_numpy(X)
    cand, cdist = build.knn_candidates(Xt, 64, metric="ip")
    Gp = build.robust_prune(Xt, cand, cdist, 32, alpha=1.2, metric="ip")
    G = build.add_reverse(Xt, Gp, 32, alpha=1.2, metric="ip").numpy().astype(np.int32)
    cat = np.sort(np.random.default_rng(0).permutation(10000)[:4096]).astype(np.int64)
    Vp = select.pool_vectors(Xt, torch.from_numpy(cat))
    ent = select.select_nearest(torch.from_numpy(Q), Vp, 8, metric=IP, precision="fp32")
    seeds = cat[ent.numpy()].astype(np.int32)                    # [200, 8]
    _C1.update(refcpu=refcpu, X=X, G=G, Q=Q, seeds=seeds)
    jobs = [(q, j) for q in range(200) for j in range(8)]
    ids = np.zeros((200, 8, 12), np.int32); dist = np.zeros((200, 8, 12), np.float32)
    expd = np.zeros((200, 8, 12), np.uint8); ctr = np.zeros((200, 8, 3), np.int32)
    with mp.get_context("fork").Pool(8) as pool:
        for q, j, (i_, d_, e_, _l, c_) in pool.imap_unordered(_c1_run, jobs, chunksize=8):
            ids[q, j], dist[q, j], expd[q, j], ctr[q, j] = i_, d_, e_, c_
    kk = 10
    bi = torch.from_numpy(ids[:, :, :kk].copy()); bd = torch.from_numpy(dist[:, :, :kk].copy())
    bd = torch.where(bi >= 0, bd, torch.full_like(bd, float("inf")))
    mi, md = engine._merge_branches_tensor(bi, bd, 10)
    X64, Q64 = X.astype(np.float64), Q.astype(np.float64)
    gt = np.argsort(-(Q64 @ X64.T), axis=1, kind="stable")[:, :10].astype(np.int32)
    np.savez_compressed(OUT / "refcpu_c1.npz",
                        X_sha=np.array(sha(X)), Q=Q, G=G.astype(np.int16),
                        catalogue=cat.astype(np.int16), seeds=seeds.astype(np.int16),
                        ids=ids.astype(np.int16), dist=dist, expanded=expd, counters=ctr,
                        merged_ids=mi.numpy().astype(np.int16), merged_dist=md.numpy(),
                        gt=gt.astype(np.int16))
    print("refcpu_c1.npz written; recall@10 of the reference C1 path:",
          float(np.mean([len(set(a) & set(b)) / 10 for a, b in zip(mi.numpy(), gt)])))


def main(which=("branch", "distance", "build", "extras", "c1", "deg96")):
    refcpu, build, select, engine, _ = ref_modules()
    if "deg96" in which:
        make_build_deg96(build)
    if "extras" in which:
        make_build_extras(build, ref_offline())
    if "distance" in which:
        make_distance(refcpu)
    if "branch" in which:
        make_branch(refcpu)
    if "build" in which:
        make_build_small(build)
    if "c1" in which:
        make_c1(refcpu, build, select, engine)


if __name__ == "__main__":
    main(tuple(sys.argv[1:]) or ("branch", "distance", "build", "c1"))
