"""Shared helpers for the CPU and GPU tests (not a test module itself)."""
import numpy as np


def knn_graph(X, deg, metric=0):
    """Exact kNN graph in float64, self excluded (tests/test_engine.py:24-34)."""
    X64 = X.astype(np.float64)
    if metric == 0:
        sim = X64 @ X64.T
    else:
        sq = (X64 * X64).sum(1)
        sim = -(sq[:, None] - 2 * X64 @ X64.T + sq[None, :])
    np.fill_diagonal(sim, -np.inf)
    return np.ascontiguousarray(np.argsort(-sim, axis=1, kind="stable")[:, :deg].astype(np.int32))


def recall(got, truth, k):
    return float(np.mean([len(set(a[:k]) & set(b[:k])) / k for a, b in zip(got, truth)]))


def exact_topk(X, Q, k, metric=0):
    X64, Q64 = X.astype(np.float64), Q.astype(np.float64)
    if metric == 0:
        d = -(Q64 @ X64.T)
    else:
        d = (X64 * X64).sum(1)[None, :] - 2 * Q64 @ X64.T
    return np.argsort(d, axis=1, kind="stable")[:, :k].astype(np.int32)


def stall_case():
    """Node 0 is the query itself (L2 distance 0) and the only seed; its eight
    neighbours point only back into {0..8}.  With kstop = 1 the k-th distance
    is 0 from the first expansion on and never improves."""
    rng = np.random.default_rng(5)
    X = rng.standard_normal((40, 8)).astype(np.float32)
    q = X[0].copy()
    G = np.full((40, 8), -1, np.int32)
    G[0] = np.arange(1, 9)
    for u in range(1, 9):
        G[u] = [v for v in range(9) if v != u]
    for u in range(9, 40):
        G[u] = rng.integers(0, 40, 8)
    return X, G, q


def crowd_case():
    """Seed 0 has four neighbours 1..4, each of which points only back into
    {0..4}: after the first expansion every neighbour list is fully covered."""
    rng = np.random.default_rng(6)
    X = rng.standard_normal((20, 8)).astype(np.float32)
    q = rng.standard_normal(8).astype(np.float32)
    G = np.full((20, 8), -1, np.int32)
    G[0, :4] = [1, 2, 3, 4]
    for u in range(1, 5):
        G[u, :4] = [v for v in range(5) if v != u]
    return X, G, q


def tie_runs(d, atol=1e-6, rtol=1e-6):
    """Split an ascending distance row into maximal runs whose neighbours tie
    within atol + rtol*|d| (north_star's tie rule: 1e-6, relative above 1)."""
    runs, p = [], 0
    while p < len(d):
        q = p
        while q + 1 < len(d) and abs(float(d[q + 1]) - float(d[q])) <= atol + rtol * abs(float(d[q])):
            q += 1
        runs.append((p, q + 1))
        p = q + 1
    return runs


def untied_rows(got, want, want_d, got_d=None, atol=1e-6, rtol=1e-6):
    """Rows where two ascending lists differ by more than ties.

    Inside each run of tied reference distances the two rows must hold the
    same ids in any order.  The run that reaches the end of the row may hold
    different ids (which of several tied rows makes the cut), but only when
    `got_d` shows the replacements at the same distances.  Returns the row
    indices that break this; an empty list means equal up to named ties."""
    bad = []
    for r in np.nonzero((got != want).any(1))[0]:
        g, w, d = got[r], want[r], want_d[r]
        for p, q in tie_runs(d, atol, rtol):
            if np.array_equal(np.sort(g[p:q]), np.sort(w[p:q])):
                continue
            at_end = q == len(w)
            if at_end and got_d is not None and np.all(
                    np.abs(got_d[r, p:q].astype(np.float64) - d[p:q]) <= atol + rtol * np.abs(d[p:q])):
                continue
            bad.append(int(r))
            break
    return bad


def graph_dist(X, G, rows, metric=0):
    """Exact float64 distance from each listed node to each of its neighbours
    in G[rows] (+inf for -1 pads): the order key of a pruned row."""
    X64 = X.astype(np.float64)
    Gr = G[rows]
    V = X64[np.where(Gr >= 0, Gr, 0)]
    if metric == 0:
        d = 1.0 - np.einsum("nkd,nd->nk", V, X64[rows])
    else:
        d = ((V - X64[rows][:, None, :]) ** 2).sum(-1)
    return np.where(Gr >= 0, d, np.inf)


def untied_graph_rows(got, want, X, metric=0, atol=1e-6, rtol=1e-6):
    """Rows of two pruned graphs that differ by more than the order of
    neighbours at tied distances: the neighbour sets must be equal, and the
    orders may differ only inside runs of tied exact distances."""
    bad = [int(r) for r in np.nonzero((got != want).any(1))[0]
           if set(got[r].tolist()) != set(want[r].tolist())]
    rows = np.array(sorted(set(np.nonzero((got != want).any(1))[0].tolist()) - set(bad)), np.int64)
    if len(rows):
        d = graph_dist(X, want, rows, metric)
        bad += [int(rows[i]) for i in untied_rows(got[rows], want[rows], d, None, atol, rtol)]
    return sorted(bad)
