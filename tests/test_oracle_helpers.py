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
    within atol + rtol*|d| (north_star's tie rule: 1e-6, relative above 1).
    `atol` may be a scalar or one value per position."""
    at = np.broadcast_to(np.asarray(atol, np.float64), np.shape(d))
    runs, p = [], 0
    while p < len(d):
        q = p
        while q + 1 < len(d) and abs(float(d[q + 1]) - float(d[q])) <= \
                at[q] + rtol * abs(float(d[q])):
            q += 1
        runs.append((p, q + 1))
        p = q + 1
    return runs


def untied_rows(got, want, want_d, got_d=None, atol=1e-6, rtol=1e-6):
    """Rows where two ascending lists differ by more than ties.

    Inside each run of tied reference distances the two rows must hold the
    same ids in any order.  The run that reaches the end of the row may hold
    different ids (which of several tied rows makes the cut), but only when
    `got_d` shows the replacements at the same distances.  `atol` is a
    scalar or an array shaped like the rows.  Returns the row indices that
    break this; an empty list means equal up to ties."""
    bad = []
    at_all = np.broadcast_to(np.asarray(atol, np.float64), np.shape(want))
    for r in np.nonzero((got != want).any(1))[0]:
        g, w, d, at = got[r], want[r], want_d[r], at_all[r]
        for p, q in tie_runs(d, at, rtol):
            if np.array_equal(np.sort(g[p:q]), np.sort(w[p:q])):
                continue
            at_end = q == len(w)
            if at_end and got_d is not None and np.all(
                    np.abs(got_d[r, p:q].astype(np.float64) - d[p:q])
                    <= at[p:q] + rtol * np.abs(d[p:q])):
                continue
            bad.append(int(r))
            break
    return bad


def describe_rows(rows, got, want, want_d, got_d=None, limit=3):
    """A short text of the first differing rows, for a failing assertion."""
    out = []
    for r in rows[:limit]:
        diff = np.nonzero(got[r] != want[r])[0]
        out.append(f"row {r} cols {diff[:6].tolist()} got {got[r][diff[:6]].tolist()} "
                   f"want {want[r][diff[:6]].tolist()} want_d {np.asarray(want_d[r])[diff[:6]].tolist()}"
                   + ("" if got_d is None else f" got_d {np.asarray(got_d[r])[diff[:6]].tolist()}"))
    return "; ".join(out)


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


def prune_margins(X, cand, cdist, rows, deg, alpha=1.2, metric=0, deg_per_node=None,
                  protect=None):
    """For each listed node, the smallest relative margin of any detour test
    that robust_prune's rule (build.py:46-91) decides on its way down the
    candidate list, replayed in float64 on the same inputs:
    |alpha d(w, i) - d(u, i)| / (|alpha d(w, i)| + |d(u, i)|) over the kept w
    of every candidate i that is tested.  Two correct implementations whose
    pair distances round differently can disagree on a row only through a
    test whose margin is below their rounding error, so a differing row with
    a large margin is a real difference."""
    X64 = X.astype(np.float64)
    out = []
    for u in rows:
        c, du = cand[u], cdist[u].astype(np.float64)
        cap = deg if deg_per_node is None else min(deg, int(deg_per_node[u]))
        V = X64[np.where(c >= 0, c, 0)]
        if metric == 0:
            pair = 1.0 - V @ V.T
        else:
            vn = (V * V).sum(1)
            pair = np.maximum(vn[:, None] - 2.0 * V @ V.T + vn[None, :], 0.0)
        kept, margin = [], np.inf
        for i in range(len(c)):
            if len(kept) >= cap:
                break
            if c[i] < 0:
                continue
            if protect is not None and protect[u, i]:
                kept.append(i)
                continue
            a = alpha * pair[kept, i]
            if len(kept):
                margin = min(margin, float(np.min(np.abs(a - du[i]) / (np.abs(a) + abs(du[i]) + 1e-30))))
            if not (a <= du[i]).any():
                kept.append(i)
        out.append(margin)
    return np.array(out)


def untied_prune_rows(got, want, X, cand, cdist, deg, alpha=1.2, metric=0, deg_per_node=None,
                      protect=None, tol=2e-5):
    """Rows of two prunes of the same candidate lists that differ although no
    detour test on the row lies within `tol` (relative) of its threshold."""
    rows = np.nonzero((got != want).any(1))[0]
    if not len(rows):
        return []
    m = prune_margins(X, cand, cdist, rows, deg, alpha, metric, deg_per_node, protect)
    return [int(r) for r, v in zip(rows, m) if v > tol]
