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
