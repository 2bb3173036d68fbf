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
