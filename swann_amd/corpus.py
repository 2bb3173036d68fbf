"""The on-disk corpus layout the reference's offline tools share
(offline/prep_annbench.py:91-123, offline/prep_fvecs.py:77-116,
swann/_pools.py:12-24):

    manifest.json                 corpus, n, d, d_original, k, seed, metric, ...
    X.npy                         fp32 [n, d], d padded to a multiple of 8
    Q_val.npy, Q_test.npy         fp32 query splits (a seeded permutation)
    qidx_val.npy, qidx_test.npy   each split's rows in the original query set
    gt_{val,test}_ids.npy         exact top-k ids (int32)
    gt_{val,test}_sim.npy         their similarity: <q, x>, or -||q - x||
    G_knn.npy, G.npy              an exact kNN graph (the stand-in the builder replaces)
    pools/pool_<name>.npy         entry pools

Ground truth and the kNN stand-in come from this library's exact GPU
selection and sweep.
"""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import torch

from . import _select as S
from . import build as B


def _exact_topk(X: torch.Tensor, Q: torch.Tensor, k: int, metric: str, block: int = 1024):
    """Exact top-k of every query over the whole corpus: ids and similarity
    (<q, x> for ip, -||q - x|| for l2)."""
    m = 0 if metric == "ip" else 1
    ids = np.empty((Q.shape[0], k), np.int32)
    sim = np.empty((Q.shape[0], k), np.float32)
    ws = None
    for s in range(0, Q.shape[0], block):
        q = Q[s:s + block].contiguous()
        need = int(S._ws_size(q.shape[0], X.shape[0]))
        if ws is None or ws.numel() < need:
            ws = torch.empty(need, dtype=torch.uint8, device=X.device)
        idx = S.select_nearest(q, X, k, metric=m, workspace=ws)
        xs = X[idx]                                            # [b, k, d]
        if metric == "ip":
            v = (xs * q[:, None, :]).sum(-1)
        else:
            v = -((xs - q[:, None, :]) ** 2).sum(-1).clamp(min=0).sqrt()
        ids[s:s + q.shape[0]] = idx.cpu().numpy().astype(np.int32)
        sim[s:s + q.shape[0]] = v.cpu().numpy()
    return ids, sim


def write_corpus(out, X, Q, metric="ip", name=None, k=10, deg=64, seed=0, source="",
                 split=True, drop_degenerate=True):
    """Write a corpus in the shared layout.  ip corpora are L2-normalised
    (zero-length rows dropped unless `drop_degenerate` is False); both sides
    are zero-padded to a multiple of 8 dimensions."""
    out = Path(out)
    out.mkdir(parents=True, exist_ok=True)
    X = np.asarray(X, dtype=np.float32)
    Q = np.asarray(Q, dtype=np.float32)
    d0 = X.shape[1]
    pad = (-d0) % 8
    if pad:
        X = np.pad(X, ((0, 0), (0, pad)))
        Q = np.pad(Q, ((0, 0), (0, pad)))
    if metric == "ip":
        xn = np.linalg.norm(X, axis=1, keepdims=True)
        qn = np.linalg.norm(Q, axis=1, keepdims=True)
        if drop_degenerate:
            kx, kq = xn[:, 0] > 1e-12, qn[:, 0] > 1e-12
            X, xn, Q, qn = X[kx], xn[kx], Q[kq], qn[kq]
        X = X / np.maximum(xn, 1e-12)
        Q = Q / np.maximum(qn, 1e-12)
    X = np.ascontiguousarray(X, dtype=np.float32)
    Q = np.ascontiguousarray(Q, dtype=np.float32)
    Xg = torch.from_numpy(X).cuda()
    np.save(out / "X.npy", X)
    if split:
        perm = np.random.default_rng(seed).permutation(Q.shape[0])
        half = Q.shape[0] // 2
        splits = (("val", np.sort(perm[:half])), ("test", np.sort(perm[half:])))
    else:
        splits = (("test", np.arange(Q.shape[0])),)
    for tag, rows in splits:
        Qs = np.ascontiguousarray(Q[rows])
        np.save(out / f"Q_{tag}.npy", Qs)
        np.save(out / f"qidx_{tag}.npy", rows)
        ids, sim = _exact_topk(Xg, torch.from_numpy(Qs).cuda(), k, metric)
        np.save(out / f"gt_{tag}_ids.npy", ids)
        np.save(out / f"gt_{tag}_sim.npy", sim)
    G = B.knn_candidates(Xg, deg, metric=metric)[0].cpu().numpy().astype(np.int32)
    np.save(out / "G_knn.npy", G)
    np.save(out / "G.npy", G)
    (out / "manifest.json").write_text(json.dumps({
        "corpus": name or out.name, "n": int(X.shape[0]), "d": int(X.shape[1]),
        "d_original": int(d0), "deg": int(deg), "k": int(k), "seed": int(seed),
        "metric": "ip_on_l2_normalised" if metric == "ip" else "sqeuclidean",
        "graph": "exact_knn", "source": str(source),
    }, indent=2))
    return out


def load_corpus(data, split="test", mmap=True):
    """(manifest, X, Q, gt_ids, gt_sim) of a corpus directory; X is
    memory-mapped unless `mmap` is False."""
    d = Path(data)
    man = json.loads((d / "manifest.json").read_text())
    X = np.load(d / "X.npy", mmap_mode="r" if mmap else None)
    Q = np.load(d / f"Q_{split}.npy")
    ids = np.load(d / f"gt_{split}_ids.npy")
    sim = np.load(d / f"gt_{split}_sim.npy")
    return man, X, Q, ids, sim


def metric_of(manifest) -> str:
    return "ip" if manifest["metric"].startswith("ip") else "l2"


def write_pool(data, name, ids) -> Path:
    p = Path(data) / "pools" / f"pool_{name}.npy"
    p.parent.mkdir(parents=True, exist_ok=True)
    np.save(p, np.asarray(ids, dtype=np.int32))
    return p


def load_pool(data, name="random", P=512, seed=0):
    """A named entry pool, or an inline random one when none is written
    (swann/_pools.py:12-24)."""
    p = Path(data) / "pools" / f"pool_{name}.npy"
    if p.exists():
        pool = np.load(p).astype(np.int32)
        return pool[:P] if P and len(pool) != P else pool
    if name != "random":
        raise FileNotFoundError(f"no pool '{name}' under {p.parent}")
    n = np.load(Path(data) / "X.npy", mmap_mode="r").shape[0]
    return np.sort(np.random.default_rng(seed).choice(n, size=P, replace=False)).astype(np.int32)
