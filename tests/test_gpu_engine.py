"""The engine on the GPU against the oracle and the reference's golden vectors
(tests/test_engine.py of the reference, plus fp16, team 64, both workgroup
layouts and config C1).  Every call goes through the C ABI (ctypes).

Bar: bit-exact queues (ids, distance bits, expanded flags, lineage) and
counters wherever the search is deterministic (no claims, no bound).
"""
import os
import sys

import numpy as np
import pytest
import torch

import oracle as O
from conftest import gaussian, golden, regen
from test_oracle_helpers import crowd_case, exact_topk, knn_graph, recall, stall_case

pytestmark = pytest.mark.gpu

E = pytest.importorskip("swann_amd._engine")
DEV = "cuda"


def note(*a):
    print("[case]", *a, flush=True)
    sys.stdout.flush()


def to_gpu(*arrs):
    return [torch.from_numpy(np.ascontiguousarray(a)).to(DEV) for a in arrs]


def toy(n=2000, d=64, deg=32, seed=0, metric=0):
    X = gaussian(n, d, seed, metric == 0)
    return X, knn_graph(X, deg, metric)


@pytest.fixture(params=["64", "256", "1024"], autouse=False)
def block(request, opt):
    opt(search_block=int(request.param))
    return int(request.param)


def assert_queue(st, qi, j, br, what):
    gi = st.ids[qi, j].cpu().numpy(); gd = st.dist[qi, j].cpu().numpy()
    ge = st.expanded[qi, j].cpu().numpy(); gl = st.lineage[qi, j].cpu().numpy()
    gc = st.counters[qi, j].cpu().numpy()
    assert np.array_equal(gi, br.ids), f"ids differ {what}"
    assert gd.tobytes() == br.dist.tobytes(), f"distances differ {what}"
    assert np.array_equal(ge, br.expanded), f"expanded differs {what}"
    assert np.array_equal(gl, br.lineage), f"lineage differs {what}"
    for c in (0, 1, 2, 3, 6, 7, 8, 9):
        assert gc[c] == br.counters[c], f"counter {c} differs {what}: {gc[c]} vs {br.counters[c]}"


@pytest.mark.parametrize("metric", [0, 1])
@pytest.mark.parametrize("dtype", ["f32", "f16"])
def test_cpu_gpu_exact(metric, dtype, block):
    """Same queue, same distance bits, every team size (test_engine.py:42-78)."""
    X, G = toy(metric=metric)
    if dtype == "f16":
        X = X.astype(np.float16)
    rng = np.random.default_rng(7)
    nq, J, L, budget = 5, 3, 16, 12
    Qv = gaussian(nq, X.shape[1], 77, metric == 0)
    seeds = rng.integers(0, X.shape[0], size=(nq, J)).astype(np.int32)
    Xg, Gg, Qg = to_gpu(X, G, Qv)
    for team in (4, 8, 16, 32, 64):
        note("cpu_gpu_exact", metric, dtype, block, team)
        st = E.init_states(Xg, Qg, torch.from_numpy(seeds), L=L, B=budget, D=G.shape[1],
                           metric=metric, team_size=team)
        E.advance(Xg, Gg, Qg, st, budget)
        st.check()
        for qi in range(nq):
            for j in range(J):
                br = O.run(X, G, Qv[qi], int(seeds[qi, j]), L=L, B=budget, metric=metric, team=team)
                assert_queue(st, qi, j, br, (metric, dtype, team, qi, j))


@pytest.mark.parametrize("tag,metric", [("ip", 0), ("l2", 1)])
def test_matches_reference_golden(tag, metric):
    """The reference's own _refcpu trajectories (tests/golden/refcpu_branch.npz)."""
    g = golden("refcpu_branch.npz")
    X = regen(2000, 64, 0, metric == 0, g[f"{tag}_X_sha"])
    G = g[f"{tag}_G"].astype(np.int32); Q = g[f"{tag}_Q"]; seeds = g[f"{tag}_seeds"]
    Xg, Gg, Qg = to_gpu(X, G, Q)
    for team in (4, 8, 16, 32):
        note("golden", tag, team)
        st = E.init_states(Xg, Qg, torch.from_numpy(seeds), L=16, B=12, D=32, metric=metric,
                           team_size=team)
        E.advance(Xg, Gg, Qg, st, 12)
        gi = st.ids.cpu().numpy(); gd = st.dist.cpu().numpy(); gc = st.counters.cpu().numpy()
        want_i = g[f"{tag}_t{team}_ids"]; want_d = g[f"{tag}_t{team}_dist"]
        want_c = g[f"{tag}_t{team}_counters"]
        for qi in range(Q.shape[0]):
            for j in range(seeds.shape[1]):
                n = int((want_i[qi, j] >= 0).sum())
                assert list(gi[qi, j, :n]) == list(want_i[qi, j, :n])
                assert gd[qi, j, :n].tobytes() == want_d[qi, j, :n].tobytes()
                assert gc[qi, j, 0] == want_c[qi, j, 0] and gc[qi, j, 1] == want_c[qi, j, 1]


def test_resume_equivalence(block):
    X, G = toy(seed=3)
    rng = np.random.default_rng(11)
    nq, J, L, budget = 8, 4, 32, 24
    Qv = gaussian(nq, 64, 33, True)
    seeds = torch.from_numpy(rng.integers(0, X.shape[0], (nq, J)).astype(np.int32))
    Xg, Gg, Qg = to_gpu(X, G, Qv)
    kw = dict(L=L, B=budget, D=G.shape[1], team_size=32)
    one = E.init_states(Xg, Qg, seeds, **kw)
    E.advance(Xg, Gg, Qg, one, budget)
    for split in (1, 2, 7, budget - 1):
        note("resume", block, split)
        two = E.init_states(Xg, Qg, seeds, **kw)
        E.advance(Xg, Gg, Qg, two, split)
        E.advance(Xg, Gg, Qg, two, budget - split)
        for f in ("ids", "dist", "expanded", "lineage", "counters"):
            assert torch.equal(getattr(one, f), getattr(two, f)), (split, f)
        # the visited table holds the same set (slot positions may differ)
        a = torch.sort(one.visited.reshape(nq * J, -1), dim=1).values
        b = torch.sort(two.visited.reshape(nq * J, -1), dim=1).values
        assert torch.equal(a, b)


def test_budget_is_a_state_property():
    X, G = toy(seed=5)
    rng = np.random.default_rng(13)
    Qv = gaussian(4, 64, 55, True)
    seeds = torch.from_numpy(rng.integers(0, X.shape[0], (4, 2)).astype(np.int32))
    Xg, Gg, Qg = to_gpu(X, G, Qv)
    st = E.init_states(Xg, Qg, seeds, L=16, B=10, D=G.shape[1])
    E.advance(Xg, Gg, Qg, st, 100)
    assert int(st.expansions.max()) == 10


def test_brute_force_on_complete_graph():
    n, d, L = 96, 48, 16
    X = gaussian(n, d, 17, True)
    G = np.stack([np.delete(np.arange(n), i) for i in range(n)]).astype(np.int32)[:, :95]
    Qv = gaussian(6, d, 18, True)
    Xg, Gg, Qg = to_gpu(X, G, Qv)
    seeds = torch.zeros((6, 1), dtype=torch.int32)
    ids, dist, st = E.search(Xg, Gg, Qg, seeds, k=10, L=L, B=1)
    exact = 1.0 - (Qv.astype(np.float64) @ X.astype(np.float64).T)
    want = np.argsort(exact, axis=1, kind="stable")[:, :10]
    assert (ids.cpu().numpy() == want).all()
    assert np.allclose(dist.cpu().numpy(), np.take_along_axis(exact, want, 1), atol=2e-6)


def test_dead_branch_and_exhaustion():
    n, d = 64, 16
    X = gaussian(n, d, 19, True)
    G = np.full((n, 8), -1, dtype=np.int32)
    Qv = gaussian(2, d, 20, True)
    Xg, Gg, Qg = to_gpu(X, G, Qv)
    seeds = torch.tensor([[0, -1], [5, -1]], dtype=torch.int32)
    st = E.init_states(Xg, Qg, seeds, L=16, B=16, D=8)
    E.advance(Xg, Gg, Qg, st, 16)
    st.check()
    assert int(st.expansions[0, 0]) == 1 and int(st.exhausted[0, 0]) == 1
    assert int(st.expansions[0, 1]) == 0 and int(st.exhausted[0, 1]) == 1
    assert int(st.ids[0, 1, 0]) == -1
    ids, _ = E.branch_topk(st, 10)
    assert int((ids >= 0).sum()) == 2


def test_out_of_range_ids_are_empty():
    """Seeds and edges >= n are treated as empty, never read."""
    n, d = 64, 16
    X = gaussian(n, d, 21, True)
    G = np.full((n, 8), 10 ** 6, dtype=np.int32)
    Qv = gaussian(2, d, 22, True)
    Xg, Gg, Qg = to_gpu(X, G, Qv)
    seeds = torch.tensor([[3, 10 ** 7], [n, 7]], dtype=torch.int32)
    st = E.init_states(Xg, Qg, seeds, L=8, B=4, D=8)
    E.advance(Xg, Gg, Qg, st, 4)
    assert int(st.ids[0, 1, 0]) == -1 and int(st.ids[1, 0, 0]) == -1
    assert int(st.expansions[0, 0]) == 1 and int(st.dist_evals.sum()) == 2


def test_visited_overflow_is_reported():
    X, G = toy(n=1000, seed=23)
    Qv = gaussian(2, 64, 29, True)
    Xg, Gg, Qg = to_gpu(X, G, Qv)
    st = E.init_states(Xg, Qg, torch.zeros((2, 1), dtype=torch.int32), L=16, B=16, D=G.shape[1])
    st.visited = torch.zeros((2, 1, 64), dtype=torch.int32, device=DEV)
    st.counters.zero_()
    E.advance(Xg, Gg, Qg, st, 16)
    assert int(st.hash_failures.sum()) > 0
    assert int(st.overflow()) == int(st.hash_failures.sum())
    with pytest.raises(RuntimeError):
        st.check()


def test_merge_dedup_matches_oracle():
    """Every kernel shape (one wave with 1..32 keys a lane, n up to 2048; the
    1024-thread walk above that), C4's 128 branches x 10, k up to n, against
    the oracle's sort-and-scan restatement of local_search.cu:863-919, bit
    for bit."""
    rng = np.random.default_rng(37)
    for Q, V, kk, k in ((6, 5, 10, 10), (50, 32, 10, 10), (9, 128, 12, 10), (3, 7, 3, 5),
                        (4, 1, 1, 1), (5, 2, 40, 80), (7, 64, 10, 10), (11, 128, 10, 10),
                        (3, 128, 16, 10), (2, 256, 10, 100), (2, 1000, 10, 10000),
                        (300, 64, 10, 10)):
        note("merge", Q, V, kk, k)
        pool = max(8, V * kk // 3)
        ids = rng.integers(-1, pool, (Q, V, kk)).astype(np.int32)
        base = rng.random(pool).astype(np.float32)
        dist = np.where(ids >= 0, base[np.clip(ids, 0, None)], np.float32(3e38)).astype(np.float32)
        gi, gd = E.merge_branches(*to_gpu(ids, dist), k)
        wi, wd = O.merge(ids, dist, k)
        assert np.array_equal(gi.cpu().numpy(), wi), (Q, V, kk, k)
        assert gd.cpu().numpy().tobytes() == wd.tobytes(), (Q, V, kk, k)


def test_merge_reads_queues_in_place():
    """merge_state reads the first min(k, L) slots of each branch's L-slot
    queue where they lie; against the oracle's merge of the [Q, V, kk] copy
    that branch_topk would make, bit for bit.  Slot counts that do and do not
    divide a wave (64) or a workgroup (1024), both kernel shapes, k above L."""
    from types import SimpleNamespace
    rng = np.random.default_rng(41)
    for Q, V, L, k in ((5, 6, 16, 10), (7, 40, 44, 10), (3, 9, 13, 7), (4, 3, 5, 12),
                       (2, 300, 44, 10), (3, 128, 24, 100), (2, 1, 1, 1), (6, 64, 12, 10)):
        kk = min(k, L)
        note("merge in place", Q, V, L, k)
        pool = max(8, V * kk // 3)
        ids = rng.integers(-1, pool, (Q, V, L)).astype(np.int32)
        base = rng.random(pool).astype(np.float32)
        dist = np.where(ids >= 0, base[np.clip(ids, 0, None)], np.float32(3e38)).astype(np.float32)
        gi, gd = to_gpu(ids, dist)
        oi, od = E.merge_state(SimpleNamespace(ids=gi, dist=gd), k)
        wi, wd = O.merge(np.ascontiguousarray(ids[..., :kk]),
                         np.ascontiguousarray(dist[..., :kk]), k)
        assert np.array_equal(oi.cpu().numpy(), wi), (Q, V, L, k)
        assert od.cpu().numpy().tobytes() == wd.tobytes(), (Q, V, L, k)
    with pytest.raises(RuntimeError):
        E.merge_state(SimpleNamespace(ids=gi, dist=gd), V * L + 1)


def test_merge_keeps_the_reference_quirks():
    """Hand cases of the (distance, id) walk with the predecessor rule of
    local_search.cu:903-910: an id seen again at a larger distance is dropped
    only when nothing lies between the two copies; equal distances go by id;
    a valid id at +inf comes before the invalid ones; -0 keeps its sign; too
    few distinct ids pad with (-1, +inf)."""
    inf = np.float32(np.inf)
    cases = [
        ([7, 3, 7], [0.5, 0.55, 0.6], 3),          # 7 3 7: not adjacent, both kept
        ([7, 7, 3], [0.5, 0.6, 0.7], 3),           # 7 3: the copies are adjacent
        ([9, 4, 4, 2], [0.25, 0.25, 0.25, 0.25], 4),   # ties by id: 2 4 9
        ([5, -1, 6, -1], [inf, 0.1, 0.2, 0.3], 4),     # 6, then 5 at +inf, then padding
        ([1, 2, 3], [-0.0, 0.0, -1.0], 3),         # -1, then -0 (id 1) before +0 (id 2)
        ([-1, -1, -1], [0.1, 0.2, 0.3], 2),        # nothing valid
    ]
    for ids_l, d_l, k in cases:
        ids = np.array(ids_l, np.int32).reshape(1, 1, -1)
        dist = np.array(d_l, np.float32).reshape(1, 1, -1)
        gi, gd = E.merge_branches(*to_gpu(ids, dist), k)
        wi, wd = O.merge(ids, dist, k)
        assert np.array_equal(gi.cpu().numpy(), wi), ids_l
        assert gd.cpu().numpy().tobytes() == wd.tobytes(), ids_l
    gi, _ = E.merge_branches(*to_gpu(np.array([[[7, 3, 7]]], np.int32),
                                     np.array([[[0.5, 0.55, 0.6]]], np.float32)), 3)
    assert gi.cpu().numpy().tolist() == [[7, 3, 7]]


def test_shared_cache_is_free_of_consequence(block):
    X, G = toy(seed=79)
    rng = np.random.default_rng(83)
    nq, Ebr, L, budget = 16, 24, 32, 12
    Qv = gaussian(nq, 64, 84, True)
    seeds = torch.from_numpy(rng.integers(0, X.shape[0], (nq, Ebr)).astype(np.int32))
    Xg, Gg, Qg = to_gpu(X, G, Qv)
    plain = E.search(Xg, Gg, Qg, seeds, k=10, L=L, B=budget)
    cached = E.search(Xg, Gg, Qg, seeds, k=10, L=L, B=budget, shared_cache=True)
    assert torch.equal(plain[0], cached[0]) and torch.equal(plain[1], cached[1])
    assert torch.equal(plain[2].ids, cached[2].ids)
    assert torch.equal(plain[2].expansions, cached[2].expansions)
    a = plain[2].dist_evals.sum(); b = cached[2].dist_evals.sum()
    hits = cached[2].cache_hits.sum()
    assert int(b) < int(a) and int(a - b) == int(hits)


def test_determinism():
    X, G = toy(seed=41)
    rng = np.random.default_rng(43)
    Qv = gaussian(16, 64, 44, True)
    seeds = torch.from_numpy(rng.integers(0, X.shape[0], (16, 8)).astype(np.int32))
    Xg, Gg, Qg = to_gpu(X, G, Qv)
    ref = None
    for _ in range(5):
        ids, dist, st = E.search(Xg, Gg, Qg, seeds, k=10, L=16, B=16)
        now = (ids.cpu().numpy(), dist.cpu().numpy(), st.counters.cpu().numpy())
        if ref is None:
            ref = now
        for a, b in zip(ref, now):
            assert (a == b).all()


@pytest.mark.parametrize("policy", [0, 1])
def test_multiseed_matches_oracle(policy, block):
    X, G = toy(seed=53)
    rng = np.random.default_rng(59)
    nq, V, L, budget = 4, 6, 32, 20
    Qv = gaussian(nq, 64, 60, True)
    seeds = rng.integers(0, X.shape[0], (nq, 1, V)).astype(np.int32)
    seeds[0, 0, 3] = seeds[0, 0, 1]                 # a repeated seed
    Xg, Gg, Qg = to_gpu(X, G, Qv)
    st = E.init_states(Xg, Qg, torch.from_numpy(seeds), L=L, B=budget, D=G.shape[1], policy=policy)
    E.advance(Xg, Gg, Qg, st, budget)
    for q in range(nq):
        br = O.init_branch(X, Qv[q], list(seeds[q, 0]), L=L, B=budget, D=32)
        O.advance_branch(X, G, Qv[q], br, budget, budget, policy=policy)
        assert_queue(st, q, 0, br, (policy, q))


def test_early_stop_matches_oracle(block):
    X, G = toy(seed=71)
    rng = np.random.default_rng(73)
    nq, V, L, budget, k = 4, 4, 32, 64, 10
    Qv = gaussian(nq, 64, 74, True)
    seeds = rng.integers(0, X.shape[0], (nq, 1, V)).astype(np.int32)
    Xg, Gg, Qg = to_gpu(X, G, Qv)
    for eps in (0.0, 0.1, 0.25):
        st = E.init_states(Xg, Qg, torch.from_numpy(seeds), L=L, B=budget, D=G.shape[1],
                           policy=E.POLICY_ROUND_ROBIN, stop_eps=eps, kstop=k)
        E.advance(Xg, Gg, Qg, st, budget)
        for q in range(nq):
            br = O.init_branch(X, Qv[q], list(seeds[q, 0]), L=L, B=budget, D=32)
            O.advance_branch(X, G, Qv[q], br, budget, budget, policy=1, stop_eps=eps, kstop=k)
            assert_queue(st, q, 0, br, (eps, q))
        assert int(st.expansions.max()) < budget


def test_stall_and_crowd_match_oracle():
    X, G = toy(seed=91)
    rng = np.random.default_rng(93)
    nq, V, L, budget = 6, 4, 24, 40
    Qv = gaussian(nq, 64, 94, True)
    seeds = rng.integers(0, X.shape[0], (nq, 1, V)).astype(np.int32)
    Xg, Gg, Qg = to_gpu(X, G, Qv)
    st = E.init_states(Xg, Qg, torch.from_numpy(seeds), L=L, B=budget, D=G.shape[1],
                       policy=1, stall_patience=3, crowd_frac=0.5)
    E.advance(Xg, Gg, Qg, st, budget)
    for q in range(nq):
        br = O.init_branch(X, Qv[q], list(seeds[q, 0]), L=L, B=budget, D=32)
        O.advance_branch(X, G, Qv[q], br, budget, budget, policy=1, stall_patience=3,
                         crowd_frac=0.5)
        assert_queue(st, q, 0, br, q)


@pytest.mark.parametrize("patience", [1, 4])
def test_stall_hand_case(patience, block):
    """The stall rule's hand case on the GPU: exactly patience + 1 expansions,
    counter 6 set, and the queue equal to the oracle's."""
    X, G, q = stall_case()
    Xg, Gg, Qg = to_gpu(X, G, q[None, :])
    st = E.init_states(Xg, Qg, torch.tensor([[0]], dtype=torch.int32), L=16, B=64, D=8,
                       metric=1, team_size=4, stop_eps=-1.0, kstop=1, stall_patience=patience)
    E.advance(Xg, Gg, Qg, st, 64)
    br = O.init_branch(X, q, [0], L=16, B=64, D=8, metric=O.METRIC_L2, team=4)
    O.advance_branch(X, G, q, br, 64, 64, metric=O.METRIC_L2, team=4, stop_eps=-1.0, kstop=1,
                     stall_patience=patience)
    assert int(st.counters[0, 0, 0]) == patience + 1 and int(st.counters[0, 0, 6]) == 1
    assert_queue(st, 0, 0, br, ("stall", patience))


def test_crowd_hand_case(block):
    """The crowd rule's hand case on the GPU: the seed's lineage is retired
    after the third expansion (counter 7) and the branch then finds no slot
    (counter 3); the queue equals the oracle's."""
    X, G, q = crowd_case()
    Xg, Gg, Qg = to_gpu(X, G, q[None, :])
    st = E.init_states(Xg, Qg, torch.tensor([[0]], dtype=torch.int32), L=16, B=64, D=8,
                       metric=1, team_size=4, stop_eps=-1.0, kstop=10, crowd_frac=1.0)
    E.advance(Xg, Gg, Qg, st, 64)
    br = O.init_branch(X, q, [0], L=16, B=64, D=8, metric=O.METRIC_L2, team=4)
    O.advance_branch(X, G, q, br, 64, 64, metric=O.METRIC_L2, team=4, stop_eps=-1.0, kstop=10,
                     crowd_frac=1.0)
    c = st.counters[0, 0].cpu().numpy()
    assert c[0] == 3 and c[7] == 1 and c[3] == 1
    assert_queue(st, 0, 0, br, "crowd")


def test_shared_state_beats_split_branches_on_work():
    X, G = toy(seed=61)
    rng = np.random.default_rng(67)
    nq, V, budget, L = 32, 8, 64, 64
    Qv = gaussian(nq, 64, 68, True)
    seeds = rng.integers(0, X.shape[0], (nq, V)).astype(np.int32)
    Xg, Gg, Qg = to_gpu(X, G, Qv)
    split = E.init_states(Xg, Qg, torch.from_numpy(seeds), L=L, B=budget // V, D=G.shape[1])
    E.advance(Xg, Gg, Qg, split, budget // V)
    shared = E.init_states(Xg, Qg, torch.from_numpy(seeds).unsqueeze(1), L=L, B=budget,
                           D=G.shape[1], policy=E.POLICY_ROUND_ROBIN)
    E.advance(Xg, Gg, Qg, shared, budget)
    a = (split.dist_evals.sum(1).float() / split.expansions.sum(1).clamp(min=1).float()).mean()
    b = (shared.dist_evals[:, 0].float() / shared.expansions[:, 0].clamp(min=1).float()).mean()
    assert float(b) < float(a)


def test_chunked_advance_equals_one_shot():
    X, G = toy(seed=97)
    rng = np.random.default_rng(98)
    nq, J = 20, 6
    Qv = gaussian(nq, 64, 99, True)
    seeds = torch.from_numpy(rng.integers(0, X.shape[0], (nq, J)).astype(np.int32))
    Xg, Gg, Qg = to_gpu(X, G, Qv)
    a = E.search(Xg, Gg, Qg, seeds, k=10, L=16, B=20, stop_eps=0.1)
    b = E.search(Xg, Gg, Qg, seeds, k=10, L=16, B=20, stop_eps=0.1, chunk=3)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
    assert torch.equal(a[2].ids, b[2].ids)


def test_c1_matches_reference_path():
    """Config C1 as the reference's CPU path ran it: 200 queries x 8
    independent branches (claims off), L=12 B=64 eps=0.05 team=16, merged
    top-10 -- ids and distance bits identical."""
    g = golden("refcpu_c1.npz")
    X = regen(10000, 128, 0, True, g["X_sha"])
    G = g["G"].astype(np.int32); Q = g["Q"]; seeds = g["seeds"].astype(np.int32)
    Xg, Gg, Qg = to_gpu(X, G, Q)
    ids, dist, st = E.search(Xg, Gg, Qg, torch.from_numpy(seeds), k=10, L=12, B=64,
                             metric=0, team_size=16, stop_eps=0.05)
    assert np.array_equal(ids.cpu().numpy(), g["merged_ids"].astype(np.int32))
    assert dist.cpu().numpy().tobytes() == g["merged_dist"].astype(np.float32).tobytes()
    assert np.array_equal(st.ids.cpu().numpy(), g["ids"].astype(np.int32))
    assert np.array_equal(st.counters[..., :2].cpu().numpy(), g["counters"][..., :2])


def test_large_batch_one_wave_layout_matches_oracle():
    """Q*J >= 4096 takes the one-wave layout by default; compare a sample."""
    X, G = toy(seed=101)
    rng = np.random.default_rng(102)
    nq, J = 600, 8
    Qv = gaussian(nq, 64, 103, True)
    seeds = rng.integers(0, X.shape[0], (nq, J)).astype(np.int32)
    Xg, Gg, Qg = to_gpu(X, G, Qv)
    from swann_amd import _lib
    assert _lib.get_option("search_block") == 0          # chosen per batch
    st = E.init_states(Xg, Qg, torch.from_numpy(seeds), L=12, B=30, D=32, team_size=16,
                       stop_eps=0.05)
    E.advance(Xg, Gg, Qg, st, 30)
    for qi in range(0, nq, 37):
        for j in range(0, J, 3):
            br = O.run(X, G, Qv[qi], int(seeds[qi, j]), L=12, B=30, team=16, stop_eps=0.05)
            assert_queue(st, qi, j, br, (qi, j))


@pytest.mark.parametrize("bits", [False, True])
def test_claims_and_bound_multi_branch_statistics(bits):
    """Claims, bound and the elided visited table are racy by design: judge
    them by recall within 0.005 of the oracle's rounds schedule (every branch
    of a query starts together, as on the GPU), by distances that equal exact
    recomputation, and by no duplicate ids in the answer.  Claim bits are
    judged against the oracle's table at a size no probe chain fills."""
    g = golden("refcpu_c1.npz")
    X = regen(10000, 128, 0, True, g["X_sha"])
    G = g["G"].astype(np.int32)
    Q = gaussian(2000, 128, 501, True)
    cat = g["catalogue"].astype(np.int64)
    idx, _ = O.select_nearest(Q, X[cat], 16, 0, nthreads=8)
    seeds = cat[idx].astype(np.int32)
    Xg, Gg, Qg = to_gpu(X, G, Q)
    ids, dist, st = E.search(Xg, Gg, Qg, torch.from_numpy(seeds), k=10, L=12, B=64, metric=0,
                             team_size=16, stop_eps=0.05, shared_cache=True, shared_bound=True,
                             exclusive=True, elide_visited=True, claim_bits=bits)
    ids = ids.cpu().numpy(); dist = dist.cpu().numpy()
    Hc = 16 * E.next_pow2(X.shape[0]) if bits else E.cache_size(16, 64, 32)
    oi, od = O.search_batch(X, G, Q, seeds, k=10, L=12, B=64, metric=0, team=16, stop_eps=0.05,
                            H=1, Hc=Hc, bound=True, exclusive=True, nthreads=8,
                            schedule="rounds")
    truth = exact_topk(X, Q, 10)
    r_gpu, r_cpu = recall(ids, truth, 10), recall(oi, truth, 10)
    note("claims recall gpu", r_gpu, "oracle rounds", r_cpu, "bits", bits)
    assert abs(r_gpu - r_cpu) <= 0.005
    for q in range(Q.shape[0]):
        got = ids[q][ids[q] >= 0]
        assert len(set(got.tolist())) == len(got)
        for i, dv in zip(ids[q], dist[q]):
            if i >= 0:
                assert dv == O.team_distance(Q[q], X, int(i), 0, 16)


def test_code_filter_matches_oracle(block):
    """The sign-code pre-filter (local_search.cu:205-243, :560-575) against the
    oracle: independent branches, several teams and margins, bit-exact queues
    and counters -- counter 3 carries the skips, as in the reference."""
    X, G = toy(seed=5)
    codes, alpha, mu = O.build_codes(X)
    rng = np.random.default_rng(17)
    nq, J, L, budget = 6, 3, 16, 24
    Qv = gaussian(nq, X.shape[1], 55, True)
    seeds = rng.integers(0, X.shape[0], (nq, J)).astype(np.int32)
    Xg, Gg, Qg, Cg, Ag, Mg = to_gpu(X, G, Qv, codes, alpha, mu)
    skipped = 0
    for team in (4, 16, 64):
        for margin in (0.0, 0.05, 0.2):
            note("code filter", block, team, margin)
            st = E.init_states(Xg, Qg, torch.from_numpy(seeds), L=L, B=budget, D=G.shape[1],
                               team_size=team, stop_eps=0.1, kstop=10)
            E.advance(Xg, Gg, Qg, st, budget, codes=(Cg, Ag, Mg, margin))
            for qi in range(nq):
                for j in range(J):
                    br = O.init_branch(X, Qv[qi], [int(seeds[qi, j])], L=L, B=budget,
                                       D=G.shape[1], team=team)
                    O.advance_branch(X, G, Qv[qi], br, budget, budget, team=team, stop_eps=0.1,
                                     kstop=10, codes=(codes, alpha, mu, margin))
                    assert_queue(st, qi, j, br, ("codes", team, margin, qi, j))
            skipped += int(st.counters[..., 3].sum())
    assert skipped > 0                      # the filter did act


@pytest.mark.parametrize("spike", [0.0, 3.0, 40.0])
def test_code_filter_bracket_and_exact_fallback_match_oracle(spike):
    """The kernel decides most code estimates from a bracket of the exact
    sum (a 12-bit quantised query) and takes the exact reference-order sum
    only where the bracket straddles the line.  A query with one large
    component (x spike) quantises the rest coarsely, so the bracket is wide
    and most decisions fall back to the exact sum; without one almost none
    do.  Every decision must be the reference's: queues and counters
    bit-exact against the oracle, for teams 4, 16, 64 and several margins."""
    X, G = toy(seed=7)
    codes, alpha, mu = O.build_codes(X)
    rng = np.random.default_rng(29)
    nq, J, L, budget = 6, 3, 16, 24
    Qv = gaussian(nq, X.shape[1], 57, True)
    if spike:
        Qv[:, 3] += spike
        Qv = np.ascontiguousarray(Qv, dtype=np.float32)
    seeds = rng.integers(0, X.shape[0], (nq, J)).astype(np.int32)
    Xg, Gg, Qg, Cg, Ag, Mg = to_gpu(X, G, Qv, codes, alpha, mu)
    skipped = 0
    for team in (4, 16, 64):
        for margin in (0.0, 0.02, 0.1):
            note("code bracket", spike, team, margin)
            st = E.init_states(Xg, Qg, torch.from_numpy(seeds), L=L, B=budget, D=G.shape[1],
                               team_size=team, stop_eps=0.1, kstop=10)
            E.advance(Xg, Gg, Qg, st, budget, codes=(Cg, Ag, Mg, margin))
            for qi in range(nq):
                for j in range(J):
                    br = O.init_branch(X, Qv[qi], [int(seeds[qi, j])], L=L, B=budget,
                                       D=G.shape[1], team=team)
                    O.advance_branch(X, G, Qv[qi], br, budget, budget, team=team, stop_eps=0.1,
                                     kstop=10, codes=(codes, alpha, mu, margin))
                    assert_queue(st, qi, j, br, ("bracket", spike, team, margin, qi, j))
            skipped += int(st.counters[..., 3].sum())
    assert skipped > 0


@pytest.mark.parametrize("d", [200, 96, 1024])
def test_code_filter_word_layouts_match_oracle(d):
    """The estimate's word handling: 200 dimensions end inside a word (the
    straddling word walks its set bits below d), 96 gives fewer words than a
    64-lane team has lanes, 1024 gives several four-word chunks per lane.
    Queues and counters bit-exact against the oracle."""
    X = gaussian(1500, d, 70 + d, True)
    G = knn_graph(X, 24, 0)
    codes, alpha, mu = O.build_codes(X)
    rng = np.random.default_rng(d)
    nq, J, L, budget = 4, 2, 16, 16
    Qv = gaussian(nq, d, 71 + d, True)
    seeds = rng.integers(0, X.shape[0], (nq, J)).astype(np.int32)
    Xg, Gg, Qg, Cg, Ag, Mg = to_gpu(X, G, Qv, codes, alpha, mu)
    skipped = 0
    for team in (4, 16, 64):
        for margin in (0.0, 0.03):
            note("code words", d, team, margin)
            st = E.init_states(Xg, Qg, torch.from_numpy(seeds), L=L, B=budget, D=G.shape[1],
                               team_size=team, stop_eps=0.1, kstop=10)
            E.advance(Xg, Gg, Qg, st, budget, codes=(Cg, Ag, Mg, margin))
            for qi in range(nq):
                for j in range(J):
                    br = O.init_branch(X, Qv[qi], [int(seeds[qi, j])], L=L, B=budget,
                                       D=G.shape[1], team=team)
                    O.advance_branch(X, G, Qv[qi], br, budget, budget, team=team, stop_eps=0.1,
                                     kstop=10, codes=(codes, alpha, mu, margin))
                    assert_queue(st, qi, j, br, ("codes", d, team, margin, qi, j))
            skipped += int(st.counters[..., 3].sum())
    assert skipped > 0


def test_code_filter_with_shared_table_matches_serial_schedule():
    """Codes plus the shared table (no claims, no bound): a skipped neighbour
    leaves its claimed slot unfilled and other branches score it themselves,
    so every branch's answer equals the oracle's serial schedule."""
    X, G = toy(seed=6)
    codes, alpha, mu = O.build_codes(X)
    rng = np.random.default_rng(19)
    nq, J, L, budget = 4, 4, 16, 16
    Qv = gaussian(nq, X.shape[1], 56, True)
    seeds = rng.integers(0, X.shape[0], (nq, J)).astype(np.int32)
    Xg, Gg, Qg, Cg, Ag, Mg = to_gpu(X, G, Qv, codes, alpha, mu)
    st = E.init_states(Xg, Qg, torch.from_numpy(seeds), L=L, B=budget, D=G.shape[1],
                       team_size=16, stop_eps=0.1, kstop=10, shared_cache=True)
    E.advance(Xg, Gg, Qg, st, budget, codes=(Cg, Ag, Mg, 0.05))
    Hc = st.cache_id.shape[1]
    for qi in range(nq):
        r = O.search_query(X, G, Qv[qi], seeds[qi], L=L, B=budget, team=16, stop_eps=0.1,
                           kstop=10, Hc=Hc, codes=(codes, alpha, mu, 0.05))
        assert np.array_equal(st.ids[qi].cpu().numpy(), r["ids"])
        assert st.dist[qi].cpu().numpy().tobytes() == r["dist"].tobytes()


@pytest.mark.parametrize("dtype", ["f32", "f16"])
def test_build_codes_matches_oracle(dtype):
    from swann_amd.codes import build_codes
    X = gaussian(5000, 200, 9, False)            # 200 = 6 words + 8 bits
    if dtype == "f16":
        X = X.astype(np.float16)
    Xg = torch.from_numpy(X).cuda()
    c, a, m = build_codes(Xg)
    oc, oa, om = O.build_codes(X.astype(np.float32))
    assert c.shape == (5000, 7) and c.dtype == torch.int32
    assert np.allclose(m.cpu().numpy(), om, rtol=1e-6, atol=1e-8)
    # given the same mean, the bits are exact and alpha agrees to rounding
    c2, a2, m2 = build_codes(Xg, mu=torch.from_numpy(om).cuda())
    assert np.array_equal(c2.cpu().numpy(), oc)
    assert np.allclose(a2.cpu().numpy(), oa, rtol=1e-6, atol=0)
    assert torch.equal(m2.cpu(), torch.from_numpy(om))
    # with its own mean, a bit differs only where x lies between the two
    # means (the GPU's and the oracle's sums round differently)
    mg = m.cpu().numpy().astype(np.float64)
    diff = np.unpackbits((c.cpu().numpy() ^ oc).view(np.uint8), axis=1, bitorder="little")[:, :200]
    r, t = np.nonzero(diff)
    x = X.astype(np.float32).astype(np.float64)[r, t]
    lo, hi = np.minimum(mg[t], om[t]), np.maximum(mg[t], om[t])
    assert ((x >= lo - 1e-7) & (x <= hi + 1e-7)).all()


def test_code_filter_cuts_reads_at_small_recall_cost():
    """Multi-branch search with claims and bound on a low-rank corpus: the
    filter reads fewer rows, and recall stays close (statistical: the
    reference reports 100% of admitted candidates kept at its margin)."""
    from swann_amd.codes import build_codes
    rng = np.random.default_rng(3)
    n, d, r = 20000, 128, 16
    W = rng.standard_normal((r, d)).astype(np.float32)

    def draw(m):
        x = rng.standard_normal((m, r)).astype(np.float32) @ W / np.sqrt(r)
        x += 0.1 * rng.standard_normal((m, d)).astype(np.float32)
        return (x / np.linalg.norm(x, axis=1, keepdims=True)).astype(np.float32)
    X, Q = draw(n), draw(300)
    G = knn_graph(X, 32, 0)
    Xg, Gg, Qg = to_gpu(X, G, Q)
    cd, al, cm = build_codes(Xg)
    seeds = torch.from_numpy(rng.integers(0, n, (300, 16)).astype(np.int32)).cuda()
    truth = exact_topk(X, Q, 10)
    out = {}
    for name, codes in (("plain", None), ("codes", (cd, al, cm, 0.2))):
        ids, _, st = E.search(Xg, Gg, Qg, seeds, k=10, L=32, B=48, metric=0, team_size=16,
                              stop_eps=0.1, shared_cache=True, shared_bound=True, exclusive=True,
                              elide_visited=True, codes=codes)
        out[name] = (recall(ids.cpu().numpy(), truth, 10), int(st.dist_evals.sum()))
    note("code filter recall/evals", out)
    assert out["codes"][1] < out["plain"][1]
    assert out["codes"][0] >= out["plain"][0] - 0.05


def test_interleaved_and_separate_tables_agree():
    """The shared table as one allocation of (id, d) pairs (cache_d one word
    after cache_id, as init_states allocates it, probed as 64-bit words) and
    as two separate arrays (what the reference passes) give the same answers
    and the same table contents.  Shared table on, no claims or bound: the
    queues are deterministic; whether a branch finds a neighbour's distance
    already stored (a hit) or still pending (it scores the row itself) is
    timing, so counters 1, 4 and 5 are compared through what that choice
    leaves fixed (scored + hits, scored - stores)."""
    X, G = toy(seed=8)
    rng = np.random.default_rng(23)
    nq, J, L, budget = 6, 4, 16, 20
    Qv = gaussian(nq, X.shape[1], 57, True)
    seeds = torch.from_numpy(rng.integers(0, X.shape[0], (nq, J)).astype(np.int32))
    Xg, Gg, Qg = to_gpu(X, G, Qv)
    kw = dict(L=L, B=budget, D=G.shape[1], team_size=16, stop_eps=0.1, kstop=10,
              shared_cache=True)
    a = E.init_states(Xg, Qg, seeds, **kw)
    assert a.cache_d.data_ptr() == a.cache_id.data_ptr() + 4      # interleaved pairs
    E.advance(Xg, Gg, Qg, a, budget)
    b = E.init_states(Xg, Qg, seeds, **kw)
    b.cache_id = b.cache_id.clone()
    b.cache_d = b.cache_d.clone()
    assert b.cache_d.data_ptr() != b.cache_id.data_ptr() + 4       # separate arrays
    E.advance(Xg, Gg, Qg, b, budget)
    for f in ("ids", "dist", "expanded", "lineage"):
        assert torch.equal(getattr(a, f), getattr(b, f)), f
    ca, cb = a.counters.long(), b.counters.long()
    for c in (0, 2, 3, 6, 7, 8, 9):
        assert torch.equal(ca[..., c], cb[..., c]), c
    assert torch.equal(ca[..., 1] + ca[..., 4], cb[..., 1] + cb[..., 4])
    assert torch.equal(ca[..., 1] - ca[..., 5], cb[..., 1] - cb[..., 5])
    for q in range(nq):          # same (key, distance) entries; slots may differ by insert order
        ea = sorted(zip(a.cache_id[q].tolist(), a.cache_d[q].view(torch.int32).tolist()))
        eb = sorted(zip(b.cache_id[q].tolist(), b.cache_d[q].view(torch.int32).tolist()))
        assert ea == eb, q


@pytest.mark.parametrize("bits", [False, True])
def test_claims_in_the_serial_schedule_are_exact(block, bits):
    """Claims, bound and the elided visited table made deterministic: one
    branch of each query per launch, one expansion each, is the oracle's
    serial schedule (branch 0 step s, branch 1 step s, ...).  With a table
    too sparse for a probe to fail, the (id, d) table and the claim bits
    decide every claim alike, so both equal the oracle bit for bit: queues,
    lineage and counters (claims stored, hits, scores)."""
    X, G = toy(seed=141)
    rng = np.random.default_rng(142)
    nq, J, L, budget = 5, 4, 16, 20
    Qv = gaussian(nq, X.shape[1], 143, True)
    seeds = rng.integers(0, X.shape[0], (nq, J)).astype(np.int32)
    Xg, Gg, Qg = to_gpu(X, G, Qv)
    Hc = 64 * E.next_pow2(X.shape[0])
    st = E.init_states(Xg, Qg, torch.from_numpy(seeds), L=L, B=budget, D=G.shape[1],
                       team_size=16, stop_eps=0.1, kstop=10, shared_cache=True,
                       shared_bound=True, exclusive=True, elide_visited=True,
                       cache_slots=None if bits else Hc, claim_bits=bits)
    assert st.visited.shape[-1] == 1 and (st.cache_d.numel() == 0) == bits
    for _ in range(budget):
        for j in range(J):
            act = torch.arange(nq, dtype=torch.int32, device=DEV) * J + j
            E.advance(Xg, Gg, Qg, st, 1, active=act)
    claims = 0
    for qi in range(nq):
        r = O.search_query(X, G, Qv[qi], seeds[qi], L=L, B=budget, team=16, stop_eps=0.1,
                           kstop=10, H=1, Hc=Hc, bound=True, exclusive=True, schedule="serial")
        gc = st.counters[qi].cpu().numpy()
        for j in range(J):
            assert np.array_equal(st.ids[qi, j].cpu().numpy(), r["ids"][j]), (qi, j)
            assert st.dist[qi, j].cpu().numpy().tobytes() == r["dist"][j].tobytes(), (qi, j)
            assert np.array_equal(st.expanded[qi, j].cpu().numpy(), r["expanded"][j]), (qi, j)
            assert np.array_equal(st.lineage[qi, j].cpu().numpy(), r["lineage"][j]), (qi, j)
            for c in (0, 1, 3, 4, 5, 6, 7, 8, 9):
                assert gc[j, c] == r["counters"][j, c], (qi, j, c)
        claims += int(gc[:, 4].sum())
    assert claims > 0                       # branches did meet each other's claims


def test_nan_distances_never_enter_a_queue():
    """A NaN distance (a NaN in a corpus row or in the query) has no place in
    the (d, id) order the queue is kept in: such a seed or candidate is scored
    and dropped.  Rows with a NaN never appear, every kept distance is
    finite, ids stay in range, and a query that is NaN throughout ends with
    an empty queue.  (The reference leaves this case undefined: its sorting
    network compares NaN as unordered.)"""
    X, G = toy(seed=9)
    X = X.copy()
    bad = np.array([3, 50, 700, 1200])
    X[bad, 5] = np.nan
    Qv = gaussian(4, X.shape[1], 78, True)
    Qv[3, :] = np.nan
    rng = np.random.default_rng(29)
    seeds = rng.integers(0, X.shape[0], (4, 4)).astype(np.int32)
    seeds[0, 0] = bad[0]
    seeds[1, :] = bad                                   # every seed of query 1 is NaN
    Xg, Gg, Qg = to_gpu(X, G, Qv)
    for shared in (False, True):
        note("nan rows", shared)
        st = E.init_states(Xg, Qg, torch.from_numpy(seeds), L=16, B=24, D=G.shape[1],
                           team_size=16, stop_eps=0.1, kstop=10, shared_cache=shared,
                           shared_bound=shared, exclusive=shared)
        E.advance(Xg, Gg, Qg, st, 24)
        ids = st.ids.cpu().numpy(); dist = st.dist.cpu().numpy()
        live = ids >= 0
        assert ((ids >= -1) & (ids < X.shape[0])).all()
        assert np.isfinite(dist[live]).all()
        assert not np.isin(ids[live], bad).any()
        assert (ids[3] == -1).all()
        assert live[0].any() and live[2].any()


def test_branches_spread_over_xcds_match_oracle(opt):
    """48 branches a query of 1024 threads do not fit the 32 workgroups one XCD
    holds, so the advance keeps dispatch order instead of grouping a query's
    branches on one XCD: every branch must still find its own (query,
    branch) state.  Independent branches, queues bit-exact against the
    oracle."""
    opt(search_block=1024)
    X, G = toy(seed=131)
    rng = np.random.default_rng(132)
    nq, J = 3, 48
    Qv = gaussian(nq, 64, 133, True)
    seeds = rng.integers(0, X.shape[0], (nq, J)).astype(np.int32)
    Xg, Gg, Qg = to_gpu(X, G, Qv)
    st = E.init_states(Xg, Qg, torch.from_numpy(seeds), L=12, B=30, D=32, team_size=16,
                       stop_eps=0.05)
    E.advance(Xg, Gg, Qg, st, 30)
    for qi in range(nq):
        for j in range(0, J, 5):
            br = O.run(X, G, Qv[qi], int(seeds[qi, j]), L=12, B=30, team=16, stop_eps=0.05)
            assert_queue(st, qi, j, br, (qi, j))
