"""Pin the CPU oracle before it judges anything (CPU only).

Each check is chosen so that a plausible mistake in the oracle -- a dropped
term, a wrong lane index, a reversed tree, a wrong tie-break, a lost lineage --
fails one of them:

  * golden vectors written from the reference's own _refcpu.py and CPU-torch
    build stages (tests/golden/make_golden.py);
  * closed forms: integer-valued inputs make every summation order exact;
  * hand-built cases whose value depends on the lane layout and the tree order;
  * brute force: complete graph, exact top-k, exact merge.
"""
import numpy as np
import pytest

import oracle as O
from conftest import deg96_corpus, gaussian, golden, regen
from test_oracle_helpers import crowd_case, stall_case, untied_graph_rows, untied_rows

F32MAX = np.finfo(np.float32).max


# -- distance ----------------------------------------------------------------
def test_distance_matches_reference_vectors():
    g = golden("refcpu_distance.npz")
    for i in range(int(g["n"])):
        d, metric, team = (int(v) for v in g[f"c{i}_meta"])
        q, x, x16 = g[f"c{i}_q"], g[f"c{i}_x"], g[f"c{i}_x16"]
        got32 = O.team_distance(q, x[None, :], 0, metric, team)
        got16 = O.team_distance(q, x16[None, :], 0, metric, team)
        assert got32.tobytes() == g[f"c{i}_d32"].tobytes(), (d, metric, team, "fp32")
        assert got16.tobytes() == g[f"c{i}_d16"].tobytes(), (d, metric, team, "fp16")


@pytest.mark.parametrize("team", [4, 8, 16, 32, 64])
@pytest.mark.parametrize("metric", [O.METRIC_IP, O.METRIC_L2])
def test_distance_integer_inputs_are_exact(team, metric):
    """Small integers: every partial sum is exact, so any order gives the
    true value -- a dropped, doubled or misindexed term cannot hide."""
    rng = np.random.default_rng(5)
    for d in (1, 5, 8, 64, 96, 130, 1536):
        q = rng.integers(-3, 4, d).astype(np.float32)
        x = rng.integers(-3, 4, (3, d)).astype(np.float32)
        for r in range(3):
            if metric == O.METRIC_IP:
                want = np.float32(1.0 - float(np.dot(q.astype(np.int64), x[r].astype(np.int64))))
            else:
                want = np.float32(float(((q - x[r]).astype(np.int64) ** 2).sum()))
            assert O.team_distance(q, x, r, metric, team) == want
            assert O.team_distance(q, x.astype(np.float16), r, metric, team) == want


def test_distance_lane_layout_fp32():
    """team=2, vec=4: lane 0 owns elements 0-3 and 8-11, lane 1 owns 4-7 and
    12-15.  2^24 and -2^24 both fall to lane 0, so the 1s in lane 1 survive:
    the kernel's order gives 2; summing in element order would give 0."""
    q = np.ones(16, np.float32)
    x = np.zeros(16, np.float32)
    x[0], x[4], x[5], x[8] = 2.0 ** 24, 1.0, 1.0, -(2.0 ** 24)
    assert O.team_distance(q, x[None], 0, O.METRIC_IP, 2) == np.float32(1 - 2)
    # within lane 0 the order is sequential: 2^24 + 1 + 1 rounds back to 2^24
    x2 = np.zeros(16, np.float32)
    x2[0], x2[1], x2[2], x2[8] = 2.0 ** 24, 1.0, 1.0, -(2.0 ** 24)
    assert O.team_distance(q, x2[None], 0, O.METRIC_IP, 2) == np.float32(1 - 0)


def test_distance_lane_layout_fp16():
    """fp16 reads 8 elements per lane per step: with team=2 lane 0 owns 0-7
    and 16-23, lane 1 owns 8-15.  Products 2^13*2048 = 2^24 at 0 and -2^24 at
    16 cancel in lane 0 and the 1 at element 8 survives in lane 1: result 1.
    With vec=4 element 8 would join lane 0 between them and be rounded away
    (2^24 + 1 = 2^24), giving 0."""
    q = np.ones(32, np.float32)
    q[0] = q[16] = 2.0 ** 13
    x = np.zeros(32, np.float16)
    x[0], x[8], x[16] = 2048, 1, -2048
    assert O.team_distance(q, x[None], 0, O.METRIC_IP, 2) == np.float32(1 - 1)


def test_distance_tree_is_halving_from_the_top():
    """team=4, one value per lane: [2^24, 1, -2^24, 1].  Folding off=2 then
    off=1 gives (2^24 - 2^24) + (1 + 1) = 2; folding off=1 first would give 1."""
    q = np.ones(16, np.float32)
    x = np.zeros(16, np.float32)
    x[0], x[4], x[8], x[12] = 2.0 ** 24, 1.0, -(2.0 ** 24), 1.0
    assert O.team_distance(q, x[None], 0, O.METRIC_IP, 4) == np.float32(1 - 2)


def test_distance_l2_is_rounded_square_then_sum():
    """L2 terms are fl(fl(q-x)^2): q - x = 1 + 2^-12 squares to 1 + 2^-11 +
    2^-24, whose last bit fp32 rounds away (ties to even)."""
    q = np.array([1.0 + 2.0 ** -12, 0, 0, 0], np.float32)
    x = np.zeros((1, 4), np.float32)
    assert O.team_distance(q, x, 0, O.METRIC_L2, 4) == np.float32(1.0 + 2.0 ** -11)


def test_half_conversion_is_exact():
    h = np.arange(0, 1 << 16, dtype=np.uint32).astype(np.uint16)
    f = h.view(np.float16).astype(np.float32)
    L = O.lib()
    got = np.array([L.so_half_to_float_export(int(v)) for v in h[::97]], np.float32)
    want = f[::97]
    same = (got.view(np.uint32) == want.view(np.uint32)) | (np.isnan(got) & np.isnan(want))
    assert same.all()


# -- one branch -------------------------------------------------------------
def _check_branch(br, g, key, L, what):
    ids = g[f"{key}_ids"]; dist = g[f"{key}_dist"]; expd = g[f"{key}_expanded"]
    lin = g[f"{key}_lineage"]; ctr = g[f"{key}_counters"]
    n = int((ids >= 0).sum())
    assert list(br.ids[:n]) == list(ids[:n]) and (br.ids[n:] == -1).all(), what
    assert br.dist[:n].tobytes() == dist[:n].tobytes(), what
    assert list(br.expanded[:n]) == list(expd[:n]), what
    assert list(br.lineage[:n]) == list(lin[:n]), what
    assert br.counters[0] == ctr[0] and br.counters[1] == ctr[1], what
    assert int(br.counters[3]) == int(ctr[2]), what


@pytest.mark.parametrize("tag,metric", [("ip", O.METRIC_IP), ("l2", O.METRIC_L2)])
def test_branch_matches_refcpu_every_team(tag, metric):
    g = golden("refcpu_branch.npz")
    X = regen(2000, 64, 0, metric == O.METRIC_IP, g[f"{tag}_X_sha"])
    G = g[f"{tag}_G"].astype(np.int32); Q = g[f"{tag}_Q"]; seeds = g[f"{tag}_seeds"]
    for team in (4, 8, 16, 32):
        for q in range(Q.shape[0]):
            for j in range(seeds.shape[1]):
                br = O.run(X, G, Q[q], int(seeds[q, j]), L=16, B=12, metric=metric, team=team)
                sub = {k[len(f"{tag}_t{team}_"):]: v[q, j] for k, v in g.items()
                       if k.startswith(f"{tag}_t{team}_")}
                _check_branch(br, {f"x_{k}": v for k, v in sub.items()}, "x", 16,
                              (tag, team, q, j))


@pytest.mark.parametrize("pol", [O.POLICY_BEST, O.POLICY_ROUND_ROBIN])
def test_multiseed_matches_refcpu(pol):
    g = golden("refcpu_branch.npz")
    X = regen(2000, 64, 53, True, g["ms_X_sha"])
    G = g["ms_G"].astype(np.int32); Q = g["ms_Q"]; seeds = g["ms_seeds"]
    for q in range(Q.shape[0]):
        br = O.run(X, G, Q[q], list(seeds[q]), L=32, B=20, policy=pol)
        _check_branch(br, {f"x_{n}": g[f"ms_p{pol}_{n}"][q] for n in
                           ("ids", "dist", "expanded", "lineage", "counters")}, "x", 32, (pol, q))


def test_early_stop_matches_refcpu():
    g = golden("refcpu_branch.npz")
    X = regen(2000, 64, 71, True, g["es_X_sha"])
    G = g["es_G"].astype(np.int32); Q = g["es_Q"]; seeds = g["es_seeds"]
    for e, eps in enumerate((0.0, 0.1, 0.25)):
        for q in range(Q.shape[0]):
            br = O.run(X, G, Q[q], list(seeds[q]), L=32, B=64, policy=O.POLICY_ROUND_ROBIN,
                       stop_eps=eps, kstop=10)
            _check_branch(br, {f"x_{n}": g[f"es_e{e}_{n}"][q] for n in
                               ("ids", "dist", "expanded", "lineage", "counters")}, "x", 32,
                          (eps, q))
            assert br.counters[0] < 64


def test_complete_graph_equals_brute_force():
    """tests/test_engine.py:122-142: one expansion over a complete graph sees
    every node, so the queue is the exact top-L."""
    n, d, L = 96, 48, 16
    rng = np.random.default_rng(17)
    X = gaussian(n, d, 17, True)
    G = np.stack([np.delete(np.arange(n), i) for i in range(n)]).astype(np.int32)[:, :95]
    Q = gaussian(6, d, 18, True)
    for qi in range(6):
        br = O.run(X, G, Q[qi], 0, L=L, B=1)
        exact = 1.0 - (Q[qi].astype(np.float64) @ X.astype(np.float64).T)
        want = np.argsort(exact, kind="stable")[:L]
        # node 0 is the seed and is never its own neighbour; it is in the
        # queue only if it ranks, which the brute force also says
        assert list(br.ids) == list(want)
        assert np.allclose(br.dist, exact[want], atol=2e-6)
    del rng


def test_dead_branch_and_sink():
    n, d = 64, 16
    X = gaussian(n, d, 19, True)
    G = np.full((n, 8), -1, np.int32)
    q = gaussian(1, d, 20, True)[0]
    br = O.run(X, G, q, 0, L=16, B=16)
    assert br.counters[0] == 1 and br.counters[3] == 1
    br = O.run(X, G, q, -1, L=16, B=16)
    assert br.counters[0] == 0 and br.counters[3] == 1 and (br.ids == -1).all()


def test_resume_equivalence():
    X = gaussian(2000, 64, 3, True)
    from test_oracle_helpers import knn_graph
    G = knn_graph(X, 32)
    Q = gaussian(4, 64, 4, True)
    for qi in range(4):
        one = O.init_branch(X, Q[qi], [qi * 7], L=32, B=24, D=32)
        O.advance_branch(X, G, Q[qi], one, 24, 24)
        for split in (1, 2, 7, 23):
            two = O.init_branch(X, Q[qi], [qi * 7], L=32, B=24, D=32)
            O.advance_branch(X, G, Q[qi], two, split, 24)
            O.advance_branch(X, G, Q[qi], two, 24 - split, 24)
            for f in ("ids", "dist", "expanded", "lineage", "visited", "counters"):
                assert np.array_equal(getattr(one, f), getattr(two, f)), (qi, split, f)


def test_budget_is_a_state_property():
    X = gaussian(2000, 64, 5, True)
    from test_oracle_helpers import knn_graph
    G = knn_graph(X, 32)
    q = gaussian(1, 64, 6, True)[0]
    br = O.init_branch(X, q, [3, 99], L=16, B=10, D=32)
    O.advance_branch(X, G, q, br, 100, 10)
    assert br.counters[0] == 10


def test_visited_overflow_is_counted():
    X = gaussian(1000, 64, 23, True)
    from test_oracle_helpers import knn_graph
    G = knn_graph(X, 32)
    q = gaussian(1, 64, 24, True)[0]
    br = O.init_branch(X, q, [0], L=16, H=64, B=16, D=32)
    O.advance_branch(X, G, q, br, 16, 16)
    assert br.counters[2] > 0


# -- several branches of one query --------------------------------------------
def test_shared_cache_changes_work_not_results():
    """tests/test_engine.py:213-239, in the serial schedule."""
    X = gaussian(2000, 64, 79, True)
    from test_oracle_helpers import knn_graph
    G = knn_graph(X, 32)
    Q = gaussian(6, 64, 80, True)
    rng = np.random.default_rng(83)
    for qi in range(6):
        seeds = rng.integers(0, 2000, 24).astype(np.int32)
        plain = O.search_query(X, G, Q[qi], seeds, L=32, B=12)
        Hc = O.cache_size(24, 12, 32)
        cached = O.search_query(X, G, Q[qi], seeds, L=32, B=12, Hc=Hc)
        for f in ("ids", "dist", "expanded", "lineage"):
            assert np.array_equal(plain[f], cached[f]), f
        a = plain["counters"][:, 1].sum(); b = cached["counters"][:, 1].sum()
        hits = cached["counters"][:, 4].sum()
        assert b < a and a - b == hits


def test_claims_keep_branches_disjoint():
    """Exclusive claims with the visited table elided: a node scored by one
    branch is never entered by another (seeds aside, which are not claimed)."""
    X = gaussian(2000, 64, 81, True)
    from test_oracle_helpers import knn_graph
    G = knn_graph(X, 32)
    q = gaussian(1, 64, 82, True)[0]
    seeds = np.random.default_rng(84).integers(0, 2000, 16).astype(np.int32)
    Hc = O.cache_size(16, 16, 32)
    r = O.search_query(X, G, q, seeds, L=12, B=16, H=1, Hc=Hc, bound=True, exclusive=True,
                       stop_eps=0.05)
    owner = {}
    for j in range(16):
        for i in r["ids"][j]:
            if i < 0 or i in set(seeds.tolist()):
                continue
            assert owner.setdefault(int(i), j) == j
    # every cached distance is the exact team distance
    for slot in np.nonzero(r["cache_id"])[0][:50]:
        v = int(r["cache_id"][slot]) - 1
        assert r["cache_d"][slot] == O.team_distance(q, X, v, O.METRIC_IP, 32)


@pytest.mark.parametrize("schedule", ["serial", "rounds", "rounds2"])
def test_claim_bits_decide_like_a_table_that_never_fails(schedule):
    """Exclusive claims as one bit per row equal the (id, d) table wherever
    the table's probes never fail: every queue, lineage and counter.  A
    small table, whose probe chains do run out, must differ (a failed probe
    scores the row and keeps it as a candidate, a bit never fails), and so
    must the bits without exclusive claims' skip of an owned row."""
    X = gaussian(2000, 64, 85, True)
    from test_oracle_helpers import knn_graph
    G = knn_graph(X, 32)
    Q = gaussian(6, 64, 86, True)
    rng = np.random.default_rng(87)
    kw = dict(L=12, B=24, H=1, bound=True, exclusive=True, stop_eps=0.05, schedule=schedule)
    differs_small = 0
    for qi in range(6):
        seeds = rng.integers(0, 2000, 16).astype(np.int32)
        bits = O.search_query(X, G, Q[qi], seeds, claim_bits=True, **kw)
        table = O.search_query(X, G, Q[qi], seeds, Hc=1 << 17, **kw)
        for f in ("ids", "dist", "expanded", "lineage", "counters"):
            assert np.array_equal(bits[f], table[f]), (qi, f)
        assert bits["counters"][:, 4].sum() > 0                 # branches met
        owned = np.unpackbits(bits["cache_id"].view(np.uint8), bitorder="little")
        assert owned.sum() == bits["counters"][:, 5].sum()     # one bit per claim
        small = O.search_query(X, G, Q[qi], seeds, Hc=32, **kw)
        differs_small += not np.array_equal(small["counters"], bits["counters"])
    assert differs_small > 0
    with pytest.raises(ValueError):
        O.search_query(X, G, Q[0], seeds, claim_bits=True, L=12, B=24, H=1, exclusive=False)


@pytest.mark.parametrize("schedule", ["serial", "rounds", "rounds2"])
@pytest.mark.parametrize("kstop", [1, 5, 10, 40])
@pytest.mark.parametrize("exclusive", [False, True])
def test_bound_is_the_least_kth_distance_any_branch_reached(kstop, exclusive, schedule):
    """The shared bound is lowered after every expansion to the branch's
    kr-th distance, kr = min(kstop, L) (local_search.cu:655-658).  A queue
    position only ever improves, so the final bound must equal, bit for bit,
    the least final kr-th distance over the branches that expanded at least
    once with that position filled -- and stay FLT_MAX when none did.  A bound
    never lowered, lowered from the wrong position (L-th instead of kr-th) or
    from a branch's seeds fails this.  L2 keeps every distance >= 0, where the
    integer atomicMin on the bits is the float minimum."""
    X = gaussian(2000, 64, 91, False)
    from test_oracle_helpers import knn_graph
    G = knn_graph(X, 16, metric=1)
    Q = gaussian(8, 64, 92, False)
    rng = np.random.default_rng(93)
    L = 12
    kr = min(kstop, L)
    for qi in range(8):
        seeds = rng.integers(0, 2000, 12).astype(np.int32)
        Hc = O.cache_size(12, 10, 16) if exclusive else 0
        r = O.search_query(X, G, Q[qi], seeds, L=L, B=10, metric=O.METRIC_L2, H=None if not
                           exclusive else 1, Hc=Hc, bound=True, exclusive=exclusive,
                           stop_eps=0.1, kstop=kstop, schedule=schedule)
        live = (r["counters"][:, 0] >= 1) & (r["ids"][:, kr - 1] >= 0)
        want = r["dist"][live, kr - 1].min() if live.any() else F32MAX
        assert np.float32(r["bound"]).tobytes() == np.float32(want).tobytes(), (qi, kstop)
        assert live.any()


def _bound_case():
    """L2 on a line (dim 4, fp32).  Node 0 sits at distance 1 from the query
    and its only neighbour, node 1, at 0.25.  Nodes 5, 6, 7, 8 form a chain
    walking in from distance 100 (10, 9, 8, 7 along the axis); node 8 is a
    dead end.  With kstop = 1 and stop_eps = 0 a branch expands only while its
    best entry is unexpanded and within its radius."""
    X = np.zeros((10, 4), np.float32)
    X[0, 0], X[1, 0] = 1.0, 0.5
    for i, x in zip((5, 6, 7, 8), (10.0, 9.0, 8.0, 7.0)):
        X[i, 0] = x
    G = np.full((10, 2), -1, np.int32)
    G[0, 0], G[1, 0] = 1, 0
    G[5, 0], G[6, 0], G[7, 0] = 6, 7, 8
    return X, G, np.zeros(4, np.float32)


@pytest.mark.parametrize("schedule", ["serial", "rounds", "rounds2"])
@pytest.mark.parametrize("near_first", [True, False])
def test_bound_stops_a_branch_its_own_radius_would_not(near_first, schedule):
    """Two branches of one query, the near one seeded at node 0, the far one
    at node 5.  Alone, the far branch walks the whole chain (4 expansions).
    With the shared bound, the near branch's first expansion lowers the bound
    to 0.25; the far branch's next pick (distance >= 49) then exceeds
    min(own radius, bound) and it stops, exhausted.  The serial schedule
    steps branch 0 then branch 1 and each step reads the bound as the one
    before it left it: stepped after the near branch the far one expands
    nothing; stepped before it, exactly one node.  In rounds, both branches'
    first steps read the bound the round began with (FLT_MAX), so the far
    branch expands exactly one node in either order; in rounds2 a step reads
    the bound as the round before began, so the far branch's second step
    still reads FLT_MAX and it expands exactly two.  A bound that is read but
    ignored, or never lowered, gives 4."""
    X, G, q = _bound_case()
    seeds = np.array([0, 5] if near_first else [5, 0], np.int32)
    far = 1 if near_first else 0
    kw = dict(L=4, B=8, metric=O.METRIC_L2, team=4, stop_eps=0.0, kstop=1, schedule=schedule)
    alone = O.search_query(X, G, q, seeds, bound=False, **kw)
    assert alone["counters"][far, 0] == 4
    r = O.search_query(X, G, q, seeds, bound=True, **kw)
    want = {"serial": 0 if near_first else 1, "rounds": 1, "rounds2": 2}[schedule]
    assert r["counters"][far, 0] == want
    assert r["counters"][far, 3] == 1
    assert r["counters"][1 - far, 0] == 2          # node 0, then node 1
    assert r["bound"] == np.float32(0.25)
    # the near branch is untouched by the bound: it owns the bound's value
    assert np.array_equal(r["ids"][1 - far], alone["ids"][1 - far])


def test_schedules_agree_without_a_bound():
    """The three schedules differ only in when a branch sees the shared
    bound: with the bound off they give the same queues, bit for bit (claims
    land at once in all three)."""
    X = gaussian(3000, 32, 95, True)
    from test_oracle_helpers import knn_graph
    G = knn_graph(X, 16, 0)
    Q = gaussian(4, 32, 96, True)
    seeds = np.random.default_rng(97).integers(0, 3000, (4, 8)).astype(np.int32)
    out = {}
    for sch in ("serial", "rounds", "rounds2"):
        oi, od = O.search_batch(X, G, Q, seeds, k=10, L=12, B=20, team=16, stop_eps=0.05,
                                H=1, Hc=None, bound=False, exclusive=True, schedule=sch,
                                claim_bits=True, nthreads=2)
        out[sch] = (oi, od.tobytes())
    assert all(np.array_equal(out[s][0], out["serial"][0]) and out[s][1] == out["serial"][1]
               for s in out)


# -- merge ----------------------------------------------------------------------
def test_merge_is_a_dedup_selection():
    rng = np.random.default_rng(37)
    Q, V, kk, k = 20, 5, 10, 10
    ids = rng.integers(-1, 40, (Q, V, kk)).astype(np.int32)
    base = rng.random(40).astype(np.float32)
    dist = np.where(ids >= 0, base[np.clip(ids, 0, None)], F32MAX).astype(np.float32)
    oi, od = O.merge(ids, dist, k)
    for q in range(Q):
        pool = {}
        for j in range(V):
            for t in range(kk):
                if ids[q, j, t] >= 0:
                    pool.setdefault(int(ids[q, j, t]), float(dist[q, j, t]))
        want = sorted(pool.items(), key=lambda kv: (kv[1], kv[0]))[:k]
        got = [(int(i), float(d)) for i, d in zip(oi[q], od[q]) if i >= 0]
        assert got == [(i, float(np.float32(d))) for i, d in want]
        assert (oi[q, len(want):] == -1).all() and np.isinf(od[q, len(want):]).all()


# -- config C1 against the reference path ----------------------------------------
def test_c1_branches_match_refcpu():
    g = golden("refcpu_c1.npz")
    X = regen(10000, 128, 0, True, g["X_sha"])
    G = g["G"].astype(np.int32); Q = g["Q"]; seeds = g["seeds"].astype(np.int32)
    for q in range(0, 200, 5):
        for j in range(8):
            br = O.run(X, G, Q[q], int(seeds[q, j]), L=12, B=64, metric=O.METRIC_IP, team=16,
                       stop_eps=0.05, kstop=10)
            n = int((g["ids"][q, j] >= 0).sum())
            assert list(br.ids[:n]) == list(g["ids"][q, j, :n].astype(np.int32)), (q, j)
            assert br.dist[:n].tobytes() == g["dist"][q, j, :n].tobytes(), (q, j)
            assert br.counters[0] == g["counters"][q, j, 0]
            assert br.counters[1] == g["counters"][q, j, 1]


def test_c1_merged_answer_matches_reference():
    g = golden("refcpu_c1.npz")
    X = regen(10000, 128, 0, True, g["X_sha"])
    G = g["G"].astype(np.int32); Q = g["Q"]; seeds = g["seeds"].astype(np.int32)
    oi, od = O.search_batch(X, G, Q, seeds, k=10, L=12, B=64, metric=O.METRIC_IP, team=16,
                            stop_eps=0.05, nthreads=4)
    assert np.array_equal(oi, g["merged_ids"].astype(np.int32))
    assert od.tobytes() == g["merged_dist"].astype(np.float32).tobytes()


def test_c1_select_matches_reference():
    """_select.py:93-128 in fp32: the E=8 nearest catalogue rows."""
    g = golden("refcpu_c1.npz")
    X = regen(10000, 128, 0, True, g["X_sha"])
    cat = g["catalogue"].astype(np.int64)
    want = np.random.default_rng(0).permutation(10000)[:4096]
    assert np.array_equal(cat, np.sort(want))
    idx, _ = O.select_nearest(g["Q"], X[cat], 8, O.METRIC_IP, nthreads=4)
    got = cat[idx].astype(np.int32)
    want = g["seeds"].astype(np.int32)
    Q64 = g["Q"].astype(np.float64)
    dist = lambda s: 1.0 - np.einsum("qd,qkd->qk", Q64, X[s].astype(np.float64))  # noqa: E731
    assert untied_rows(got, want, dist(want), dist(got)) == []


# -- build stages ---------------------------------------------------------------
@pytest.mark.parametrize("tag,metric", [("ip", O.METRIC_IP), ("l2", O.METRIC_L2)])
def test_sweep_matches_reference(tag, metric):
    g = golden("refbuild_small.npz")
    X = g[f"{tag}_X"]
    cand, cdist = O.knn_candidates(X, 32, metric, nthreads=4)
    rc = g[f"{tag}_cand"].astype(np.int32); rd = g[f"{tag}_cdist"]
    assert untied_rows(cand, rc, rd, cdist) == []
    assert np.allclose(cdist, rd, atol=2e-5, rtol=1e-5)


@pytest.mark.parametrize("tag,metric", [("ip", O.METRIC_IP), ("l2", O.METRIC_L2)])
def test_prune_and_reverse_match_reference(tag, metric):
    g = golden("refbuild_small.npz")
    X = g[f"{tag}_X"]
    rc = g[f"{tag}_cand"].astype(np.int32); rd = g[f"{tag}_cdist"]
    Gp = O.robust_prune(X, rc, rd, 16, 1.2, metric, nthreads=4)
    want_p = g[f"{tag}_Gp"].astype(np.int32)
    assert np.array_equal(Gp, want_p)
    Gf = O.add_reverse(X, want_p, 16, 1.2, 64, metric, nthreads=4)
    assert untied_graph_rows(Gf, g[f"{tag}_Gf"].astype(np.int32), X, metric) == []


def _union_width(Gp, max_in=64):
    """Per node: distinct out-neighbours plus the first max_in in-sources in
    ascending source order (add_reverse's union before its cut)."""
    ins = [[] for _ in range(Gp.shape[0])]
    for u, row in enumerate(Gp):
        for v in row[row >= 0]:
            ins[v].append(u)
    return np.array([len(set(row[row >= 0].tolist()) | set(ins[u][:max_in]))
                     for u, row in enumerate(Gp)])


@pytest.mark.parametrize("tag,metric", [("ip", O.METRIC_IP), ("l2", O.METRIC_L2)])
def test_build_at_default_degree_matches_reference(tag, metric):
    """The build at the reference API's defaults (build.py:153-171,
    index.py:76: candidates 128, degree 96, alpha 1.2, max_in 64), where
    add_reverse's 160-wide union is cut to its 128 nearest (build.py:138-148):
    the sweep equal up to ties, the prune identical, the reverse pass equal up
    to the order of tied neighbours (tests/golden/refbuild_deg96.npz)."""
    g = golden("refbuild_deg96.npz")
    X = deg96_corpus(tag, g)
    rc = g[f"{tag}_cand"].astype(np.int32); rd = g[f"{tag}_cdist"]
    cand, cdist = O.knn_candidates(X, 128, metric, nthreads=8)
    assert untied_rows(cand, rc, rd, cdist) == []
    want_p = g[f"{tag}_Gp"].astype(np.int32)
    assert np.array_equal(O.robust_prune(X, rc, rd, 96, 1.2, metric, nthreads=8), want_p)
    assert (_union_width(want_p) > 128).sum() >= 100        # the cut binds on many rows
    want_f = g[f"{tag}_Gf"].astype(np.int32)
    Gf = O.add_reverse(X, want_p, 96, 1.2, 64, metric, nthreads=8)
    assert untied_graph_rows(Gf, want_f, X, metric) == []


@pytest.mark.parametrize("tag,metric", [("adv_l2", O.METRIC_L2), ("adv_ip", O.METRIC_IP)])
def test_reverse_cut_and_in_edge_order_match_reference(tag, metric):
    """A hand-made graph on which add_reverse's cut to 128 and its
    ascending-source in-edges decide node 0's row (1 + 32 neighbours, as
    tests/golden/make_golden.py:reverse_cut_case lays out): the oracle equals
    the reference on every row, and a re-prune of node 0's whole 160-wide
    union, or of a union with the last 64 in-sources, would not."""
    g = golden("refbuild_deg96.npz")
    X = g[f"{tag}_X"]; G = g[f"{tag}_G"].astype(np.int32)
    want = g[f"{tag}_Gf"].astype(np.int32)
    assert (want[0] >= 0).sum() == 33
    assert untied_graph_rows(O.add_reverse(X, G, 96, 1.2, 64, metric, nthreads=4), want, X,
                             metric) == []
    ins = [u for u in range(X.shape[0]) if 0 in G[u]]
    assert len(ins) == 70

    def prune_union(extra, cut=160):
        ids = np.array(sorted(set(G[0][G[0] >= 0].tolist()) | set(extra)), np.int64)
        X64 = X.astype(np.float64)
        d = (((X64[ids] - X64[0]) ** 2).sum(1) if metric == O.METRIC_L2
             else 1.0 - X64[ids] @ X64[0]).astype(np.float32)
        o = np.argsort(d, kind="stable")
        c = np.full((X.shape[0], 160), -1, np.int32); cd = np.full(c.shape, np.inf, np.float32)
        w = min(len(ids), cut)
        c[0, :w] = ids[o][:w]; cd[0, :w] = d[o][:w]
        return O.robust_prune(X, c, cd, 96, 1.2, metric, nthreads=1)[0]
    assert set(prune_union(ins[:64], 128).tolist()) == set(want[0].tolist())
    assert (prune_union(ins[:64]) >= 0).sum() == 65                          # no cut
    assert set(prune_union(ins[-64:], 128).tolist()) != set(want[0].tolist())  # other in-edges


@pytest.mark.parametrize("tag,metric", [("ip", O.METRIC_IP), ("l2", O.METRIC_L2)])
def test_prune_per_node_degree_and_protect_match_reference(tag, metric):
    """robust_prune's deg_per_node and protect, and add_reverse's
    deg_per_node, against the reference's CPU-torch build.py on its own
    candidate lists (tests/golden/refbuild_extras.npz)."""
    g = golden("refbuild_extras.npz")
    X = regen(800, 24, 23 if tag == "ip" else 24, tag == "ip", g[f"{tag}_X_sha"])
    rc = g[f"{tag}_cand"].astype(np.int32); rd = g[f"{tag}_cdist"]
    dpn = g[f"{tag}_dpn"].astype(np.int32); prot = g[f"{tag}_prot"]
    for key, kw in (("Gp", {}), ("Gd", dict(deg_per_node=dpn)), ("Gm", dict(protect=prot)),
                    ("Gb", dict(deg_per_node=dpn, protect=prot))):
        got = O.robust_prune(X, rc, rd, 12, 1.2, metric, nthreads=4, **kw)
        want = g[f"{tag}_{key}"].astype(np.int32)
        assert got.shape == want.shape, key
        assert np.array_equal(got, want), key
    got = O.add_reverse(X, g[f"{tag}_Gd"].astype(np.int32), 12, 1.2, 64, metric, nthreads=4,
                        deg_per_node=dpn)
    assert untied_graph_rows(got, g[f"{tag}_Rd"].astype(np.int32), X, metric) == []


def test_prune_caps_and_protect_closed_forms():
    """A cap keeps a prefix of the uncapped kept list; protecting every
    candidate keeps the first cap valid ones; protecting none is no protect."""
    X = gaussian(600, 20, 61, False)
    rc, rd = O.knn_candidates(X, 32, O.METRIC_L2, nthreads=4)
    rc[::7, 5] = -1                                   # holes are never kept
    full = O.robust_prune(X, rc, rd, 32, 1.2, O.METRIC_L2, nthreads=4)
    caps = np.random.default_rng(3).integers(1, 20, 600).astype(np.int32)
    capped = O.robust_prune(X, rc, rd, 20, 1.2, O.METRIC_L2, nthreads=4, deg_per_node=caps)
    assert capped.shape == (600, int(caps.max()))
    for u in range(600):
        k = min(caps[u], int((full[u] >= 0).sum()))
        assert list(capped[u, :k]) == list(full[u, :k])
        assert (capped[u, k:] == -1).all()
    allp = O.robust_prune(X, rc, rd, 12, 1.2, O.METRIC_L2, nthreads=4,
                          protect=np.ones(rc.shape, bool))
    for u in range(600):
        valid = [c for c in rc[u] if c >= 0][:12]
        assert list(allp[u, :len(valid)]) == valid
    nonep = O.robust_prune(X, rc, rd, 12, 1.2, O.METRIC_L2, nthreads=4,
                           protect=np.zeros(rc.shape, bool))
    assert np.array_equal(nonep, O.robust_prune(X, rc, rd, 12, 1.2, O.METRIC_L2, nthreads=4))


def test_prune_rule_invariants():
    """DiskANN's rule, stated as invariants: every kept edge has no kept,
    nearer neighbour that is alpha-closer to it; every dropped candidate
    (before the row filled) has one."""
    X = gaussian(400, 16, 31, False)
    cand, cdist = O.knn_candidates(X, 24, O.METRIC_L2)
    G = O.robust_prune(X, cand, cdist, 8, 1.2, O.METRIC_L2)
    X64 = X.astype(np.float64)
    for u in range(0, 400, 7):
        kept = [c for c in G[u] if c >= 0]
        pos = {int(c): i for i, c in enumerate(cand[u])}
        assert [pos[c] for c in kept] == sorted(pos[c] for c in kept)
        for i, c in enumerate(cand[u]):
            if len([k for k in kept if pos[k] < i]) >= 8:
                break
            blockers = [w for w in kept if pos[w] < i and
                        1.2 * ((X64[w] - X64[c]) ** 2).sum() <= cdist[u, i] + 1e-4]
            if c in kept:
                assert not [w for w in kept if pos[w] < i and
                            1.2 * ((X64[w] - X64[c]) ** 2).sum() <= cdist[u, i] - 1e-4]
            else:
                assert blockers


# -- sign-code filter (local_search.cu:205-243, :560-575) ---------------------
def test_code_builder_matches_its_definition():
    """Bits are x > mu with bit b of word w for dimension 32w + b; mu is the
    column mean and alpha the mean |x - mu| (both against float64 numpy)."""
    rng = np.random.default_rng(21)
    X = rng.standard_normal((60, 70)).astype(np.float32)
    codes, alpha, mu = O.build_codes(X)
    assert codes.shape == (60, 3) and codes.dtype == np.int32
    assert np.allclose(mu, X.astype(np.float64).mean(0), rtol=0, atol=1e-7)
    w = codes.view(np.uint32)
    bits = np.stack([(w[:, t // 32] >> np.uint32(t % 32)) & 1 for t in range(70)], 1)
    assert np.array_equal(bits.astype(bool), X > mu[None, :])
    assert (w[:, 2] >> np.uint32(6)).max() == 0                       # bits past dim stay 0
    want = np.abs(X.astype(np.float64) - mu.astype(np.float64)).mean(1)
    assert np.allclose(alpha, want, rtol=1e-6, atol=0)
    # a given mu is used as is
    c2, a2, m2 = O.build_codes(X, mu=np.zeros(70, np.float32))
    assert np.array_equal(m2, np.zeros(70, np.float32))
    w2 = c2.view(np.uint32)
    assert np.array_equal(np.stack([(w2[:, t // 32] >> np.uint32(t % 32)) & 1 for t in range(70)], 1)
                          .astype(bool), X > 0)
    assert np.allclose(a2, np.abs(X.astype(np.float64)).mean(1), rtol=1e-6)


def test_code_estimate_closed_form():
    """1 - (alpha <q, b> + <q, mu>) with b in {-1, +1}, in float64, for every
    team: a dropped sum(q), a sign error or a misread bit moves it by O(1)."""
    rng = np.random.default_rng(22)
    for d in (32, 70, 128, 1536):
        X = rng.standard_normal((5, d)).astype(np.float32)
        codes, alpha, mu = O.build_codes(X)
        q = rng.standard_normal(d).astype(np.float32) / np.sqrt(d)
        for r in range(5):
            b = np.where(X[r] > mu, 1.0, -1.0)
            want = 1.0 - (float(alpha[r]) * float(q.astype(np.float64) @ b)
                          + float(q.astype(np.float64) @ mu.astype(np.float64)))
            for team in (4, 16, 64):
                got = O.code_ip(q, codes[r], alpha[r], mu, team)
                assert abs(float(got) - want) < 1e-5 * max(1.0, abs(want)), (d, r, team)


def test_code_estimate_bit_order():
    """q = 3 e_37 and mu = 0: the estimate is 1 - alpha (2 * 3 * bit - 3), so
    only bit 5 of word 1 may move it."""
    q = np.zeros(70, np.float32); q[37] = 3.0
    mu = np.zeros(70, np.float32)
    code = np.zeros(3, np.int32)
    assert O.code_ip(q, code, 0.5, mu, 4) == np.float32(1.0 - 0.5 * -3.0)
    code[1] = 1 << 5
    assert O.code_ip(q, code, 0.5, mu, 4) == np.float32(1.0 - 0.5 * 3.0)
    code[1] = 1 << 4; code[0] = -1
    assert O.code_ip(q, code, 0.5, mu, 4) == np.float32(1.0 - 0.5 * -3.0)


def test_code_estimate_lane_layout():
    """team 2: lane 0 owns words 0 and 2, lane 1 owns word 1.  With 2^24 in
    word 0 and -2^24 in word 2 cancelling in lane 0, the two 1s of lane 1
    survive; summed in dimension order they would be absorbed.  sum(q) uses
    64 partials (t = l, l + 64, ...): 2^24 and -2^24 meet in partial 0."""
    q = np.zeros(96, np.float32)
    q[0], q[64], q[32], q[33] = 2.0 ** 24, -(2.0 ** 24), 1.0, 1.0
    mu = np.zeros(96, np.float32)
    code = np.array([1, 3, 1], np.int32)          # bits at dims 0, 32, 33, 64
    qmu, qsum = O.code_sums(q, mu)
    assert qsum == np.float32(2.0) and qmu == np.float32(0.0)
    # acc = 2 (lane order), est = 1 - (1 * (2 * 2 - 2) + 0) = -1
    assert O.code_ip(q, code, 1.0, mu, 2) == np.float32(-1.0)


def _star_case():
    """Seed 0 with neighbours 1..5; q = e_0.  Codes put 1 and 2 at estimate 0.5
    and 3, 4, 5 at 1.5; the stop line after init is d(seed) = 0.5."""
    d = 32
    X = np.zeros((6, d), np.float32)
    X[0, 0], X[1, 0], X[2, 0], X[3, 0], X[4, 0], X[5, 0] = 0.5, 0.9, 0.8, 0.95, 0.97, 0.99
    X[:, 1] = np.sqrt(1.0 - X[:, 0] ** 2)
    G = np.full((6, 8), -1, np.int32)
    G[0, :5] = [1, 2, 3, 4, 5]
    q = np.zeros(d, np.float32); q[0] = 1.0
    codes = np.zeros((6, 1), np.int32)
    codes[[1, 2], 0] = 1                           # bit 0 set: estimate 1 - 0.5 = 0.5
    alpha = np.full(6, 0.5, np.float32)
    mu = np.zeros(d, np.float32)
    return X, G, q, (codes, alpha, mu, 0.1)


def test_code_filter_skip_semantics():
    """One expansion: 3, 4 and 5 estimate beyond 0.5 + 0.1 and are skipped --
    their rows are not read and [3] counts 3.  They stay candidates at
    FLT_MAX and pass the filter (the queue is not full, so its worst is
    FLT_MAX: [8] counts 5), but the queue's empty slots are (FLT_MAX, -1) and
    win that tie in the merge, so they never enter."""
    X, G, q, codes = _star_case()
    br = O.init_branch(X, q, [0], L=8, H=64, B=4, D=8, metric=O.METRIC_IP, team=4)
    O.advance_branch(X, G, q, br, 1, 4, metric=O.METRIC_IP, team=4, stop_eps=0.0, kstop=1,
                     codes=codes)
    d1 = O.team_distance(q, X, 1, O.METRIC_IP, 4)
    d2 = O.team_distance(q, X, 2, O.METRIC_IP, 4)
    d0 = O.team_distance(q, X, 0, O.METRIC_IP, 4)
    assert list(br.ids) == [1, 2, 0, -1, -1, -1, -1, -1]
    assert list(br.dist[:3]) == [d1, d2, d0] and (br.dist[3:] == F32MAX).all()
    assert list(br.expanded) == [0, 0, 1, 1, 1, 1, 1, 1]
    assert br.counters[3] == 3 and br.counters[1] == 3 and br.counters[8] == 5
    # without codes every neighbour is scored and [3] stays 0
    br2 = O.init_branch(X, q, [0], L=8, H=64, B=4, D=8, metric=O.METRIC_IP, team=4)
    O.advance_branch(X, G, q, br2, 1, 4, metric=O.METRIC_IP, team=4, stop_eps=0.0, kstop=1)
    assert br2.counters[3] == 0 and br2.counters[1] == 6


def test_code_filter_is_inert_with_a_huge_margin():
    X, G = gaussian(1500, 64, 31, True), None
    from test_oracle_helpers import knn_graph
    G = knn_graph(X, 24, 0)
    codes, alpha, mu = O.build_codes(X)
    Qv = gaussian(6, 64, 32, True)
    for qi in range(6):
        a = O.run(X, G, Qv[qi], [qi * 7], L=16, B=20, team=16, stop_eps=0.1, kstop=10)
        br = O.init_branch(X, Qv[qi], [qi * 7], L=16, B=20, D=24, team=16)
        O.advance_branch(X, G, Qv[qi], br, 20, 20, team=16, stop_eps=0.1, kstop=10,
                         codes=(codes, alpha, mu, 1e30))
        assert np.array_equal(a.ids, br.ids) and a.dist.tobytes() == br.dist.tobytes()
        assert np.array_equal(a.counters, br.counters)


# -- the offline builder's extras (offline/build_graph.py) --------------------
@pytest.mark.parametrize("tag,metric", [("ip", O.METRIC_IP), ("l2", O.METRIC_L2)])
def test_offline_extras_match_reference(tag, metric):
    """candidates_from_graph, mutual_rank and fill_degree (all three rules)
    against the reference's CPU-torch offline/build_graph.py on its own
    graphs (tests/golden/refbuild_extras.npz): identical."""
    g = golden("refbuild_extras.npz")
    X = regen(800, 24, 23 if tag == "ip" else 24, tag == "ip", g[f"{tag}_X_sha"])
    cand = g[f"{tag}_cand"].astype(np.int32)
    assert np.array_equal(O.mutual_rank(cand, 8), g[f"{tag}_prot"])
    ci, cd = O.candidates_from_graph(X, g[f"{tag}_R"].astype(np.int32), 12, metric, nthreads=4)
    assert np.array_equal(ci, g[f"{tag}_cg"].astype(np.int32))
    assert np.allclose(cd, g[f"{tag}_cgd"], rtol=1e-5, atol=1e-5)
    for rule in ("near", "far", "bridge"):
        f = O.fill_degree(g[f"{tag}_Gp24"].astype(np.int32), cand, rule)
        assert np.array_equal(f, g[f"{tag}_fill_{rule}"].astype(np.int32)), rule


@pytest.mark.parametrize("tag", ["ip", "l2"])
def test_enforce_min_in_against_reference(tag):
    """enforce_min_in: where no target receives two offers in one column the
    rule is deterministic and the oracle equals the reference (ip here);
    otherwise the reference's winner follows torch's unstable argsort, so the
    check is the rule's invariants -- edge count and first slots unchanged,
    the floor met as the reference meets it -- and agreement on most rows."""
    g = golden("refbuild_extras.npz")
    R = g[f"{tag}_R"].astype(np.int32); want = g[f"{tag}_Gmin"].astype(np.int32)
    cand = g[f"{tag}_cand"].astype(np.int32)
    got = O.enforce_min_in(R, cand, 8, 4)
    indeg = lambda G: np.bincount(G[G >= 0].astype(np.int64), minlength=G.shape[0])  # noqa: E731
    assert (got >= 0).sum() == (R >= 0).sum() == (want >= 0).sum()
    assert np.array_equal(got[:, 0], R[:, 0])
    assert (indeg(got) < 8).sum() == (indeg(want) < 8).sum() == 0
    rows = (got == want).all(1).mean()
    if tag == "ip":
        assert rows == 1.0
    else:
        assert rows > 0.6, rows


def test_fill_rules_closed_forms():
    """near fills the empty slots with the first free candidates in column
    order, far with the last; a full graph is unchanged; bridge never adds a
    candidate that is already two hops away."""
    rng = np.random.default_rng(4)
    n, W, C = 50, 6, 12
    cand = np.stack([rng.permutation(n)[:C] for _ in range(n)]).astype(np.int32)
    G = np.full((n, W), -1, np.int32)
    G[:, 0] = cand[:, 0]
    near = O.fill_degree(G, cand, "near", chunk=7)
    far = O.fill_degree(G, cand, "far", chunk=7)
    for u in range(n):
        free = [c for c in cand[u] if c != u and c != G[u, 0]]
        assert list(near[u, 1:]) == free[:W - 1]
        assert list(far[u, 1:]) == free[::-1][:W - 1]
    assert np.array_equal(O.fill_degree(near, cand, "near"), near)
    br = O.fill_degree(G, cand, "bridge", chunk=n)
    for u in range(n):
        two = set(G[G[u, 0]]) if G[u, 0] >= 0 else set()
        assert not (set(br[u, 1:]) - {-1}) & two


# -- stall and crowd retirement (local_search.cu:659-682): hand cases whose
#    counts follow from the rule alone (stall_case / crowd_case)

@pytest.mark.parametrize("patience", [1, 2, 4, 6])
def test_stall_stops_after_patience_expansions_without_progress(patience):
    """s_best_k starts at FLT_MAX each call: the first expansion moves it to 0
    and resets the count, each later one adds 1; the branch stops when the
    count reaches the patience, so it expands exactly patience + 1 nodes and
    sets counter 6."""
    X, G, q = stall_case()
    br = O.init_branch(X, q, [0], L=16, B=64, D=8, metric=O.METRIC_L2, team=4)
    O.advance_branch(X, G, q, br, 64, 64, metric=O.METRIC_L2, team=4, stop_eps=-1.0, kstop=1,
                     stall_patience=patience)
    assert br.counters[0] == patience + 1
    assert br.counters[6] == 1
    # patience 0 disables the rule: the branch runs until its queue is spent
    br0 = O.init_branch(X, q, [0], L=16, B=64, D=8, metric=O.METRIC_L2, team=4)
    O.advance_branch(X, G, q, br0, 64, 64, metric=O.METRIC_L2, team=4, stop_eps=-1.0, kstop=1)
    assert br0.counters[0] == 9 and br0.counters[6] == 0


def test_crowd_retires_a_lineage_after_two_covered_expansions():
    """crowd_frac = 1: expansion 1 (the seed) sees four new nodes; expansions
    2 and 3 see only covered ones, so after the third the seed's lineage is
    retired (counter 7) and, every queued node being of that lineage, the
    next pick finds nothing (counter 3)."""
    X, G, q = crowd_case()
    br = O.init_branch(X, q, [0], L=16, B=64, D=8, metric=O.METRIC_L2, team=4)
    O.advance_branch(X, G, q, br, 64, 64, metric=O.METRIC_L2, team=4, stop_eps=-1.0, kstop=10,
                     crowd_frac=1.0)
    assert br.counters[0] == 3
    assert br.counters[7] == 1
    assert br.counters[3] == 1
    # a fraction no expansion reaches leaves the lineage alone: all 5 nodes expand
    br2 = O.init_branch(X, q, [0], L=16, B=64, D=8, metric=O.METRIC_L2, team=4)
    O.advance_branch(X, G, q, br2, 64, 64, metric=O.METRIC_L2, team=4, stop_eps=-1.0, kstop=10,
                     crowd_frac=1.5)
    assert br2.counters[0] == 5 and br2.counters[7] == 0


# -- the tie rules the parity tests use -----------------------------------------
def test_tie_rules_catch_planted_differences():
    """The comparators the parity tests hold the GPU to (tests/
    test_oracle_helpers.py) accept only differences at ties: a swap of two
    entries at distinct distances, a dropped neighbour, or a prune at
    another alpha (planted on the CPU, in the oracle's outputs) is reported;
    the same lists, or a swap inside a tie, are not."""
    from test_oracle_helpers import untied_graph_rows, untied_prune_rows, untied_rows
    g = golden("refbuild_small.npz")
    X = g["l2_X"]
    rc = g["l2_cand"].astype(np.int32); rd = g["l2_cdist"]
    assert untied_rows(rc, rc, rd, rd) == []
    swapped = rc.copy()
    swapped[5, [3, 4]] = swapped[5, [4, 3]]
    assert untied_rows(swapped, rc, rd, rd) == [5]                 # distinct distances
    tied_d = rd.copy()
    tied_d[5, 4] = tied_d[5, 3]
    assert untied_rows(swapped, rc, tied_d, tied_d) == []          # a tie: either order
    Gp = O.robust_prune(X, rc, rd, 16, 1.2, O.METRIC_L2, nthreads=2)
    assert untied_prune_rows(Gp, Gp, X, rc, rd, 16, 1.2, 1) == []
    other = O.robust_prune(X, rc, rd, 16, 1.25, O.METRIC_L2, nthreads=2)
    differ = int((other != Gp).any(1).sum())
    assert differ > 100
    assert len(untied_prune_rows(other, Gp, X, rc, rd, 16, 1.2, 1)) > 0.9 * differ
    dropped = Gp.copy()
    dropped[7, 0] = -1
    assert untied_graph_rows(dropped, Gp, X, 1) == [7]
