"""swann_amd: SWANN's intra-query multi-branch graph search and exact-sweep
graph build, MI355X-native (gfx950 HIP kernels behind a C ABI).

A query is split into `branches` trajectories that advance at the same time
and share a per-query distance table, a bound on the answer, and node claims.

    import swann                  # or: import swann_amd as swann
    index = swann.Index.build(X, metric="ip")
    ids, dist = index.search(Q, k=10)
"""
from ._engine import overflow_guard
from .index import Index, SearchConfig

__all__ = ["Index", "SearchConfig", "overflow_guard"]
__version__ = "0.1.0"
