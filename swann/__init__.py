"""`import swann` served by swann_amd, the MI355X (gfx950) implementation of
SWANN's search and graph build: the reference's public names
(swann/__init__.py:13-16) and its module names -- `swann._engine`,
`swann._select`, `swann.build`, `swann.index` -- resolve to swann_amd's
objects and modules themselves, not to copies.

    import swann
    index = swann.Index.build(X, metric="ip")
    ids, dist = index.search(Q, k=10)
"""
import importlib
import sys

from swann_amd import Index, SearchConfig, __version__, overflow_guard  # noqa: F401

__all__ = ["Index", "SearchConfig", "overflow_guard"]

# `import swann._engine as E`, `from swann.build import build_graph`, ...: the
# import system finds these entries before it looks for files.
for _name in ("_engine", "_select", "build", "index", "codes", "corpus", "offline"):
    _module = importlib.import_module(f"swann_amd.{_name}")
    sys.modules[f"{__name__}.{_name}"] = _module
    globals()[_name] = _module
del _name, _module
