import hashlib
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
GOLDEN = ROOT / "tests" / "golden"
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP C-ABI)")


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def gaussian(n, d, seed, normalise):
    """The golden generator's input recipe (tests/golden/make_golden.py)."""
    X = np.random.default_rng(seed).standard_normal((n, d), dtype=np.float32)
    if normalise:
        X64 = X.astype(np.float64)
        X = (X64 / np.sqrt((X64 * X64).sum(1, keepdims=True))).astype(np.float32)
    return np.ascontiguousarray(X)


def golden(name):
    path = GOLDEN / name
    if not path.exists():
        pytest.skip(f"golden file {name} missing")
    return np.load(path, allow_pickle=False)


def regen(n, d, seed, normalise, want_sha):
    X = gaussian(n, d, seed, normalise)
    if sha(X) != str(want_sha):
        pytest.skip("regenerated inputs differ from the golden inputs on this platform")
    return X
