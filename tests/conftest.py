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


def norm_spread(X, sigma, seed):
    """Rows scaled by exp(sigma * N(0,1)) in float64, then cast
    (tests/golden/make_golden.py's recipe for the degree-96 ip corpus)."""
    s = np.exp(sigma * np.random.default_rng(seed).standard_normal((X.shape[0], 1)))
    return np.ascontiguousarray((X.astype(np.float64) * s).astype(np.float32))


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


def deg96_corpus(tag, g):
    """The degree-96 golden's corpus (tests/golden/refbuild_deg96.npz):
    l2 is 2,000 x 128 N(0,1); ip is 2,000 x 256 unit rows scaled by
    exp(0.2 N(0,1))."""
    if tag == "l2":
        X = gaussian(2000, 128, 961, False)
    else:
        X = norm_spread(gaussian(2000, 256, 962, True), 0.2, 963)
    if sha(X) != str(g[f"{tag}_X_sha"]):
        pytest.skip("regenerated inputs differ from the golden inputs on this platform")
    return X


@pytest.fixture
def opt():
    """Set library options (swann_set_option) for one test; every option is
    back at its default afterwards."""
    from swann_amd import _lib

    def set_(**values):
        for k, v in values.items():
            _lib.set_option(k, v)
    yield set_
    _lib.lib().swann_reset_options()
