"""Host-side checks that need no GPU: the C ABI loads and exports what its
header declares, argument validation refuses what the reference refuses
(swann/csrc/local_search.cu:726-841), the sizing closed forms, the tensor
merge against the oracle, and the product refusing to run without a GPU."""
import re
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle as O
from conftest import ROOT

from swann_amd import _engine as E
from swann_amd import _lib
from swann_amd.index import SearchConfig

HEADER = ROOT / "include" / "swann_amd.h"


def declared_symbols():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:const char\*|int64_t|int)\s+(swann_\w+)\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    L = _lib.lib()
    names = declared_symbols()
    assert len(names) >= 15, names
    for name in names:
        assert hasattr(L, name), f"{name} declared in swann_amd.h but not exported"
        assert name in _lib.PROTOTYPES, f"{name} has no ctypes prototype"
    assert set(_lib.PROTOTYPES) == set(names)
    assert b"gfx950" in L.swann_version()


def _vinit(**kw):
    a = dict(n=1000, dim=128, x_dtype=0, Q=4, J=2, V=1, L=16, H=1024, metric=0, team_size=16, Hc=0)
    a.update(kw)
    return _lib.lib().swann_validate_init(*a.values())


def _vadv(**kw):
    a = dict(n=1000, dim=128, x_dtype=0, D=32, Q=4, J=2, L=16, H=1024, metric=0, team_size=16,
             policy=0, V=1, Hc=0, nactive=0, cwords=0)
    a.update(kw)
    return _lib.lib().swann_validate_advance(*a.values())


def _err():
    return _lib.lib().swann_last_error().decode()


def test_validation_accepts_the_reference_configs():
    assert _vinit() == 0 and _vadv() == 0
    for team in (4, 8, 16, 32, 64):
        assert _vinit(team_size=team) == 0 and _vadv(team_size=team) == 0
    # C3/C4 shapes: d=1536 and 4096 fp16, D=64, L=12
    assert _vadv(dim=1536, x_dtype=1, D=64, L=12, Q=10000, J=32, H=1, Hc=131072) == 0
    assert _vadv(dim=4096, x_dtype=1, D=64, L=12, Q=512, J=128, H=1, Hc=524288) == 0
    # no 65535-query cap
    assert _vinit(Q=70000, J=32) == 0 and _vadv(Q=70000, J=32) == 0
    # sign codes (ip): one bit per dimension, at least ceil(dim / 32) words
    assert _vadv(cwords=4) == 0 and _vadv(dim=1536, x_dtype=1, D=64, cwords=48) == 0


@pytest.mark.parametrize("kw,msg", [
    (dict(team_size=3), "team_size"),
    (dict(L=513), "L"),
    (dict(H=1000), "power of two"),
    (dict(Hc=1000), "power of two"),
    (dict(V=129), "seeds per branch"),
    (dict(metric=2), "metric"),
    (dict(x_dtype=5), "float32 or float16"),
    (dict(dim=40000), "LDS"),
])
def test_init_validation_refuses(kw, msg):
    assert _vinit(**kw) != 0
    assert msg in _err()


@pytest.mark.parametrize("kw,msg", [
    (dict(D=129), "MAXD"),
    (dict(L=600), "MAXL"),
    (dict(V=300), "uint8"),
    (dict(policy=7), "policy"),
    (dict(cwords=4, metric=1), "inner-product"),
    (dict(cwords=3), "code words do not cover"),
    (dict(cwords=-1), "cwords"),
    (dict(nactive=100), "active"),
    (dict(dim=20000), "LDS"),
])
def test_advance_validation_refuses(kw, msg):
    assert _vadv(**kw) != 0
    assert msg in _err()


def test_sizing_closed_forms():
    """_engine.py:66-77, :186-198 at the configs' shapes."""
    assert E.visited_size(64, 64) == 16384 and E.visited_size(64, 32) == 8192
    assert E.cache_size(8, 64, 32) == 16384          # C1
    assert E.cache_size(32, 64, 64) == 131072        # C2/C3
    assert E.cache_size(128, 64, 64) == 524288       # C4, J=128
    assert E.cache_size(10_000, 64, 64) == 1 << 20   # the cap
    assert E.cache_size(8, 64, 32) == O.cache_size(8, 64, 32)
    assert E.visited_size(12, 32) == O.visited_size(12, 32)


def test_search_config_defaults():
    c = SearchConfig()
    assert (c.branches, c.queue, c.budget, c.stop_eps, c.team, c.k) == (32, 12, 64, 0.05, 16, 10)


def test_product_refuses_cpu_tensors():
    X = torch.zeros((10, 8))
    with pytest.raises(RuntimeError):
        E.init_states(X, X[:2].clone(), torch.zeros((2, 1), dtype=torch.int32), D=4)
    with pytest.raises(RuntimeError):
        E.merge_branches(torch.zeros((2, 3, 4), dtype=torch.int32), torch.zeros((2, 3, 4)), 4)
    from types import SimpleNamespace
    with pytest.raises(RuntimeError):
        E.merge_state(SimpleNamespace(ids=torch.zeros((2, 3, 4), dtype=torch.int32),
                                      dist=torch.zeros((2, 3, 4))), 4)


def test_no_oracle_in_the_product():
    """The product package never imports the oracle."""
    for f in (ROOT / "swann_amd").rglob("*.py"):
        text = f.read_text()
        assert "import oracle" not in text and "from oracle" not in text, f


def test_interleaved_table_must_be_8_byte_aligned():
    """An interleaved (id, d) table is probed as 64-bit words: a start that is
    only 4-byte aligned is refused before anything runs (Q = 0: no launch, no
    GPU needed); an aligned one, and separate arrays, pass."""
    L = _lib.lib()

    def init(cid, cdd):
        return L.swann_init_states(None, 0, 1000, 128, None, 0, None, 2, 1, None, None, None,
                                   None, 16, None, 1, None, 0, 16, cid, cdd, 1024, None, None)

    def adv(cid, cdd):
        return L.swann_advance(None, 0, 1000, 128, None, 32, None, 0, 2, None, None, None, None,
                               16, None, 1, None, 0, 16, 4, 4, 0, 1, 0.0, 10, cid, cdd, 1024,
                               None, 0, 0, 0.0, None, 0, None, 0, None, None, 0.0, None)

    base = 0x10000
    for fn in (init, adv):
        assert fn(base + 4, base + 8) != 0 and "8-byte aligned" in _err()
        assert fn(base, base + 4) == 0                       # aligned pairs
        assert fn(base + 4, base + 0x8000) == 0              # separate arrays


def test_swann_is_the_drop_in_name():
    """`import swann` gives the reference's public names and module paths
    (swann/__init__.py:13-16), bound to this implementation's objects."""
    import swann
    import swann_amd
    assert swann.Index is swann_amd.Index and swann.SearchConfig is swann_amd.SearchConfig
    assert swann.overflow_guard is swann_amd.overflow_guard
    assert sorted(swann.__all__) == ["Index", "SearchConfig", "overflow_guard"]
    import swann._engine as E2
    from swann.build import build_graph, knn_candidates  # noqa: F401
    from swann._select import select_nearest  # noqa: F401
    from swann.index import Index
    assert E2 is E and Index is swann_amd.Index
    assert E2.cache_size(32, 64, 64) == 131072


def test_direct_loads_are_padded_for_their_sgpr_operands(tmp_path):
    """The sweep's direct global->LDS loads are inline assembly, whose
    operands the compiler's hazard padding does not see.  A base address
    restored into SGPRs by v_readlane (a VALU write) must be 5 wait states
    old when a VMEM instruction reads it; with one, the load read a stale
    base and faulted.  Compile the sweep for gfx950 and check every direct
    load for a VALU write of its base within the last 5 wait states."""
    import shutil
    import subprocess
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(hipcc).exists():
        pytest.skip("hipcc not available")
    src = ROOT / "swann_amd" / "csrc" / "sweep_mfma.hip"
    out = tmp_path / "sweep.s"
    subprocess.run([hipcc, "-O3", "-std=c++17", "--offload-arch=gfx950", "--cuda-device-only",
                    "-S", "-ffp-contract=off", "-Xclang", "-target-feature", "-Xclang",
                    "-packed-fp32-ops", f"-I{ROOT / 'include'}",
                    f"-I{ROOT / 'swann_amd' / 'csrc'}", str(src), "-o", str(out)],
                   check=True, capture_output=True)

    def sregs(tok):
        m = re.match(r"s\[(\d+):(\d+)\]", tok)
        if m:
            return set(range(int(m.group(1)), int(m.group(2)) + 1))
        m = re.match(r"s(\d+)$", tok)
        return {int(m.group(1))} if m else set()

    lines = [ln.strip() for ln in out.read_text().splitlines()]
    loads, hazards = 0, []
    for i, ln in enumerate(lines):
        if not ln.startswith("global_load_lds"):
            continue
        loads += 1
        base = sregs(ln.split(",")[-1].strip())
        waits, j = 0, i - 1
        while j >= 0 and waits < 5:
            t = lines[j]
            j -= 1
            if not t or t.startswith((";", ".")) or t.endswith(":"):
                continue
            op = t.split()[0]
            if op == "s_nop":
                waits += int(t.split()[1], 0) + 1
                continue
            if op.startswith("v_") and len(t.split()) > 1 and sregs(t.split()[1].rstrip(",")) & base:
                hazards.append((i, t, ln))
            waits += 1
    assert loads > 0
    assert not hazards, hazards[:3]


def test_sym_panel_order_is_a_permutation(tmp_path):
    """A symmetric-sweep band launch gives workgroup b the row panel
    sym_panel(b, g, B); every panel of the launch must be taken exactly once,
    for every launch size up to 4,096 panels (n = 1M has 3,907) and band
    widths from 1 past the widest band.  The header is compiled as host code
    and run here, so the check is of the very function the kernel calls; it
    also checks the balance it is for: the XCDs (b % 8) get the same work to
    within two bands' tiles (one panel more or less, and the triangle's
    panels dealt round-robin), where equal contiguous runs of panels leave the
    last XCDs up to about T^2 / 2 tiles short for a triangle of T panels."""
    import shutil
    import subprocess
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not available")
    src = tmp_path / "perm.cpp"
    src.write_text(r'''
#include <cstdio>
#include <vector>
#include "panel_order.h"
int main() {
    long bad = 0, unbalanced = 0, pairs = 0;
    for (int g = 1; g <= 4096; ++g)
        for (int B = 1; B <= 1100; B += (B < 40 ? 1 : 37)) {
            std::vector<char> seen(g, 0);
            long work[8] = {0};
            for (int b = 0; b < g; ++b) {
                const int l = swann::sym_panel(b, g, B);
                if (l < 0 || l >= g || seen[l]) { ++bad; break; }
                seen[l] = 1;
                work[b & 7] += (B < g - l ? B : g - l);
            }
            long lo = work[0], hi = work[0];
            for (int x = 1; x < 8; ++x) { lo = work[x] < lo ? work[x] : lo; hi = work[x] > hi ? work[x] : hi; }
            if (hi - lo >= 2L * B) ++unbalanced;
            ++pairs;
        }
    printf("%ld %ld %ld\n", pairs, bad, unbalanced);
    return 0;
}
''')
    exe = tmp_path / "perm"
    subprocess.run([gxx, "-O2", "-std=c++17", f"-I{ROOT / 'swann_amd' / 'csrc'}", str(src),
                    "-o", str(exe)], check=True, capture_output=True)
    pairs, bad, unbalanced = map(int, subprocess.run([str(exe)], check=True, capture_output=True,
                                                     text=True).stdout.split())
    assert pairs > 200_000
    assert bad == 0
    assert unbalanced == 0


def test_options_are_a_closed_documented_list():
    """The library's code-path switches are options of the C ABI, each with
    its documented default and values; unknown names and values are refused,
    and the product reads no environment variable."""
    from swann_amd import _lib
    L = _lib.lib()
    L.swann_reset_options()
    want = {"search_block": 0, "prune_simt": 0, "prune_f32": 0, "sweep_sym": -1,
            "sweep_waves": 16, "sweep_rowscale": 0, "sweep_regstage": 0, "sweep_sym_fcap": 0,
            "sweep_noseed": 0, "sweep_order": 1, "sweep_repair_max": 4}
    header = (ROOT / "include" / "swann_amd.h").read_text()
    for name, default in want.items():
        assert _lib.get_option(name) == default, name
        assert f" *   {name} " in header, name
    with _lib.options(search_block=256, sweep_sym=0):
        assert _lib.get_option("search_block") == 256 and _lib.get_option("sweep_sym") == 0
    assert _lib.get_option("search_block") == 0 and _lib.get_option("sweep_sym") == -1
    with pytest.raises(_lib.SwannError, match="unknown option"):
        _lib.set_option("no_such_option", 1)
    with pytest.raises(_lib.SwannError, match="not one of its values"):
        _lib.set_option("search_block", 128)
    for src in (ROOT / "swann_amd" / "csrc").iterdir():
        assert "getenv" not in src.read_text(), src.name
    assert "os.environ" not in (ROOT / "swann_amd" / "_lib.py").read_text()
