"""swann_select_nearest_noalloc (the library's fixed scratch instead of a
caller's workspace) against swann_select_nearest (caller's workspace): the
same indices and distance bits on two calls in a row, the second smaller and
on the split-K path, for both metrics; and a batch beyond the scratch is
refused before anything runs."""
import ctypes
import sys

import numpy as np
import pytest
import torch

from conftest import gaussian

pytestmark = pytest.mark.gpu

from swann_amd import _lib  # noqa: E402
from swann_amd._lib import call, ptr, stream_of  # noqa: E402

SCRATCH = 32 << 20          # SWANN_SELECT_SCRATCH_BYTES in include/swann_amd.h


def note(*a):
    print("[case]", *a, flush=True)
    sys.stdout.flush()


def both(Q, V, E, metric):
    nq, P = Q.shape[0], V.shape[0]
    dev = Q.device
    ws = torch.empty(int(_lib.lib().swann_select_workspace_size(nq, P)), dtype=torch.uint8,
                     device=dev)
    ai = torch.full((nq, E), -7, dtype=torch.int32, device=dev)
    ad = torch.full((nq, E), -7.0, dtype=torch.float32, device=dev)
    bi = torch.full((nq, E), -9, dtype=torch.int32, device=dev)
    bd = torch.full((nq, E), -9.0, dtype=torch.float32, device=dev)
    st = stream_of(dev)
    call("swann_select_nearest", ptr(Q), nq, Q.shape[1], ptr(V), P, E, metric, ptr(ai), ptr(ad),
         ptr(ws), st)
    call("swann_select_nearest_noalloc", ptr(Q), nq, Q.shape[1], ptr(V), P, E, metric, ptr(bi),
         ptr(bd), st)
    torch.cuda.synchronize()
    return ai.cpu().numpy(), ad.cpu().numpy(), bi.cpu().numpy(), bd.cpu().numpy()


@pytest.mark.parametrize("metric", [0, 1])
def test_noalloc_select_equals_the_workspace_select(metric):
    # first a large batch (one K pass, 4096-row catalogue), then a smaller one
    # whose grid is split over K: the second call reuses the first's scratch
    for nq, P, dim, E in ((1500, 4096, 128, 32), (24, 1000, 96, 16)):
        note("noalloc select", metric, nq, P, dim, E)
        need = int(_lib.lib().swann_select_workspace_size(nq, P))
        assert need <= SCRATCH
        Q = torch.from_numpy(gaussian(nq, dim, 7 + nq, metric == 0)).cuda()
        V = torch.from_numpy(gaussian(P, dim, 8 + P, metric == 0)).cuda()
        ai, ad, bi, bd = both(Q, V, E, metric)
        assert np.array_equal(ai, bi)
        assert ad.tobytes() == bd.tobytes()
        assert (ai >= 0).all() and (np.diff(ad, axis=1) >= 0).all()


def test_noalloc_select_refuses_a_batch_beyond_its_scratch():
    L = _lib.lib()
    nq, P = 4096, 4096                                    # 64 MiB of distances
    assert L.swann_select_workspace_size(nq, P) > SCRATCH
    rc = L.swann_select_nearest_noalloc(None, nq, 64, None, P, 8, 0, None, None, None)
    assert rc == -1
    msg = L.swann_last_error().decode()
    assert "scratch" in msg and str(SCRATCH) in msg
