"""ctypes binding of libswann_amd.so (the C ABI declared in include/swann_amd.h).

There is no fallback: if the library is not built, or there is no GPU, the
calls raise.  Build it with `python -m swann_amd._build`.
"""
from __future__ import annotations

import contextlib
import ctypes
import threading
from pathlib import Path

# The in-tree build (swann_amd/_build.py writes it there).
LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libswann_amd.so"

P = ctypes.c_void_p
I = ctypes.c_int
I64 = ctypes.c_int64
F = ctypes.c_float

# name -> (restype, argtypes); must match include/swann_amd.h
PROTOTYPES = {
    "swann_last_error": (ctypes.c_char_p, []),
    "swann_version": (ctypes.c_char_p, []),
    "swann_device_count": (I, []),
    "swann_set_option": (I, [ctypes.c_char_p, I]),
    "swann_get_option": (I, [ctypes.c_char_p, ctypes.POINTER(I)]),
    "swann_reset_options": (I, []),
    "swann_validate_init": (I, [I64, I, I, I64, I, I, I, I, I, I, I]),
    "swann_validate_advance": (I, [I64, I, I, I, I64, I, I, I, I, I, I, I, I, I64, I]),
    "swann_init_states": (I, [P, I, I64, I, P, I64, P, I, I, P, P, P, P, I, P, I, P,
                              I, I, P, P, I, P, P]),
    "swann_advance": (I, [P, I, I64, I, P, I, P, I64, I, P, P, P, P, I, P, I, P,
                          I, I, I, I, I, I, F, I, P, P, I, P, I, I, F, P, I64,
                          P, I, P, P, F, P]),
    "swann_merge_branches": (I, [P, P, I64, I, I, I, P, P, P]),
    "swann_merge_branches_strided": (I, [P, P, I64, I, I, I64, I, P, P, P]),
    "swann_overflow_async": (I, [P, I64, P, P]),
    "swann_select_workspace_size": (I64, [I64, I64]),
    "swann_select_nearest": (I, [P, I64, I, P, I64, I, I, P, P, P, P]),
    "swann_select_nearest_noalloc": (I, [P, I64, I, P, I64, I, I, P, P, P]),
    "swann_mfma_probe_flop": (I64, [I, I]),
    "swann_mfma_probe": (I, [I, I, P, P]),
    "swann_sweep_workspace_size": (I64, [I64, I, I, I]),
    "swann_build_sweep": (I, [P, I, I64, I, I, I, P, P, P, P]),
    "swann_sweep_tiles_scored": (I64, []),
    "swann_sweep_dense_panels": (I64, []),
    "swann_prune_workspace_size": (I64, [I64, I, I]),
    "swann_build_prune": (I, [P, I, I64, I, I, P, P, I, I, F, P, P, P, P, P]),
    "swann_reverse_workspace_size": (I64, [I64, I, I]),
    "swann_build_reverse": (I, [P, I, I64, I, I, P, I, F, I, P, P, P, P]),
    "swann_codes_workspace_size": (I64, [I64, I]),
    "swann_build_codes": (I, [P, I, I64, I, P, P, P, P, P, P]),
    "swann_candidates_from_graph": (I, [P, I, I64, I, I, P, I, I, P, P, P]),
    "swann_mutual_rank": (I, [P, I64, I, I, P, P]),
    "swann_fill_workspace_size": (I64, [I64, I, I]),
    "swann_fill_degree": (I, [P, I64, I, P, I, I, I, P, P, P]),
    "swann_min_in_workspace_size": (I64, [I64]),
    "swann_enforce_min_in": (I, [P, I64, I, P, I, I, I, P, P]),
}

_lib = None
_lock = threading.Lock()


class SwannError(RuntimeError):
    """A call into libswann_amd failed; the message is the library's own."""


def load(path):
    """Open a build of the library at `path` and declare its prototypes."""
    path = Path(path)
    if not path.exists():
        raise SwannError(f"{path} is not built; run `python -m swann_amd._build` "
                         "(there is no CPU fallback)")
    L = ctypes.CDLL(str(path))
    for name, (res, args) in PROTOTYPES.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    return L


def lib():
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                _lib = load(LIB_PATH)
    return _lib


def call(name, *args):
    """Call an int-returning entry point and raise on a nonzero code."""
    L = lib()
    rc = getattr(L, name)(*args)
    if rc != 0:
        msg = L.swann_last_error().decode(errors="replace")
        raise SwannError(msg or f"{name} failed with code {rc}")
    return rc


def ptr(t):
    """Device (or host) address of a tensor, or None for an absent one."""
    if t is None or t.numel() == 0:
        return None
    return ctypes.c_void_p(t.data_ptr())


def stream_of(device):
    import torch
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def set_option(name: str, value: int) -> None:
    """Select an alternative code path of the same computation (the list and
    the values are in include/swann_amd.h: swann_set_option).  For tests and
    diagnosis; every option defaults to the production path."""
    call("swann_set_option", name.encode(), int(value))


def get_option(name: str) -> int:
    v = I(0)
    call("swann_get_option", name.encode(), ctypes.byref(v))
    return int(v.value)


@contextlib.contextmanager
def options(**values):
    """Set options for the body of a `with`, restoring the earlier values."""
    old = {k: get_option(k) for k in values}
    try:
        for k, v in values.items():
            set_option(k, v)
        yield
    finally:
        for k, v in old.items():
            set_option(k, v)
