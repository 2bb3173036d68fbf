"""Sign codes for the search's pre-filter.

The reference consumes (codes, alpha, mu, margin) in `advance`
(swann/_engine.py:281-317, swann/csrc/local_search.cu:205-243) and reads them
from codes_<name>.npy, alpha_<name>.npy and mu_<name>.npy (`load_codes`,
swann/_engine.py:320-337); the script that writes them is not part of it.
`build_codes` makes them on the GPU from the definition the consumer's
estimator assumes, and `save_codes` writes the files `load_codes` reads.
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import torch

from ._lib import call, lib, ptr, stream_of

_DTYPES = {torch.float32: 0, torch.float16: 1}


def build_codes(X: torch.Tensor, mu: torch.Tensor | None = None):
    """(codes [n, ceil(d/32)] int32, alpha [n] fp32, mu [d] fp32) for a cuda
    fp32/fp16 corpus: mu is the column mean (or the given one), bit b of word
    w is set where x[32w + b] > mu[32w + b], alpha = mean |x - mu| per row."""
    if not (X.is_cuda and X.dim() == 2 and X.dtype in _DTYPES):
        raise RuntimeError("X: cuda float32/float16 [n, d]")
    X = X.contiguous()
    n, d = X.shape
    dev = X.device
    codes = torch.empty((n, (d + 31) // 32), dtype=torch.int32, device=dev)
    alpha = torch.empty((n,), dtype=torch.float32, device=dev)
    mu_out = torch.empty((d,), dtype=torch.float32, device=dev)
    ws = None
    if mu is not None:
        mu = mu.to(device=dev, dtype=torch.float32).contiguous()
        if mu.numel() != d:
            raise RuntimeError("mu must have one entry per dimension")
    else:
        ws = torch.empty((int(lib().swann_codes_workspace_size(n, d)),), dtype=torch.uint8,
                         device=dev)
    with torch.cuda.device(dev):
        call("swann_build_codes", ptr(X), _DTYPES[X.dtype], n, d, ptr(mu), ptr(codes),
             ptr(alpha), ptr(mu_out), ptr(ws), stream_of(dev))
    return codes, alpha, mu_out


def save_codes(data, codes, alpha, mu, name: str = "1bit") -> None:
    """Write codes_<name>.npy, alpha_<name>.npy and mu_<name>.npy under `data`."""
    d = Path(data)
    d.mkdir(parents=True, exist_ok=True)
    np.save(d / f"codes_{name}.npy", codes.cpu().numpy().astype(np.int32))
    np.save(d / f"alpha_{name}.npy", alpha.cpu().numpy().astype(np.float32))
    np.save(d / f"mu_{name}.npy", mu.cpu().numpy().astype(np.float32))
