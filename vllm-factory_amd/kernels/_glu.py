"""Shared launcher for the gated-activation and residual kernels."""
from __future__ import annotations

import torch

from . import _lib


def flat2d(t: torch.Tensor) -> torch.Tensor:
    """[..., n] -> [rows, n] as a view when strides allow it (chunk() halves do)."""
    n = t.shape[-1]
    t2 = t.reshape(-1, n) if t.dim() != 2 else t
    if t2.stride(-1) != 1:
        t2 = t2.contiguous()
    return t2


def binary(entry: str, act: int, a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    dev = _lib.require_gpu(a, b)
    if a.shape != b.shape:
        raise AssertionError("operands must have identical shapes")
    if a.dtype != b.dtype:
        raise ValueError("operands must share a dtype")
    a2, b2 = flat2d(a), flat2d(b)
    out = torch.empty(a2.shape, dtype=a.dtype, device=a.device)
    if out.numel():
        if entry == "vfk_glu_fwd":
            _lib.on_device(entry, dev, int(act), _lib.ref(_lib.desc(a2)),
                           _lib.ref(_lib.desc(b2)), _lib.ref(_lib.desc(out)))
        else:
            _lib.on_device(entry, dev, _lib.ref(_lib.desc(a2)), _lib.ref(_lib.desc(b2)),
                           _lib.ref(_lib.desc(out)))
    return out.view(a.shape)
