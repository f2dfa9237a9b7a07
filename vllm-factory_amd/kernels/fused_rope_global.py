"""RoPE application (cos/sin table form) on gfx950.

Drop-in for kernels/fused_rope_global.py:108-166: `fused_rope_apply(x, cos, sin)`
and `fused_rope_global_apply(q, k, cos, sin)`, non-interleaved halves:
out[d] = x[d] cos[d] - x[d+D/2] sin[d] (d < D/2), x[d] cos[d] + x[d-D/2] sin[d]
otherwise. Inputs [B,S,H,D] with any strides (no contiguous copy is made when
the last dim is contiguous); cos/sin [B,S,D] or [B,1,S,D]. Returns new
contiguous tensors.
"""
from __future__ import annotations

import torch

from . import _lib


def _cos_sin(t: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    if t.dim() == 4:  # [B, 1, S, D]
        t = t.squeeze(1)
    if t.dim() == 2:  # [S, D]
        t = t.unsqueeze(0)
    if t.dtype != x.dtype:
        t = t.to(x.dtype)
    return _lib.rows_aligned(t)


def fused_rope_apply(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Apply RoPE to a single [B, S, H, D] tensor."""
    dev = _lib.require_gpu(x, cos, sin)
    if x.dim() != 4:
        raise ValueError("x must be [B, S, H, D]")
    c = _cos_sin(cos, x)
    s = _cos_sin(sin, x)
    xx = x if x.stride(-1) == 1 else x.contiguous()
    out = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    _lib.on_device("vfk_rope_fwd", dev, _lib.ref(_lib.desc(xx)), _lib.ref(_lib.desc(c)),
                   _lib.ref(_lib.desc(s)), _lib.ref(_lib.desc(out)))
    return out


def fused_rope_global_apply(q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor,
                            sin: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Apply RoPE (global) to query and key tensors."""
    return fused_rope_apply(q, cos, sin), fused_rope_apply(k, cos, sin)
