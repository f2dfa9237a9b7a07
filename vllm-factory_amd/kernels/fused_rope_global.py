"""RoPE application (cos/sin table form) on gfx950.

Drop-in for kernels/fused_rope_global.py:108-166: `fused_rope_apply(x, cos, sin)`
and `fused_rope_global_apply(q, k, cos, sin)`, non-interleaved halves:
out[d] = x[d] cos[d] - x[d+D/2] sin[d] (d < D/2), x[d] cos[d] + x[d-D/2] sin[d]
otherwise. Inputs [B,S,H,D] (no copy when the last dim is contiguous with
16-byte aligned rows); cos/sin [B,S,D], [B,1,S,D] or [S,D], in the input's
dtype or fp32 (used at fp32, as the reference's kernel promotes mixed
operands; other dtypes are widened to fp32 exactly). Returns new contiguous
tensors of the input's dtype. q and k are rotated in one launch that loads
each cos/sin value once per thread for several heads; head dims that launch
cannot take (D not a multiple of 16 for 16-bit inputs, of 8 for fp32, e.g.
D = 36, 40 or 72) go through the general per-element kernel, one launch per
tensor, with the same arithmetic. Any even D works, as in the reference.
"""
from __future__ import annotations

import torch

from . import _lib


def _cos_sin(t: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    if t.dim() == 4:  # [B, 1, S, D]
        t = t.squeeze(1)
    if t.dim() == 2:  # [S, D]
        t = t.unsqueeze(0)
    if t.dtype not in (x.dtype, torch.float32):
        t = t.float()
    return _lib.rows_aligned(t)


def _rope_any(dev, x: torch.Tensor, c: torch.Tensor, s: torch.Tensor) -> torch.Tensor:
    """One tensor through vfk_rope_fwd (any strides, any even D)."""
    out = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    _lib.on_device("vfk_rope_fwd", dev, _lib.ref(_lib.desc(x)), _lib.ref(_lib.desc(c)),
                   _lib.ref(_lib.desc(s)), _lib.ref(_lib.desc(out)))
    return out


def _rope(q: torch.Tensor, k, cos: torch.Tensor, sin: torch.Tensor):
    dev = _lib.require_gpu(q, k, cos, sin)
    for t in (q, k):
        if t is not None and t.dim() != 4:
            raise ValueError("q/k must be [B, S, H, D]")
    c = _cos_sin(cos, q)
    s = _cos_sin(sin, q)
    if c.dtype != s.dtype:
        c, s = c.float(), s.float()
    D = q.shape[-1]
    if D <= 0 or D % (2 * (16 // q.element_size())):
        # outside the one-launch kernel's chunking: per tensor, general kernel
        if D % 2:
            raise ValueError(f"head_dim must be even, got {D}")
        return _rope_any(dev, q, c, s), (_rope_any(dev, k, c, s) if k is not None else None)
    qq = _lib.rows_aligned(q)
    qo = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    kk = _lib.rows_aligned(k) if k is not None else None
    ko = torch.empty(k.shape, dtype=k.dtype, device=k.device) if k is not None else None
    _lib.on_device("vfk_rope_qk_fwd", dev, _lib.ref(_lib.desc(qq)), _lib.ref(_lib.desc(kk)),
                   _lib.ref(_lib.desc(c)), _lib.ref(_lib.desc(s)), _lib.ref(_lib.desc(qo)),
                   _lib.ref(_lib.desc(ko)))
    return qo, ko


def fused_rope_apply(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Apply RoPE to a single [B, S, H, D] tensor."""
    return _rope(x, None, cos, sin)[0]


def fused_rope_global_apply(q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor,
                            sin: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Apply RoPE (global) to query and key tensors, both in one launch."""
    if k.dtype != q.dtype:
        raise ValueError("q and k must share a dtype")
    return _rope(q, k, cos, sin)
