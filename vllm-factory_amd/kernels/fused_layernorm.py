"""LayerNorm on gfx950: one pass over HBM, fp32 statistics in registers.

Drop-in for kernels/fused_layernorm.py:109-274 (`FusedLayerNorm`, state-dict
compatible with nn.LayerNorm, and `fused_layernorm`). Adds
`fused_add_layernorm`, which folds the residual add that precedes every norm
in the encoders into the same pass.
"""
from __future__ import annotations

from typing import Optional

import torch

from . import _lib


def _as_2d(x: torch.Tensor, n: int) -> torch.Tensor:
    x2 = x.reshape(-1, n)
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    return x2


def _norm(x: torch.Tensor, n: int, weight: Optional[torch.Tensor], bias: Optional[torch.Tensor],
          eps: float, residual: Optional[torch.Tensor] = None, rms: bool = False,
          want_sum: bool = False):
    dev = _lib.require_gpu(x, weight, bias, residual)
    if x.shape[-1] != n:
        raise ValueError(f"last dim {x.shape[-1]} != normalized size {n}")
    x2 = _as_2d(x, n)
    y = torch.empty(x2.shape, dtype=x.dtype, device=x.device)
    r2 = _as_2d(residual, n) if residual is not None else None
    s2 = torch.empty_like(y) if (residual is not None and want_sum) else None
    w = weight.contiguous() if weight is not None else None
    b = bias.contiguous() if bias is not None else None
    if rms:
        _lib.on_device("vfk_rmsnorm_fwd", dev, _lib.ref(_lib.desc(x2)), _lib.ref(_lib.desc(r2)),
                       _lib.ref(_lib.desc(w)), float(eps), _lib.ref(_lib.desc(y)),
                       _lib.ref(_lib.desc(s2)))
    else:
        _lib.on_device("vfk_layernorm_fwd", dev, _lib.ref(_lib.desc(x2)), _lib.ref(_lib.desc(r2)),
                       _lib.ref(_lib.desc(w)), _lib.ref(_lib.desc(b)), float(eps),
                       _lib.ref(_lib.desc(y)), _lib.ref(_lib.desc(s2)))
    y = y.view(x.shape)
    if s2 is not None:
        return y, s2.view(x.shape)
    return y


class FusedLayerNorm(torch.nn.Module):
    """LayerNorm over the last dimension (parameters `weight`, `bias`)."""

    def __init__(self, normalized_shape, eps=1e-5, elementwise_affine=True, bias=True,
                 dtype=None, device=None):
        super().__init__()
        if isinstance(normalized_shape, int):
            normalized_shape = (normalized_shape,)
        self.normalized_shape = tuple(normalized_shape)
        if len(self.normalized_shape) != 1:
            raise NotImplementedError("FusedLayerNorm normalizes over the last dim only")
        self.eps = eps
        self.elementwise_affine = elementwise_affine
        if elementwise_affine:
            self.weight = torch.nn.Parameter(torch.ones(normalized_shape, dtype=dtype, device=device))
            if bias:
                self.bias = torch.nn.Parameter(torch.zeros(normalized_shape, dtype=dtype, device=device))
            else:
                self.register_parameter("bias", None)
        else:
            self.register_parameter("weight", None)
            self.register_parameter("bias", None)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return _norm(x, self.normalized_shape[0], self.weight, self.bias, self.eps)

    def forward_add(self, x: torch.Tensor, residual: torch.Tensor):
        """Returns (LayerNorm(x + residual), x + residual) in one pass."""
        return _norm(x, self.normalized_shape[0], self.weight, self.bias, self.eps,
                     residual=residual, want_sum=True)

    def extra_repr(self) -> str:
        return f"{self.normalized_shape}, eps={self.eps}, elementwise_affine={self.elementwise_affine}"


def fused_layernorm(x: torch.Tensor, normalized_shape, weight=None, bias=None, eps=1e-5) -> torch.Tensor:
    """Functional LayerNorm over the last dim (weight/bias optional)."""
    n = normalized_shape if isinstance(normalized_shape, int) else normalized_shape[0]
    return _norm(x, n, weight, bias, eps)


def fused_add_layernorm(x: torch.Tensor, residual: torch.Tensor, weight=None, bias=None,
                        eps=1e-5, return_sum: bool = True):
    """LayerNorm(x + residual); also returns the sum when return_sum."""
    out = _norm(x, x.shape[-1], weight, bias, eps, residual=residual, want_sum=return_sum)
    return out


__all__ = ["FusedLayerNorm", "fused_layernorm", "fused_add_layernorm"]
