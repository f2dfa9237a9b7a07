"""T5 RMSNorm on gfx950 (the vLLM `RMSNorm` used by models/mt5/mt5_encoder.py:41,
461, 471, 519): out = x * rsqrt(mean(x^2) + eps) * weight, fp32 statistics."""
from __future__ import annotations

from typing import Optional

import torch

from .fused_layernorm import _norm


class RMSNorm(torch.nn.Module):
    def __init__(self, hidden_size: int, eps: float = 1e-6, dtype=None, device=None):
        super().__init__()
        self.variance_epsilon = eps
        self.weight = torch.nn.Parameter(torch.ones(hidden_size, dtype=dtype, device=device))

    def forward(self, x: torch.Tensor, residual: Optional[torch.Tensor] = None):
        """RMSNorm(x), or (RMSNorm(x + residual), x + residual) when residual is given
        (the vLLM fused_add_rms_norm convention)."""
        if residual is None:
            return _norm(x, x.shape[-1], self.weight, None, self.variance_epsilon, rms=True)
        return _norm(x, x.shape[-1], self.weight, None, self.variance_epsilon,
                     residual=residual, rms=True, want_sum=True)


def rms_norm(x: torch.Tensor, weight: Optional[torch.Tensor], eps: float = 1e-6) -> torch.Tensor:
    return _norm(x, x.shape[-1], weight, None, eps, rms=True)


def fused_add_rms_norm(x: torch.Tensor, residual: torch.Tensor, weight: Optional[torch.Tensor],
                       eps: float = 1e-6):
    """(RMSNorm(x + residual), x + residual) in one pass."""
    return _norm(x, x.shape[-1], weight, None, eps, residual=residual, rms=True, want_sum=True)
