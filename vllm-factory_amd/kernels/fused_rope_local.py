"""RoPE for ModernBERT local layers: the same one-launch q/k kernel as the
global layers with the local-theta cos/sin tables. Drop-in for
kernels/fused_rope_local.py:11-76."""
from __future__ import annotations

import torch

from .fused_rope_global import fused_rope_global_apply


def fused_rope_local_apply(q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor,
                           sin: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Apply RoPE (local) to query and key tensors [B, S, H, D]."""
    return fused_rope_global_apply(q, k, cos, sin)
