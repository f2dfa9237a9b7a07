"""GLU activation act(input) * gate on gfx950.

Drop-in for kernels/fused_glu_mlp.py:61-104. As in the reference, 'gelu' and
'gelu_accurate' mean the exact erf GELU, the tanh names the tanh form, and
'silu'/'swish' SiLU; unknown names fall back to erf GELU. The two operands may
be the non-contiguous halves of one chunk()ed projection (no copies are made).
"""
from __future__ import annotations

import torch

from . import _lib
from ._glu import binary


def _act_code(act_fn: str) -> int:
    if act_fn in ("gelu", "gelu_accurate"):
        return _lib.ACT_GELU_ERF
    if act_fn in ("gelu_new", "gelu_fast", "gelu_pytorch_tanh"):
        return _lib.ACT_GELU_TANH
    if act_fn in ("silu", "swish"):
        return _lib.ACT_SILU
    return _lib.ACT_GELU_ERF


def fused_gelu_mul_dropout(input_tensor: torch.Tensor, gate_tensor: torch.Tensor,
                           act_fn: str = "gelu", dropout_p: float = 0.0,
                           training: bool = False) -> torch.Tensor:
    """act(input_tensor) * gate_tensor (inference; dropout is not supported)."""
    if training and dropout_p > 0:
        raise NotImplementedError("fused_gelu_mul_dropout: training-mode dropout is not supported")
    return binary("vfk_glu_fwd", _act_code(act_fn), input_tensor, gate_tensor)
