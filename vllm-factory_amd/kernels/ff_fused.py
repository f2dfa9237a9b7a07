"""Gated FFN activation act(gate) * up on gfx950 (T5 / mT5).

Drop-in for kernels/ff_fused.py:86-125. The reference's name map applies
(:76-83): 'gelu', 'gelu_new', 'gelu_fast', 'gelu_pytorch_tanh' -> tanh GELU,
'gelu_accurate' -> erf GELU, 'relu', 'silu'/'swish'; unknown -> tanh GELU.
"""
from __future__ import annotations

import torch

from . import _lib
from ._glu import binary

_MAP = {
    "gelu": _lib.ACT_GELU_TANH, "gelu_new": _lib.ACT_GELU_TANH,
    "gelu_fast": _lib.ACT_GELU_TANH, "gelu_pytorch_tanh": _lib.ACT_GELU_TANH,
    "gelu_accurate": _lib.ACT_GELU_ERF,
    "relu": _lib.ACT_RELU,
    "silu": _lib.ACT_SILU, "swish": _lib.ACT_SILU,
}


def _act_type_map(act_fn: str) -> int:
    return _MAP.get(act_fn.lower(), _lib.ACT_GELU_TANH)


def fused_gelu_mul_dropout(gate: torch.Tensor, up: torch.Tensor, act_fn: str = "gelu",
                           dropout_p: float = 0.0, training: bool = False) -> torch.Tensor:
    """act(gate) * up, result shaped like gate (inference; no dropout)."""
    if training and dropout_p > 0.0:
        raise NotImplementedError("fused_gelu_mul_dropout: training-mode dropout is not supported")
    return binary("vfk_glu_fwd", _act_type_map(act_fn), gate, up).view_as(gate)
