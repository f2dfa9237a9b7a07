"""residual + input on gfx950. Drop-in for kernels/fused_dropout_residual.py:57-104
in inference mode (training-mode dropout is not supported and raises)."""
from __future__ import annotations

import torch

from ._glu import binary


def fused_dropout_residual(input_tensor: torch.Tensor, residual_tensor: torch.Tensor,
                           dropout_p: float = 0.0, training: bool = False) -> torch.Tensor:
    if training and dropout_p > 0.0:
        raise NotImplementedError("fused_dropout_residual: training-mode dropout is not supported")
    return binary("vfk_residual_add", 0, input_tensor, residual_tensor).view_as(input_tensor)
