"""GLU activation act(input) * gate on gfx950, and the GLU projection with
that product fused into the GEMM.

fused_gelu_mul_dropout is the drop-in for kernels/fused_glu_mlp.py:61-104. As in the reference, 'gelu' and
'gelu_accurate' mean the exact erf GELU, the tanh names the tanh form, and
'silu'/'swish' SiLU; unknown names fall back to erf GELU. The two operands may
be the non-contiguous halves of one chunk()ed projection (no copies are made).
"""
from __future__ import annotations

import torch

from . import _lib
from ._glu import binary

__all__ = ["fused_gelu_mul_dropout", "glu_linear"]


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


def glu_linear(x: torch.Tensor, weight: torch.Tensor, act_fn: str = "gelu",
               out: torch.Tensor | None = None) -> torch.Tensor:
    """act(x W_in^T) * (x W_gate^T) for weight = [W_in; W_gate] of shape [2I, K],
    in one kernel (vfk_glu_linear_fwd): the MLP projection and GLU of
    models/modernbert/modernbert_encoder.py:157-178 (Wi, chunk, GELU(input) *
    gate) without the [.., 2I] intermediate. The sums accumulate in fp32 and
    the activation is applied to them before the one rounding to x.dtype, where
    the unfused path rounds the projection first.

    x [..., K] and weight in bf16 or fp16; K a multiple of 64, I of 8. Returns
    [..., I] (or fills `out`, a [rows, I] tensor with contiguous rows)."""
    dev = _lib.require_gpu(x, weight)
    K = x.shape[-1]
    if weight.dim() != 2 or weight.shape[1] != K or weight.shape[0] % 2:
        raise ValueError(f"glu_linear: weight must be [2I, {K}], got {tuple(weight.shape)}")
    if weight.dtype != x.dtype:
        raise ValueError("glu_linear: x and weight must share a dtype")
    I = weight.shape[0] // 2
    x2 = _lib.rows_aligned(x.reshape(-1, K))
    w2 = _lib.rows_aligned(weight)
    if out is None:
        out = torch.empty(x2.shape[0], I, dtype=x.dtype, device=x.device)
    elif out.shape != (x2.shape[0], I) or out.dtype != x.dtype:
        raise ValueError(f"glu_linear: out must be [{x2.shape[0]}, {I}] {x.dtype}")
    _lib.on_device("vfk_glu_linear_fwd", dev, _act_code(act_fn), _lib.ref(_lib.desc(x2)),
                   _lib.ref(_lib.desc(w2)), _lib.ref(_lib.desc(out)))
    return out.view(*x.shape[:-1], I)
