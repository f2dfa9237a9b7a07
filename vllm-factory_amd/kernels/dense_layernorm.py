"""Dense projection + bias + residual + LayerNorm in one gfx950 kernel.

DeBERTa's post-LN output blocks, DebertaV2SelfOutput and DebertaV2Output
(models/deberta_v2/deberta_v2_encoder.py:494-510 and :553-568), compute
LayerNorm(dense(hidden_states) + input_tensor); dropout is the identity at
inference. `dense_add_layernorm` does that in one launch: the projection is
rounded to the storage type once, as the unfused Linear writes it, and the
LayerNorm statistics are fp32 over that value plus the residual, as in
`fused_add_layernorm`; the [M, N] projection never reaches memory.

The kernel reads the weight in its MFMA operand order; `pack_dense_weight`
makes that copy (`SelfOutput` keeps one per weight tensor and version through
`weight_pack.packed_weight`).

`SelfOutput` keeps the reference module's parameter names (`dense.weight`,
`dense.bias`, `LayerNorm.weight`, `LayerNorm.bias`), so a DeBERTa state dict
loads into it unchanged.
"""
from __future__ import annotations

from typing import Optional

import torch

from . import _lib
from .weight_pack import pack_weight, packed_weight


def pack_dense_weight(weight: torch.Tensor) -> torch.Tensor:
    """The [N, K] projection weight in the kernel's operand order,
    [N / 32, K / 16, 64, 8] (vfk_pack_weight_mfma32); pack once per weight."""
    return pack_weight(weight)


def dense_add_layernorm(x: torch.Tensor, weight: Optional[torch.Tensor], bias: Optional[torch.Tensor],
                        residual: torch.Tensor, ln_weight: Optional[torch.Tensor] = None,
                        ln_bias: Optional[torch.Tensor] = None, eps: float = 1e-7,
                        out: Optional[torch.Tensor] = None,
                        packed_weight: Optional[torch.Tensor] = None,
                        return_sum: bool = False, residual_out: Optional[torch.Tensor] = None):
    """LayerNorm(x weight^T + bias + residual) * ln_weight + ln_bias over the
    last dim. x [..., K], weight [N, K] (or packed_weight from
    pack_dense_weight; without it the weight is packed on every call),
    residual [..., N] with x's leading shape; N in {256, 512, 768, 1024}, K a
    multiple of 64; bf16 or fp16. out (optional, [..., N]) may be the
    residual itself. return_sum: also return the sum x weight^T + bias +
    residual (rounded once; written to residual_out when given, which may be
    the residual itself), as (normalised, sum)."""
    if packed_weight is None:
        if weight is None:
            raise ValueError("weight or packed_weight is required")
        packed_weight = pack_dense_weight(weight)
    dev = _lib.require_gpu(x, packed_weight, bias, residual, ln_weight, ln_bias, out, residual_out)
    K, N = x.shape[-1], 32 * packed_weight.shape[0]
    if packed_weight.dim() != 4 or packed_weight.shape[1] * 16 != K:
        raise ValueError(f"packed weight {tuple(packed_weight.shape)} does not match K = {K}")
    if residual.shape != x.shape[:-1] + (N,):
        raise ValueError(f"residual must be {tuple(x.shape[:-1]) + (N,)}, got {tuple(residual.shape)}")
    x2 = _lib.rows_aligned(x.reshape(-1, K))
    r2 = residual.reshape(-1, N)
    in_place = out is not None and out.data_ptr() == residual.data_ptr()
    if not in_place:
        r2 = _lib.rows_aligned(r2)
    if out is None:
        o2 = torch.empty(r2.shape, dtype=x.dtype, device=x.device)
    else:
        if out.shape != residual.shape:
            raise ValueError(f"out must be {tuple(residual.shape)}, got {tuple(out.shape)}")
        o2 = out.reshape(-1, N)
        if o2.data_ptr() != out.data_ptr():
            raise ValueError("out must be viewable as [rows, N]")
        if in_place:
            r2 = o2
    s2 = None
    if return_sum or residual_out is not None:
        if residual_out is None:
            residual_out = torch.empty_like(residual)
        if residual_out.shape != residual.shape:
            raise ValueError(f"residual_out must be {tuple(residual.shape)}")
        s2 = residual_out.reshape(-1, N)
        if s2.data_ptr() != residual_out.data_ptr():
            raise ValueError("residual_out must be viewable as [rows, N]")
        if s2.data_ptr() == residual.data_ptr():
            r2 = s2
    params = [p.contiguous() if p is not None else None for p in (bias, ln_weight, ln_bias)]
    _lib.on_device("vfk_dense_residual_layernorm_fwd", dev, _lib.ref(_lib.desc(x2)),
                   _lib.ref(_lib.desc(packed_weight)), _lib.ref(_lib.desc(params[0])),
                   _lib.ref(_lib.desc(r2)), _lib.ref(_lib.desc(params[1])),
                   _lib.ref(_lib.desc(params[2])), float(eps), _lib.ref(_lib.desc(o2)),
                   _lib.ref(_lib.desc(s2)))
    y = out if out is not None else o2.view(residual.shape)
    if s2 is not None:
        return y, residual_out
    return y


class SelfOutput(torch.nn.Module):
    """DebertaV2SelfOutput / DebertaV2Output at inference: dense, then
    LayerNorm(. + input_tensor), as one kernel."""

    def __init__(self, in_features: int, hidden_size: int, eps: float = 1e-7, dtype=None,
                 device=None):
        super().__init__()
        self.dense = torch.nn.Linear(in_features, hidden_size, bias=True, dtype=dtype, device=device)
        self.LayerNorm = torch.nn.LayerNorm(hidden_size, eps=eps, dtype=dtype, device=device)

    def forward(self, hidden_states: torch.Tensor, input_tensor: torch.Tensor) -> torch.Tensor:
        # the packed copy is made once per weight tensor and version
        return dense_add_layernorm(hidden_states, None, self.dense.bias, input_tensor,
                                   self.LayerNorm.weight, self.LayerNorm.bias, self.LayerNorm.eps,
                                   packed_weight=packed_weight(self.dense.weight))


__all__ = ["pack_dense_weight", "dense_add_layernorm", "SelfOutput"]
