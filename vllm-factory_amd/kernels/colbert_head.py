"""ColBERT output head: final LayerNorm, PyLate Dense projection and L2
normalisation in one pass (vfk_colbert_head_fwd).

No reference kernel exists for this step: the reference's ColBERT plugin runs
the encoder's final LayerNorm (models/modernbert/modernbert_encoder.py:412-415,
:478), then its projection stack and
`projected / projected.norm(dim=-1, keepdim=True).clamp(min=1e-8)`
(plugins/moderncolbert/model.py:260-267, _ResidualDense :68-95) as separate
torch ops. Here the LayerNorm output is projected while it is still in LDS,
or, when it is not wanted back, the LayerNorm is folded into the projection:
y = rstd (u (gamma W)^T - mu G) + C.
"""
from __future__ import annotations

from typing import Optional, Sequence, Tuple

import torch
import torch.nn.functional as F

from . import _lib
from .weight_pack import folded_colbert_weight, packed_weight


def colbert_head(hidden: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor] = None,
                 norm_weight: Optional[torch.Tensor] = None,
                 norm_bias: Optional[torch.Tensor] = None, eps: float = 1e-5,
                 residual: Optional[torch.Tensor] = None,
                 return_hidden: bool = False, pack: bool = True):
    """hidden [T, D] (+ residual) -> LayerNorm (if norm_weight) -> @ weight^T
    (+ bias) -> rows scaled to unit L2 norm (norm clamped at 1e-8).
    weight [N, D] with N in {32, 64, 96, 128}; D a multiple of 128 up to 4096
    in the folded form, of 256 up to 1024 in the staged one.
    pack: the kernel reads the weight in MFMA operand order, made once per
    weight tensor (weight_pack); False reads the [N, D] rows. With pack, no
    return_hidden and D a multiple of 128, the LayerNorm weight is folded into
    the projection (vfk_colbert_head_folded_fwd: the raw rows go straight
    into the matrix instructions, 128 tokens per workgroup); otherwise the
    normalised rows are staged in LDS (vfk_colbert_head_fwd).
    Returns the [T, N] embeddings, and the LayerNorm output if return_hidden."""
    dev = _lib.require_gpu(hidden, weight, bias, norm_weight, norm_bias, residual)
    if hidden.dim() != 2 or weight.dim() != 2 or weight.shape[1] != hidden.shape[1]:
        raise ValueError("hidden must be [T, D] and weight [N, D]")
    x = _lib.rows_aligned(hidden)
    r = _lib.rows_aligned(residual) if residual is not None else None
    T, N = x.shape[0], weight.shape[0]
    out = torch.empty(T, N, dtype=x.dtype, device=dev)
    if pack and not return_hidden and x.shape[1] % 128 == 0:
        # folded form: gamma multiplied into the weight, the raw rows projected
        folded, g, c = folded_colbert_weight(weight, norm_weight, norm_bias, bias)
        _lib.on_device(
            "vfk_colbert_head_folded_fwd", dev, _lib.ref(_lib.desc(x)), _lib.ref(_lib.desc(r)),
            _lib.ref(_lib.desc(folded)), _lib.ref(_lib.desc(g if norm_weight is not None else None)),
            _lib.ref(_lib.desc(c)), float(eps), _lib.ref(_lib.desc(out)))
        return out
    wt = packed_weight(weight) if pack else _lib.rows_aligned(weight)
    h = torch.empty_like(x) if return_hidden else None
    vec = lambda t: None if t is None else t.contiguous()
    _lib.on_device(
        "vfk_colbert_head_fwd", dev,
        _lib.ref(_lib.desc(x)), _lib.ref(_lib.desc(r)), _lib.ref(_lib.desc(vec(norm_weight))),
        _lib.ref(_lib.desc(vec(norm_bias))), float(eps), _lib.ref(_lib.desc(wt)),
        _lib.ref(_lib.desc(vec(bias))), _lib.ref(_lib.desc(h)), _lib.ref(_lib.desc(out)))
    return (out, h) if return_hidden else out


ProjectionLayer = Tuple[torch.Tensor, Optional[torch.Tensor], Optional[torch.Tensor], bool]


def colbert_project(hidden_states: torch.Tensor, layers: Sequence[ProjectionLayer]) -> torch.Tensor:
    """The PyLate Dense stack plus L2 normalisation of
    plugins/moderncolbert/model.py:260-267 on [T, D] hidden states.
    layers: (weight, bias, residual_weight, use_residual) per _ResidualDense
    (:68-95): y = x W^T + b, plus x (same width) or x R^T when use_residual.
    All layers but the last run as GEMMs; the last one (which must not use a
    residual) runs fused with the normalisation."""
    if not layers:
        raise ValueError("at least one projection layer is needed")
    x = hidden_states
    for wt, b, rw, use_res in layers[:-1]:
        y = F.linear(x, wt, b)
        if use_res:
            y = y + (x if rw is None else F.linear(x, rw))
        x = y
    wt, b, rw, use_res = layers[-1]
    if use_res:
        raise NotImplementedError("a residual branch on the last projection layer is not fused")
    return colbert_head(x, wt, b)
