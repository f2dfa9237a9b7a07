"""Elementwise activation act(x) on gfx950 (vfk_act_fwd): the intermediate
activation of the DeBERTa-v2 layer (models/deberta_v2/deberta_v2_encoder.py
:535-550, ACT2FN[hidden_act]); 'gelu' is the exact erf form."""
from __future__ import annotations

import torch

from . import _lib
from ._glu import flat2d


_ACT = {"gelu": _lib.ACT_GELU_ERF, "gelu_new": _lib.ACT_GELU_TANH, "gelu_pytorch_tanh": _lib.ACT_GELU_TANH,
        "silu": _lib.ACT_SILU, "swish": _lib.ACT_SILU, "relu": _lib.ACT_RELU}


def activation(x: torch.Tensor, act_fn: str = "gelu") -> torch.Tensor:
    if act_fn not in _ACT:
        raise NotImplementedError(f"activation {act_fn!r} is not built")
    dev = _lib.require_gpu(x)
    x2 = flat2d(x)
    out = torch.empty(x2.shape, dtype=x.dtype, device=x.device)
    if out.numel():
        _lib.on_device("vfk_act_fwd", dev, int(_ACT[act_fn]), _lib.ref(_lib.desc(x2)),
                       _lib.ref(_lib.desc(out)))
    return out.view(x.shape)
