"""Memory-bound epilogues (oracle; test infrastructure only).

Pinned by (tests/test_oracle_epilogues.py): torch.nn.functional.layer_norm,
F.gelu(approximate='none'|'tanh'), F.silu, transformers' T5LayerNorm for
RMSNorm; rope_table by RoPE's closed form (each (x[f], x[f+32]) pair as a
complex number times e^{i angle}), transformers' ModernBERT
apply_rotary_pos_emb and the brute-force-pinned oracle.attention.apply_rope,
with a negative control (a sign-flipped rotate_half fails all three while it
passes the RoPE identities); residual_add by torch.add; and, for the ColBERT
head, F.linear + F.normalize and unit row norms.
"""
from __future__ import annotations

import math
from typing import Optional

import torch


def layernorm(x, weight=None, bias=None, eps=1e-5, dtype=torch.float32):
    """kernels/fused_layernorm.py:56-106: mean, then E[(x-mean)^2], rstd = 1/sqrt(var+eps),
    y = (x - mean) * rstd * w (+ b), statistics in fp32."""
    x = x.to(dtype)
    mean = x.mean(-1, keepdim=True)
    var = ((x - mean) ** 2).mean(-1, keepdim=True)
    y = (x - mean) / torch.sqrt(var + eps)
    if weight is not None:
        y = y * weight.to(dtype)
    if bias is not None:
        y = y + bias.to(dtype)
    return y


def rmsnorm(x, weight=None, eps=1e-6, dtype=torch.float32):
    """vLLM RMSNorm as used by models/mt5/mt5_encoder.py:41, 461, 471, 519:
    x * rsqrt(mean(x^2) + eps) * weight (no mean subtraction, no bias)."""
    x = x.to(dtype)
    y = x / torch.sqrt((x * x).mean(-1, keepdim=True) + eps)
    if weight is not None:
        y = y * weight.to(dtype)
    return y


def gelu_erf(x):
    """kernels/fused_glu_mlp.py:45-48: 0.5 x (1 + erf(x / sqrt 2))."""
    return 0.5 * x * (1.0 + torch.erf(x / math.sqrt(2.0)))


def gelu_tanh(x):
    """kernels/ff_fused.py:47-53: 0.5 x (1 + tanh(sqrt(2/pi)(x + 0.044715 x^3))),
    the reference writing tanh(z) as 2 sigmoid(2z) - 1."""
    inner = math.sqrt(2.0 / math.pi) * (x + 0.044715 * x ** 3)
    return 0.5 * x * (1.0 + (2.0 * torch.sigmoid(2.0 * inner) - 1.0))


def glu(a, b, act: str, dtype=torch.float32):
    """act(a) * b for act in {'gelu_erf', 'gelu_tanh', 'silu', 'relu'}
    (fused_glu_mlp.py:44-56, ff_fused.py:43-62)."""
    a, b = a.to(dtype), b.to(dtype)
    if act == "gelu_erf":
        y = gelu_erf(a)
    elif act == "gelu_tanh":
        y = gelu_tanh(a)
    elif act == "silu":
        y = a * torch.sigmoid(a)
    elif act == "relu":
        y = torch.clamp(a, min=0)
    else:
        raise ValueError(act)
    return y * b


def rope_table(x, cos, sin, dtype=torch.float32):
    """kernels/fused_rope_global.py:83-101: x [B,S,H,D], cos/sin [B,S,D];
    out[d] = x[d] cos[d] - x[d+D/2] sin[d] (d < D/2), x[d] cos[d] + x[d-D/2] sin[d]."""
    x, cos, sin = x.to(dtype), cos.to(dtype), sin.to(dtype)
    if cos.dim() == 4:
        cos, sin = cos.squeeze(1), sin.squeeze(1)
    h = x.shape[-1] // 2
    rot = torch.cat((-x[..., h:], x[..., :h]), dim=-1)
    return x * cos.unsqueeze(2) + rot * sin.unsqueeze(2)


def residual_add(x, residual, dtype=torch.float32):
    """kernels/fused_dropout_residual.py:50-51 (inference): residual + x."""
    return residual.to(dtype) + x.to(dtype)


def residual_dense(x, weight, bias=None, residual_weight=None, use_residual=False,
                   dtype=torch.float32):
    """plugins/moderncolbert/model.py:68-95 (_ResidualDense.forward): x W^T (+ b),
    plus x (same width) or x R^T when use_residual."""
    x = x.to(dtype)
    y = x @ weight.to(dtype).t()
    if bias is not None:
        y = y + bias.to(dtype)
    if use_residual:
        y = y + (x if residual_weight is None else x @ residual_weight.to(dtype).t())
    return y


def dense_residual_layernorm(x, weight, bias, residual, ln_weight=None, ln_bias=None, eps=1e-7,
                             round_dtype=None, dtype=torch.float32):
    """DeBERTa's post-LN output block, DebertaV2SelfOutput.forward and
    DebertaV2Output.forward (models/deberta_v2/deberta_v2_encoder.py:504-508 and
    :563-567, dropout the identity at inference): LayerNorm(x W^T + b + residual).
    round_dtype: the storage type the unfused Linear writes its output in
    (rounded once, after the bias); None keeps the projection unrounded."""
    y = residual_dense(x, weight, bias, dtype=dtype)
    if round_dtype is not None:
        y = y.to(round_dtype).to(dtype)
    return layernorm(y + residual.to(dtype), ln_weight, ln_bias, eps, dtype)


def colbert_head(hidden, layers, norm_weight=None, norm_bias=None, eps=1e-5, residual=None,
                 layer_norm=True, dtype=torch.float32):
    """The encoder's final LayerNorm (models/modernbert/modernbert_encoder.py:412-415,
    :478; input hidden + residual when given) unless layer_norm is False, then
    the ColBERT projection stack and L2 normalisation of
    plugins/moderncolbert/model.py:260-267: projected / max(|projected|, 1e-8).
    layers: (weight, bias, residual_weight, use_residual) per Dense module."""
    x = hidden.to(dtype)
    if residual is not None:
        x = x + residual.to(dtype)
    if layer_norm:
        x = layernorm(x, norm_weight, norm_bias, eps, dtype)
    for w, b, rw, use_res in layers:
        x = residual_dense(x, w, b, rw, use_res, dtype)
    return x / x.norm(dim=-1, keepdim=True).clamp(min=1e-8)
