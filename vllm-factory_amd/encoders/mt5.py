"""mT5 encoder forward (config 4 shapes: d_model 1024, 16 heads of 64,
gated-GELU d_ff 2816) on the hot-path kernels.

mt5_encoder_forward follows models/mt5/mt5_encoder.py:524-599
(MT5Encoder.forward): token embeddings (or inputs_embeds), the [B, 1, 1, L]
additive key mask (1 - m) * finfo.min, every layer with the layer-0 bias table
[buckets, heads], then the final RMSNorm (:591).

Follows models/mt5/mt5_encoder.py:476-491 (T5EncoderLayer):
    h = x + o_proj(RPB-attention(q, k, v of RMSNorm1(x)))
    out = h + wo(gelu_new(wi_0(RMSNorm2(h))) * wi_1(RMSNorm2(h)))
with the attention call of :269-279 (flash_attention_rpb_final, shared
[buckets, heads] table, scale 1.0, additive [B, 1, 1, L] key mask). The first
residual add is fused into the second RMSNorm and the second into the wo GEMM
(beta = 1).
"""
from __future__ import annotations

import weakref
from typing import Optional

import torch

from kernels.ff_fused import fused_gelu_mul_dropout
from kernels.fused_glu_mlp import glu_linear
from kernels.flash_attention_rpb import flash_attention_rpb_final
from kernels.rms_norm import fused_add_rms_norm, rms_norm


def mt5_layer_forward(x: torch.Tensor, wq, wk, wv, wo, wi0, wi1, wff_o, ln1, ln2, table,
                      mask, num_buckets: int = 32, max_distance: int = 128,
                      eps: float = 1e-6) -> torch.Tensor:
    """x [B, L, d_model] (bf16/fp16 on the GPU); weights as x @ W ([in, out])."""
    B, L, D = x.shape
    H = table.shape[1]
    d = D // H
    h = rms_norm(x, ln1, eps)
    # [B, L, H, d] projections viewed as [B, H, L, d] (strided, no copies)
    q, k, v = ((h @ w).view(B, L, H, d).transpose(1, 2) for w in (wq, wk, wv))
    att = flash_attention_rpb_final(q, k, v, table, num_buckets, max_distance, False,
                                    padding_mask=mask, softmax_scale=1.0)
    o = att.transpose(1, 2).reshape(B, L, D) @ wo
    h2, x1 = fused_add_rms_norm(o, x, ln2, eps)
    g = fused_gelu_mul_dropout(h2 @ wi0, h2 @ wi1, "gelu_new")
    return torch.addmm(x1.reshape(-1, D), g.reshape(-1, g.shape[-1]), wff_o).view(B, L, D)


def mt5_layer_packed(x: torch.Tensor, cu_seqlens: torch.Tensor, max_len: int, wq, wk, wv, wo,
                     wi0, wi1, wff_o, ln1, ln2, table, mask=None, num_buckets: int = 32,
                     max_distance: int = 128, eps: float = 1e-6, wqkv=None,
                     wi_glu=None) -> torch.Tensor:
    """The layer of mt5_layer_forward on packed sequences, without padding.

    x [T, d_model]: sequence s owns rows cu_seqlens[s] .. cu_seqlens[s + 1] -
    1 (int32 on the device), max_len >= every sequence length. Every part
    runs on the T rows: the RMSNorms, the fused q|k|v projection, the RPB
    attention over the packed sequences (flash_attention_rpb_varlen: each
    sequence attends to its own rows, as the padded layer with the
    reference's key mask does on its valid rows), the output projection, FFN
    and residual adds. mask is accepted for the padded layer's signature and
    not used. wqkv: the [D, 3D] concatenation of wq, wk, wv when the caller
    keeps one (built here otherwise). wi_glu: wi0 and wi1 stacked as the
    [2 d_ff, D] rows of one GLU projection (stack_glu_weight); given, the
    gated FF's two projections and gelu_new gate run as one kernel
    (glu_linear), which rounds the gate product once where the reference
    rounds both projections first."""
    from kernels.flash_attention_rpb import flash_attention_rpb_varlen
    T, D = x.shape
    H = table.shape[1]
    d = D // H
    if wqkv is None:
        wqkv = torch.cat((wq, wk, wv), 1)
    h = rms_norm(x, ln1, eps)
    qkv = (h @ wqkv).view(T, 3, H, d)
    att = flash_attention_rpb_varlen(qkv[:, 0], qkv[:, 1], qkv[:, 2], cu_seqlens, max_len, table,
                                     num_buckets, max_distance, False, 1.0)
    o = att.view(T, D) @ wo
    h2, x1 = fused_add_rms_norm(o, x, ln2, eps)
    if wi_glu is not None:
        g = glu_linear(h2, wi_glu, "gelu_new")
    else:
        g = fused_gelu_mul_dropout(h2 @ wi0, h2 @ wi1, "gelu_new")
    return torch.addmm(x1, g, wff_o)


_FUSED: dict = {}


def fused_layer_weights(lw):
    """(wqkv, wi_glu) of one layer tuple (wq, wk, wv, wo, wi0, wi1, ...): the
    [D, 3D] q|k|v concatenation and stack_glu_weight(wi0, wi1), made once per
    weight set and kept while the weights live. Keyed by the five source
    tensors and their version counters, so an in-place update rebuilds;
    tensors made under inference mode carry no version counter and are keyed
    by the objects alone."""
    srcs = (lw[0], lw[1], lw[2], lw[4], lw[5])
    key = tuple(id(t) for t in srcs)
    vers = tuple(-1 if t.is_inference() else t._version for t in srcs)
    hit = _FUSED.get(key)
    if hit is not None and hit[1] == vers and all(r() is t for r, t in zip(hit[0], srcs)):
        return hit[2]
    val = (torch.cat(lw[:3], 1), stack_glu_weight(lw[4], lw[5]))
    refs = tuple(weakref.ref(t, lambda _r, k=key: _FUSED.pop(k, None)) for t in srcs)
    _FUSED[key] = (refs, vers, val)
    return val


def stack_glu_weight(wi0: torch.Tensor, wi1: torch.Tensor) -> Optional[torch.Tensor]:
    """[D, d_ff] wi0, wi1 ([in, out]) -> the [2 d_ff, D] weight of glu_linear,
    or None where glu_linear does not take the shapes (D a multiple of 64,
    d_ff of 8, 16-bit weights)."""
    D, F_ = wi0.shape
    if D % 64 or F_ % 8 or wi0.dtype not in (torch.bfloat16, torch.float16):
        return None
    return torch.cat((wi0.t(), wi1.t()), 0).contiguous()


def mt5_encoder_forward(input_ids: Optional[torch.Tensor], attention_mask: Optional[torch.Tensor],
                        layers, table: torch.Tensor, final_ln: torch.Tensor,
                        embed: Optional[torch.Tensor] = None,
                        inputs_embeds: Optional[torch.Tensor] = None, num_buckets: int = 32,
                        max_distance: int = 128, eps: float = 1e-6,
                        packed: bool = True) -> torch.Tensor:
    """Padded-batch encoder: input_ids [B, L] (or [L]) with embed [vocab, d_model],
    or inputs_embeds [B, L, d_model]; attention_mask [B, L] of 1 (keep) / 0
    (pad) or None; layers: (wq, wk, wv, wo, wi0, wi1, wff_o, ln1, ln2) per
    layer as for mt5_layer_forward; table: layer 0's [buckets, heads].
    packed: when the mask is right padding, run the layers on the valid rows
    only (mt5_layer_packed); rows past each length are then returned as
    zeros (the reference's outputs there are never consumed: its callers
    read the valid rows). Any other mask runs the padded layers."""
    x = embed[input_ids] if inputs_embeds is None else inputs_embeds
    squeeze = x.dim() == 2
    if squeeze:
        x = x.unsqueeze(0)
    mask = None
    if attention_mask is not None:
        m = attention_mask.reshape(x.shape[0], -1)[:, None, None, :].to(x.dtype)
        mask = (1.0 - m) * torch.finfo(x.dtype).min
    cu = _right_padded_cu(attention_mask, x.shape[0], x.shape[1]) if packed else None
    if cu is not None:
        # right-padded batch: every layer on the valid rows only; rows past
        # each length come back as zeros
        from kernels.packing import pad_packed, unpad_packed
        B, L, D = x.shape
        T = int(cu[-1])
        xf = unpad_packed(x, cu, T)
        for lw in layers:
            wqkv, wi_glu = fused_layer_weights(lw)
            xf = mt5_layer_packed(xf, cu, L, *lw, table, None, num_buckets, max_distance, eps,
                                  wqkv=wqkv, wi_glu=wi_glu)
        x, _ = pad_packed(rms_norm(xf, final_ln, eps), cu, B, L)
        return x.squeeze(0) if squeeze else x
    for lw in layers:
        x = mt5_layer_forward(x, *lw, table, mask, num_buckets, max_distance, eps)
    x = rms_norm(x, final_ln, eps)
    return x.squeeze(0) if squeeze else x


def _right_padded_cu(attention_mask: Optional[torch.Tensor], B: int, L: int):
    """int32 cu_seqlens [B + 1] on the device when attention_mask [B, L] is 1
    on a prefix of each row and 0 after it (right padding), else None (one
    read-back of the check)."""
    if attention_mask is None:
        return None
    m = attention_mask.reshape(B, L) != 0
    lens = m.sum(1)
    prefix = torch.arange(L, device=m.device)[None, :] < lens[:, None]
    if not bool(torch.equal(m, prefix)):
        return None
    return torch.cat([lens.new_zeros(1), lens.cumsum(0)]).to(torch.int32)


def mt5_encoder_flat(x: torch.Tensor, positions: torch.Tensor, layers, table: torch.Tensor,
                     num_buckets: int = 32, max_distance: int = 128,
                     eps: float = 1e-6) -> torch.Tensor:
    """mT5 encoder layers on a flat vLLM stream routed per sequence.

    The reference's mT5 GLiNER plugin (plugins/mt5_gliner/model.py:169-201)
    runs the encoder on the flat [1, T] stream with an all-ones mask, so the
    tokens of different requests attend to each other. Here the sequences are
    found from the position ids on the device (a sequence starts at position
    0, kernels.packing.seq_metadata rule "zero") and every layer runs on the
    packed rows (mt5_layer_packed: attention over the packed sequences, no
    padding); each sequence gets the attention it would get alone.
    x: embedding output [T, d_model]; layers: (wq, wk, wv, wo, wi0, wi1, wff_o,
    ln1, ln2) per layer as for mt5_layer_forward."""
    from kernels.packing import read_metadata, seq_metadata
    cu, meta = seq_metadata(positions, "zero")
    cu, n, max_len, _ = read_metadata(cu, meta)
    for lw in layers:
        wqkv, wi_glu = fused_layer_weights(lw)
        x = mt5_layer_packed(x, cu, max_len, *lw, table, None, num_buckets, max_distance, eps,
                             wqkv=wqkv, wi_glu=wi_glu)
    return x
