"""Encoder-level restatements (oracle; test infrastructure only).

modernbert_encoder follows the reference's ModernBERT forward
(models/modernbert/modernbert_encoder.py):
  embeddings  tok_embeddings -> LayerNorm (no bias)               :102-128
  layer i     attn_norm (Identity for layer 0, else LayerNorm)     :289-315
              Wqkv -> RoPE -> attention -> Wo, residual add         :214-260, :329-339
              mlp_norm -> Wi -> GELU(input) * gate -> Wo, residual  :135-178, :341-350
  final       LayerNorm                                             :412-415, :478
global layers are layer_id % 3 == 0 with RoPE theta 160000 and full
attention inside each sequence; the others use theta 10000 and |i - j| <= 64
(:198, :379-390, :539-549); key j is hidden when its token id is 50284
(:456-460). Everything is computed per sequence in fp32 (the packed dense
masks of :491-550 are equivalent and infeasible at benchmark sizes).

mt5_encoder is the stack with the final RMSNorm (models/mt5/mt5_encoder.py
:524-599); mt5_layer follows the reference's T5EncoderLayer (:476-491):
h = x + SelfAttention(RMSNorm1(x)); h + FF(RMSNorm2(h)), with the
relative-position-bias attention of :234-320 (bidirectional buckets, bias
table [buckets, heads] shared from layer 0, no 1/sqrt(d) scaling, additive
key mask (1 - m) * finfo.min, :571-576) and the gated FFN of :411-447
(gelu_new = tanh GELU on wi_0, times wi_1, then wo).

deberta_encoder follows the reference's DebertaV2Encoder (models/deberta_v2/
deberta_v2_encoder.py:734-819): LayerNorm of the relative table (:770-774),
then per layer (:627-645) query/key/value_proj with bias, the flash
disentangled attention of :246-330 (share_att_key: pos_key = q key_proj(rel)^T,
pos_query = k query_proj(rel)^T, sm_scale 1/sqrt(3 d), log buckets, keys at or
beyond the sequence length hidden, those query rows zero), dense ->
LayerNorm(. + x) (:494-510), GELU(erf) intermediate (:535-550), dense ->
LayerNorm(. + attention_output) (:553-568).

deberta_v1_layer follows the reference's DeBERTa v1 DebertaLayer
(models/deberta/deberta_encoder.py:132-548, flash path :246-309): one in_proj
without bias whose rows hold [q, k, v] per head, q_bias and v_bias added
after it, att_span = min(L, max_relative_positions), the relative table
rel_embeddings[max_rel - span : max_rel + span] projected by pos_proj (no
bias, c2p) and pos_q_proj (bias, p2c), sm_scale 1/sqrt(3 d), linear relative
positions; then the same post-LN blocks as v2 with DebertaLayerNorm (:71-92,
eps inside the square root; identical to LayerNorm in fp32).

Pinned by (tests/test_oracle_encoders.py): transformers' ModernBertModel,
MT5EncoderModel, DebertaV2Encoder and DebertaEncoder (v1) with the same
weights (implementations independent of this restatement and of the
reference), on reduced configurations.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import List, Optional

import torch

from .attention import (deberta_flash_attention, deberta_position_projections, rpb_attention,
                        varlen_attention)
from .epilogues import gelu_erf, gelu_tanh, layernorm, rmsnorm

MASK_TOKEN_ID = 50284  # modernbert_encoder.py:456-460


@dataclass
class ModernBertLayerWeights:
    wqkv: torch.Tensor       # [3 * hidden, hidden] (q, k, v row blocks; heads of 64)
    wo: torch.Tensor         # [hidden, hidden]
    wi: torch.Tensor         # [2 * inter, hidden] (input rows, then gate rows)
    wo_mlp: torch.Tensor     # [hidden, inter]
    attn_norm: Optional[torch.Tensor]   # [hidden] or None (layer 0: Identity)
    mlp_norm: torch.Tensor   # [hidden]


@dataclass
class ModernBertWeights:
    hidden: int
    heads: int
    inter: int
    emb: torch.Tensor        # [vocab, hidden]
    emb_norm: torch.Tensor   # [hidden]
    layers: List[ModernBertLayerWeights] = field(default_factory=list)
    final_norm: Optional[torch.Tensor] = None
    global_every: int = 3
    window: int = 64              # local_attention // 2
    theta_global: float = 160000.0
    theta_local: float = 10000.0
    eps: float = 1e-5


def modernbert_layer(x: torch.Tensor, w: ModernBertWeights, i: int, cu_seqlens: torch.Tensor,
                     key_valid: Optional[torch.Tensor], dtype=torch.float32) -> torch.Tensor:
    """One encoder layer (modernbert_encoder.py:317-352) over a packed stream [T, hidden]."""
    lw = w.layers[i]
    T = x.shape[0]
    d = w.hidden // w.heads
    h = x if lw.attn_norm is None else layernorm(x, lw.attn_norm, None, w.eps, dtype)
    qkv = h @ lw.wqkv.to(dtype).t()
    q, k, v = (t.reshape(T, w.heads, d) for t in qkv.chunk(3, dim=-1))
    is_global = i % w.global_every == 0
    att = varlen_attention(q, k, v, cu_seqlens, -1 if is_global else w.window,
                           w.theta_global if is_global else w.theta_local,
                           key_valid, 1.0 / math.sqrt(d), dtype)
    x = x + att.reshape(T, w.hidden) @ lw.wo.to(dtype).t()
    h = layernorm(x, lw.mlp_norm, None, w.eps, dtype)
    y = h @ lw.wi.to(dtype).t()
    inp, gate = y.chunk(2, dim=-1)
    return x + (gelu_erf(inp) * gate) @ lw.wo_mlp.to(dtype).t()


def modernbert_encoder(ids: torch.Tensor, cu_seqlens: torch.Tensor, w: ModernBertWeights,
                       dtype=torch.float32, num_layers: Optional[int] = None) -> torch.Tensor:
    """Full forward over packed token ids [T] -> final hidden states [T, hidden]."""
    key_valid = ids != MASK_TOKEN_ID
    x = layernorm(w.emb[ids].to(dtype), w.emb_norm, None, w.eps, dtype)
    n = len(w.layers) if num_layers is None else num_layers
    for i in range(n):
        x = modernbert_layer(x, w, i, cu_seqlens, key_valid, dtype)
    return layernorm(x, w.final_norm, None, w.eps, dtype)


def mt5_layer(x: torch.Tensor, wq, wk, wv, wo, wi0, wi1, wff_o, ln1, ln2, table,
              mask: Optional[torch.Tensor], num_buckets: int = 32, max_distance: int = 128,
              eps: float = 1e-6, dtype=torch.float32) -> torch.Tensor:
    """One mT5 encoder layer on x [B, L, d_model]; weights as x @ W ([in, out]);
    table [buckets, heads]; mask additive [B, 1, 1, L] or None."""
    x = x.to(dtype)
    B, L, D = x.shape
    H = table.shape[1]
    d = D // H
    h = rmsnorm(x, ln1, eps, dtype)
    q, k, v = ((h @ w.to(dtype)).view(B, L, H, d).transpose(1, 2) for w in (wq, wk, wv))
    att = rpb_attention(q, k, v, table.to(dtype), num_buckets, max_distance, False,
                        None if mask is None else mask.to(dtype), 1.0, dtype=dtype)
    x = x + att.transpose(1, 2).reshape(B, L, D) @ wo.to(dtype)
    h = rmsnorm(x, ln2, eps, dtype)
    return x + (gelu_tanh(h @ wi0.to(dtype)) * (h @ wi1.to(dtype))) @ wff_o.to(dtype)


def mt5_encoder(x: torch.Tensor, layers, table, final_ln, mask: Optional[torch.Tensor],
                num_buckets: int = 32, max_distance: int = 128, eps: float = 1e-6,
                dtype=torch.float32) -> torch.Tensor:
    """models/mt5/mt5_encoder.py:524-599 (MT5Encoder.forward) after the
    embeddings: every layer with layer 0's table, then the final RMSNorm (:591).
    layers: (wq, wk, wv, wo, wi0, wi1, wff_o, ln1, ln2) per layer."""
    for lw in layers:
        x = mt5_layer(x, *lw, table, mask, num_buckets, max_distance, eps, dtype)
    return rmsnorm(x, final_ln, eps, dtype)


def deberta_layer(x: torch.Tensor, seq_lengths: torch.Tensor, rel: torch.Tensor, lw, heads: int,
                  position_buckets: int = 256, max_relative_positions: int = 512,
                  eps: float = 1e-7, dtype=torch.float32) -> torch.Tensor:
    """One DebertaV2Layer on x [B, L, hidden]; rel = LayerNorm(rel_embeddings);
    lw has wqkv/bqkv (query, key, value rows), wo/bo, ln1_w/ln1_b, wi/bi,
    wo2/bo2, ln2_w/ln2_b in nn.Linear layout."""
    x = x.to(dtype)
    B, L, D = x.shape
    d = D // heads

    def lin(t, W, b):
        return t @ W.to(dtype).t() + b.to(dtype)

    def split(t):  # [..., n, D] -> [..., H, n, d]
        return t.reshape(*t.shape[:-1], heads, d).transpose(-2, -3)

    wq, wk, wv = lw.wqkv.chunk(3, dim=0)
    bq, bk, bv = lw.bqkv.chunk(3, dim=0)
    q, k, v = split(lin(x, wq, bq)), split(lin(x, wk, bk)), split(lin(x, wv, bv))
    span = position_buckets if position_buckets > 0 else max_relative_positions
    r = rel[:2 * span].to(dtype)
    pk, pq = deberta_position_projections(q, k, split(lin(r, wk, bk)), split(lin(r, wq, bq)), dtype)
    ctx = deberta_flash_attention(q, k, v, seq_lengths, pk, pq, 1.0 / math.sqrt(3 * d),
                                  position_buckets if position_buckets > 0 else span,
                                  max_relative_positions, position_buckets > 0, dtype=dtype)
    ctx = ctx.transpose(1, 2).reshape(B, L, D)
    h = layernorm(lin(ctx, lw.wo, lw.bo) + x, lw.ln1_w, lw.ln1_b, eps, dtype)
    inter = gelu_erf(lin(h, lw.wi, lw.bi))
    return layernorm(lin(inter, lw.wo2, lw.bo2) + h, lw.ln2_w, lw.ln2_b, eps, dtype)


def deberta_encoder(x: torch.Tensor, seq_lengths: torch.Tensor, w, dtype=torch.float32,
                    num_layers: Optional[int] = None) -> torch.Tensor:
    """Encoder stack on embedding output x [B, L, hidden]; w has hidden, heads,
    rel_emb, rel_ln_w, rel_ln_b, layers, position_buckets,
    max_relative_positions, eps."""
    rel = layernorm(w.rel_emb.to(dtype), w.rel_ln_w, w.rel_ln_b, w.eps, dtype)
    n = len(w.layers) if num_layers is None else num_layers
    for i in range(n):
        x = deberta_layer(x, seq_lengths, rel, w.layers[i], w.heads, w.position_buckets,
                          w.max_relative_positions, w.eps, dtype)
    return x


def deberta_v1_layer(x: torch.Tensor, seq_lengths: torch.Tensor, rel_emb: torch.Tensor, lw,
                     heads: int, max_relative_positions: int = 512, eps: float = 1e-7,
                     dtype=torch.float32) -> torch.Tensor:
    """One DeBERTa v1 DebertaLayer on x [B, L, hidden] (deberta_encoder.py:528-548).
    rel_emb = encoder.rel_embeddings.weight [2 max_rel, hidden]; lw has in_proj
    [3 hidden, hidden] (per head: q, k, v rows), q_bias, v_bias, pos_proj
    [hidden, hidden], pos_q_proj / pos_q_bias, wo/bo, ln1_w/ln1_b, wi/bi,
    wo2/bo2, ln2_w/ln2_b."""
    x = x.to(dtype)
    B, L, D = x.shape
    d = D // heads

    def lin(t, W, b=None):
        y = t @ W.to(dtype).t()
        return y if b is None else y + b.to(dtype)

    def split(t):  # [..., n, D] -> [..., H, n, d]
        return t.reshape(*t.shape[:-1], heads, d).transpose(-2, -3)

    qkv = lin(x, lw.in_proj).view(B, L, heads, 3 * d).transpose(1, 2)  # :219-220
    q, k, v = qkv.chunk(3, dim=-1)
    q = q + lw.q_bias.to(dtype).view(heads, 1, d)
    v = v + lw.v_bias.to(dtype).view(heads, 1, d)
    span = min(L, max_relative_positions)                               # :261
    r = rel_emb[max_relative_positions - span:max_relative_positions + span].to(dtype)
    key_rel = split(lin(r, lw.pos_proj))                                # :272-274
    query_rel = split(lin(r, lw.pos_q_proj, lw.pos_q_bias))             # :281-283
    pk, pq = deberta_position_projections(q, k, key_rel, query_rel, dtype)
    ctx = deberta_flash_attention(q, k, v, seq_lengths, pk, pq, 1.0 / math.sqrt(3 * d), span,
                                  max_relative_positions, False, dtype=dtype)
    ctx = ctx.transpose(1, 2).reshape(B, L, D)
    h = layernorm(lin(ctx, lw.wo, lw.bo) + x, lw.ln1_w, lw.ln1_b, eps, dtype)
    inter = gelu_erf(lin(h, lw.wi, lw.bi))
    return layernorm(lin(inter, lw.wo2, lw.bo2) + h, lw.ln2_w, lw.ln2_b, eps, dtype)
