"""DeBERTa-v3 and DeBERTa v1 encoder forwards (padded batch [B, L, hidden]) on the
hot-path kernels (v1: deberta_v1_layer_forward, linear relative positions).

Follows models/deberta_v2/deberta_v2_encoder.py: the encoder (:734-819)
LayerNorms the relative-position table once (get_rel_embedding, :770-774)
and runs each DebertaV2Layer (:627-645):
    attention   query/key/value_proj (bias) -> flash disentangled attention
                (:246-330: share_att_key, c2p|p2c, sm_scale 1/sqrt(3 d), log
                buckets) -> dense -> LayerNorm(. + x)            (:494-510)
    intermediate dense -> GELU (erf)                               (:535-550)
    output      dense -> LayerNorm(. + attention_output)           (:553-568)

Differences from the reference, by construction: the three projections are
one GEMM with concatenated weights; pos_key / pos_query are not materialised
as [B, H, L, 2S] tensors: the attention kernel computes q.key_rel and
k.query_rel per tile from the per-head projections of the relative table
(one [2S, hidden] x [hidden, 2 hidden] GEMM per layer, whose output is
copied once into the kernel's chunk-major table layout); the attention writes
its [B, L, H, d] context in place, so no permute copy precedes the dense
projection; the residual add is folded into each LayerNorm pass. Query rows
at or beyond a sequence's length attend nowhere and hold zeros after the
attention, as the reference's kernel writes them.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import List, Optional

import torch
import torch.nn.functional as F

from kernels.activation import activation
from kernels.dense_layernorm import dense_add_layernorm
from kernels.weight_pack import packed_weight
from kernels.flash_deberta_attention import (flash_deberta_attention,
                                             flash_deberta_attention_fused, unit_steps)
from kernels.fused_layernorm import fused_add_layernorm, fused_layernorm
from kernels.packing import pad_packed, read_metadata, seq_metadata, unpad_packed


@dataclass
class DebertaLayerWeights:
    wqkv: torch.Tensor   # [3 * hidden, hidden]: query_proj, key_proj, value_proj rows
    bqkv: torch.Tensor   # [3 * hidden]
    wo: torch.Tensor     # attention.output.dense [hidden, hidden]
    bo: torch.Tensor
    ln1_w: torch.Tensor  # attention.output.LayerNorm
    ln1_b: torch.Tensor
    wi: torch.Tensor     # intermediate.dense [inter, hidden]
    bi: torch.Tensor
    wo2: torch.Tensor    # output.dense [hidden, inter]
    bo2: torch.Tensor
    ln2_w: torch.Tensor  # output.LayerNorm
    ln2_b: torch.Tensor


@dataclass
class DebertaWeights:
    hidden: int
    heads: int
    inter: int
    rel_emb: torch.Tensor     # rel_embeddings.weight [2 * att_span, hidden]
    rel_ln_w: torch.Tensor    # encoder.LayerNorm (norm_rel_ebd = layer_norm)
    rel_ln_b: torch.Tensor
    layers: List[DebertaLayerWeights] = field(default_factory=list)
    position_buckets: int = 256
    max_relative_positions: int = 512
    eps: float = 1e-7

    def to(self, device=None, dtype=None) -> "DebertaWeights":
        def mv(t):
            return t.to(device=device, dtype=dtype)
        return DebertaWeights(
            self.hidden, self.heads, self.inter, mv(self.rel_emb), mv(self.rel_ln_w),
            mv(self.rel_ln_b),
            [DebertaLayerWeights(*(mv(getattr(l, f)) for f in DebertaLayerWeights.__dataclass_fields__))
             for l in self.layers],
            self.position_buckets, self.max_relative_positions, self.eps)


def random_weights(num_layers: int = 24, hidden: int = 1024, heads: int = 16, inter: int = 4096,
                   position_buckets: int = 256, seed: int = 1003, std: float = 0.02,
                   dtype=torch.bfloat16) -> DebertaWeights:
    """DeBERTa-v3-large shapes, random-init ~ N(0, std) (CPU, seeded);
    LayerNorm weights 1 + N(0, std), biases N(0, std)."""
    g = torch.Generator().manual_seed(seed)

    def rnd(*shape):
        return (torch.randn(*shape, generator=g) * std).to(dtype)

    def ln():
        return (1.0 + torch.randn(hidden, generator=g) * std).to(dtype), rnd(hidden)

    layers = []
    for _ in range(num_layers):
        wqkv, bqkv = rnd(3 * hidden, hidden), rnd(3 * hidden)
        wo, bo = rnd(hidden, hidden), rnd(hidden)
        ln1 = ln()
        wi, bi = rnd(inter, hidden), rnd(inter)
        wo2, bo2 = rnd(hidden, inter), rnd(hidden)
        layers.append(DebertaLayerWeights(wqkv, bqkv, wo, bo, *ln1, wi, bi, wo2, bo2, *ln()))
    rel = rnd(2 * position_buckets, hidden)
    return DebertaWeights(hidden, heads, inter, rel, *ln(), layers, position_buckets)


def deberta_rel_embeddings(w: DebertaWeights) -> torch.Tensor:
    """LayerNorm(rel_embeddings.weight) (deberta_v2_encoder.py:770-774)."""
    return fused_layernorm(w.rel_emb, w.hidden, w.rel_ln_w, w.rel_ln_b, w.eps)


def _rel_pair_chunk_major(pr: torch.Tensor, span: int):
    """(query_rel, key_rel) of the relative table's projection pr [2S, 2, H,
    64] (query_proj rows, key_proj rows) in the fused kernels' chunk-major
    layout [H, 8, 2S, 8], with one copy for both tables."""
    H = pr.shape[2]
    t = pr.view(2 * span, 2, H, 8, 8).permute(1, 2, 3, 0, 4).contiguous()
    return t[0], t[1]


def _dense_ln_fits(wt: torch.Tensor) -> bool:
    """Where the fused dense + residual + LayerNorm kernel is used: widths N
    up to 768 with K <= N (the attention output's square projection of the
    base-size models), where it beats the library GEMM plus the LayerNorm
    pass by ~11 us per layer at B=32, L=512. At N = 1024 the two take the same
    time, and for the FFN output (K = 4 N) the library GEMM is faster."""
    N, K = wt.shape
    return (wt.dtype in (torch.bfloat16, torch.float16) and N in (256, 512, 768)
            and K % 64 == 0 and K <= N)


def _attn_output(ctx: torch.Tensor, x: torch.Tensor, lw, eps: float,
                 fuse: bool = True) -> torch.Tensor:
    """attention.output (deberta_v2_encoder.py:504-508): LayerNorm(dense(ctx) +
    x) over [..., hidden], in one kernel when the shape allows it."""
    if fuse and _dense_ln_fits(lw.wo):
        # the packed copy is made once per weight tensor and version
        return dense_add_layernorm(ctx, None, lw.bo, x, lw.ln1_w, lw.ln1_b, eps,
                                   packed_weight=packed_weight(lw.wo))
    return fused_add_layernorm(F.linear(ctx, lw.wo, lw.bo), x, lw.ln1_w, lw.ln1_b, eps,
                               return_sum=False)


def deberta_layer_forward(x: torch.Tensor, seq_lengths: torch.Tensor, rel: torch.Tensor,
                          lw: DebertaLayerWeights, w: DebertaWeights,
                          fuse_dense_ln: bool = True) -> torch.Tensor:
    """One DebertaV2Layer on x [B, L, hidden]; seq_lengths int32 [B] on the
    device; rel = deberta_rel_embeddings(w). fuse_dense_ln: the attention
    output's dense + residual + LayerNorm in one kernel where the shape
    allows it (_dense_ln_fits); False keeps the GEMM and the LayerNorm pass."""
    B, L, D = x.shape
    H = w.heads
    d = D // H
    span = w.position_buckets if w.position_buckets > 0 else w.max_relative_positions
    qkv = F.linear(x, lw.wqkv, lw.bqkv).view(B, L, 3, H, d)
    q, k, v = (qkv[:, :, i].transpose(1, 2) for i in range(3))
    # query_proj / key_proj of the relative table in one GEMM: [2S, 2, H, d]
    pr = F.linear(rel[:2 * span], lw.wqkv[:2 * D], lw.bqkv[:2 * D]).view(2 * span, 2, H, d)
    query_rel, key_rel = pr[:, 0].transpose(0, 1), pr[:, 1].transpose(0, 1)
    ctx = torch.empty(B, L, H, d, dtype=x.dtype, device=x.device)
    pb = w.position_buckets if w.position_buckets > 0 else span
    log = w.position_buckets > 0
    sm = 1.0 / math.sqrt(3 * d)
    if unit_steps(pb, w.max_relative_positions, log, L):
        query_cm, key_cm = _rel_pair_chunk_major(pr, span)
        flash_deberta_attention_fused(q, k, v, seq_lengths, key_cm, query_cm, sm, pb,
                                      w.max_relative_positions, log, out=ctx.transpose(1, 2))
    else:
        # bucket steps above 1: the reference interface with materialised
        # pos_key = q key_rel^T, pos_query = k query_rel^T (:275-286)
        pos_key = torch.matmul(q, key_rel.transpose(-1, -2).contiguous().unsqueeze(0))
        pos_query = torch.matmul(k, query_rel.transpose(-1, -2).contiguous().unsqueeze(0))
        ctx.copy_(flash_deberta_attention(q, k, v, seq_lengths, pos_key, pos_query, False, sm, pb,
                                          w.max_relative_positions, log).transpose(1, 2))
    h = _attn_output(ctx.view(B, L, D), x, lw, w.eps, fuse_dense_ln)
    inter = activation(F.linear(h, lw.wi, lw.bi), "gelu")
    return fused_add_layernorm(F.linear(inter, lw.wo2, lw.bo2), h, lw.ln2_w, lw.ln2_b, w.eps,
                               return_sum=False)


def deberta_layer_packed(x: torch.Tensor, cu_seqlens: torch.Tensor, max_len: int,
                         rel: torch.Tensor, lw: DebertaLayerWeights,
                         w: DebertaWeights, fuse_dense_ln: bool = True) -> torch.Tensor:
    """deberta_layer_forward on packed sequences, without padding: x [T,
    hidden], sequence s owns rows cu_seqlens[s] .. cu_seqlens[s + 1] - 1
    (int32 on the device), max_len >= every sequence length. The projections,
    LayerNorms and FFN run on the T rows; the attention runs over the packed
    sequences (flash_deberta_attention_varlen), which needs unit bucket steps
    (`unit_steps`, true for the DeBERTa-v3 settings)."""
    from kernels.flash_deberta_attention import flash_deberta_attention_varlen
    T, D = x.shape
    H = w.heads
    d = D // H
    span = w.position_buckets if w.position_buckets > 0 else w.max_relative_positions
    qkv = F.linear(x, lw.wqkv, lw.bqkv).view(T, 3, H, d)
    pr = F.linear(rel[:2 * span], lw.wqkv[:2 * D], lw.bqkv[:2 * D]).view(2 * span, 2, H, d)
    query_cm, key_cm = _rel_pair_chunk_major(pr, span)
    pb = w.position_buckets if w.position_buckets > 0 else span
    log = w.position_buckets > 0
    ctx = flash_deberta_attention_varlen(qkv[:, 0], qkv[:, 1], qkv[:, 2], cu_seqlens, max_len,
                                         key_cm, query_cm, 1.0 / math.sqrt(3 * d), pb,
                                         w.max_relative_positions, log)
    h = _attn_output(ctx.view(T, D), x, lw, w.eps, fuse_dense_ln)
    inter = activation(F.linear(h, lw.wi, lw.bi), "gelu")
    return fused_add_layernorm(F.linear(inter, lw.wo2, lw.bo2), h, lw.ln2_w, lw.ln2_b, w.eps,
                               return_sum=False)


def deberta_forward(x: torch.Tensor, seq_lengths: torch.Tensor, w: DebertaWeights,
                    num_layers: Optional[int] = None) -> torch.Tensor:
    """Encoder stack on embedding output x [B, L, hidden] -> last hidden state."""
    rel = deberta_rel_embeddings(w)
    n = len(w.layers) if num_layers is None else num_layers
    for i in range(n):
        x = deberta_layer_forward(x, seq_lengths, rel, w.layers[i], w)
    return x



# ---------------------------------------------------------------------------
# DeBERTa v1 (linear relative positions)
# ---------------------------------------------------------------------------
@dataclass
class DebertaV1LayerWeights:
    in_proj: torch.Tensor     # [3 * hidden, hidden], rows per head: q, k, v (no bias)
    q_bias: torch.Tensor      # [hidden]
    v_bias: torch.Tensor      # [hidden]
    pos_proj: torch.Tensor    # [hidden, hidden] (c2p, no bias)
    pos_q_proj: torch.Tensor  # [hidden, hidden] (p2c)
    pos_q_bias: torch.Tensor  # [hidden]
    wo: torch.Tensor
    bo: torch.Tensor
    ln1_w: torch.Tensor
    ln1_b: torch.Tensor
    wi: torch.Tensor
    bi: torch.Tensor
    wo2: torch.Tensor
    bo2: torch.Tensor
    ln2_w: torch.Tensor
    ln2_b: torch.Tensor


@dataclass
class DebertaV1Weights:
    hidden: int
    heads: int
    inter: int
    rel_emb: torch.Tensor     # encoder.rel_embeddings.weight [2 * max_rel, hidden]
    layers: List[DebertaV1LayerWeights] = field(default_factory=list)
    max_relative_positions: int = 512
    eps: float = 1e-7

    def to(self, device=None, dtype=None) -> "DebertaV1Weights":
        def mv(t):
            return t.to(device=device, dtype=dtype)
        return DebertaV1Weights(
            self.hidden, self.heads, self.inter, mv(self.rel_emb),
            [DebertaV1LayerWeights(*(mv(getattr(l, f))
                                     for f in DebertaV1LayerWeights.__dataclass_fields__))
             for l in self.layers],
            self.max_relative_positions, self.eps)


def random_weights_v1(num_layers: int = 12, hidden: int = 768, heads: int = 12, inter: int = 3072,
                      max_relative_positions: int = 512, seed: int = 1013, std: float = 0.02,
                      dtype=torch.bfloat16) -> DebertaV1Weights:
    """DeBERTa-base (v1) shapes, random-init ~ N(0, std) (CPU, seeded);
    LayerNorm weights 1 + N(0, std), biases N(0, std)."""
    g = torch.Generator().manual_seed(seed)

    def rnd(*shape):
        return (torch.randn(*shape, generator=g) * std).to(dtype)

    def ln():
        return (1.0 + torch.randn(hidden, generator=g) * std).to(dtype), rnd(hidden)

    layers = []
    for _ in range(num_layers):
        att = (rnd(3 * hidden, hidden), rnd(hidden), rnd(hidden), rnd(hidden, hidden),
               rnd(hidden, hidden), rnd(hidden))
        wo, bo = rnd(hidden, hidden), rnd(hidden)
        ln1 = ln()
        wi, bi = rnd(inter, hidden), rnd(inter)
        wo2, bo2 = rnd(hidden, inter), rnd(hidden)
        layers.append(DebertaV1LayerWeights(*att, wo, bo, *ln1, wi, bi, wo2, bo2, *ln()))
    rel = rnd(2 * max_relative_positions, hidden)
    return DebertaV1Weights(hidden, heads, inter, rel, layers, max_relative_positions)


def deberta_v1_layer_forward(x: torch.Tensor, seq_lengths: torch.Tensor,
                             lw: DebertaV1LayerWeights, w: DebertaV1Weights,
                             fuse_dense_ln: bool = True) -> torch.Tensor:
    """One DeBERTa v1 DebertaLayer (models/deberta/deberta_encoder.py:528-548) on
    x [B, L, hidden] with seq_lengths int32 [B] on the device: in_proj (rows
    per head q, k, v) with q_bias / v_bias folded into the GEMM's bias, the
    linear-position disentangled attention of :246-309 (att_span =
    min(L, max_relative_positions), pos_proj / pos_q_proj applied to the
    [2 span, hidden] slice of the relative table, projections computed in the
    attention kernel), then the post-LN blocks (:445-526; DebertaLayerNorm,
    eps inside the square root, as LayerNorm)."""
    B, L, D = x.shape
    H = w.heads
    d = D // H
    mr = w.max_relative_positions
    span = min(L, mr)
    zero = torch.zeros_like(lw.q_bias).view(H, 1, d)
    b_in = torch.cat([lw.q_bias.view(H, 1, d), zero, lw.v_bias.view(H, 1, d)], 1).reshape(-1)
    qkv = F.linear(x, lw.in_proj, b_in).view(B, L, H, 3, d)
    q, k, v = (qkv[:, :, :, i].transpose(1, 2) for i in range(3))
    rel = w.rel_emb[mr - span:mr + span]
    key_rel = F.linear(rel, lw.pos_proj).view(2 * span, H, d).transpose(0, 1)
    query_rel = F.linear(rel, lw.pos_q_proj, lw.pos_q_bias).view(2 * span, H, d).transpose(0, 1)
    ctx = torch.empty(B, L, H, d, dtype=x.dtype, device=x.device)
    flash_deberta_attention_fused(q, k, v, seq_lengths, key_rel, query_rel, 1.0 / math.sqrt(3 * d),
                                  span, mr, False, out=ctx.transpose(1, 2))
    h = _attn_output(ctx.view(B, L, D), x, lw, w.eps, fuse_dense_ln)
    inter = activation(F.linear(h, lw.wi, lw.bi), "gelu")
    return fused_add_layernorm(F.linear(inter, lw.wo2, lw.bo2), h, lw.ln2_w, lw.ln2_b, w.eps,
                               return_sum=False)


def deberta_v1_forward(x: torch.Tensor, seq_lengths: torch.Tensor, w: DebertaV1Weights,
                       num_layers: Optional[int] = None) -> torch.Tensor:
    """DeBERTa v1 encoder stack (deberta_encoder.py:645-697) on embedding output
    x [B, L, hidden] -> last hidden state."""
    n = len(w.layers) if num_layers is None else num_layers
    for i in range(n):
        x = deberta_v1_layer_forward(x, seq_lengths, w.layers[i], w)
    return x


def deberta_forward_flat(x: torch.Tensor, positions: torch.Tensor, w: DebertaWeights,
                         num_layers: Optional[int] = None) -> torch.Tensor:
    """The GLiNER plugins' flat call (plugins/deberta_gliner/model.py:166-202; the
    GLiNER2 plugin, plugins/deberta_gliner2/model.py:124-137, runs the flat
    stream as one sequence and gets per-sequence attention from this path):
    embedding output x [T, hidden] of a packed stream whose sequences start at
    position 0 -> last hidden state [T, hidden]. The sequence boundaries come
    from the positions on the device; the number of sequences and the longest
    length are read back once. Every layer then runs on the packed rows
    (deberta_layer_packed); bucket settings with steps above 1 re-pad into the
    padded forward instead."""
    cu, meta = seq_metadata(positions, "zero")
    cu, n, max_len, _ = read_metadata(cu, meta)
    pb = w.position_buckets if w.position_buckets > 0 else w.max_relative_positions
    if unit_steps(pb, w.max_relative_positions, w.position_buckets > 0, max_len):
        # every layer on the packed rows (varlen attention, no padding)
        rel = deberta_rel_embeddings(w)
        nl = len(w.layers) if num_layers is None else num_layers
        for i in range(nl):
            x = deberta_layer_packed(x, cu, max_len, rel, w.layers[i], w)
        return x
    xb, lens = pad_packed(x, cu, n, max_len)
    return unpad_packed(deberta_forward(xb, lens, w, num_layers), cu, x.shape[0])
