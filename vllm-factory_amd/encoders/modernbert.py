"""ModernBERT encoder forward on the packed (varlen) stream.

Follows models/modernbert/modernbert_encoder.py (embeddings :102-128, layer
:289-352, model :430-480): tok_embeddings -> LayerNorm; 22 x [attn_norm
(Identity in layer 0) -> Wqkv -> RoPE attention -> Wo -> + residual ->
mlp_norm -> Wi -> GELU(input) * gate -> Wo -> + residual]; final LayerNorm.
The Wi projection and the GELU gate run as one kernel (glu_linear), which
rounds the GLU output once where the reference rounds the projection first.
Wqkv and the rotary step of k run as one kernel (qkv_rope_projection), which
rotates the fp32 projection sums of k and rounds once; the attention then
reads that rotated k (varlen_rope_attention_krot) with no separate k pass.
Global layers (layer_id % 3 == 0) attend inside each sequence with RoPE theta
160000, local layers within |i - j| <= 64 with theta 10000; tokens with id
50284 are hidden as keys (:456-460).

Differences from the reference, all by construction of the packed path:
sequences are given by cu_seqlens instead of position resets and dense
[T, T] masks; each residual add is fused into the LayerNorm that follows it
(vfk_layernorm_fwd with a residual); a query row that sees no key at all
(every key of its sequence is token 50284) returns zeros where the reference's
finite mask would average over the stream.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import List, Optional

import torch
import torch.nn.functional as F

from kernels.colbert_head import colbert_head
from kernels.dense_layernorm import dense_add_layernorm
from kernels.fused_glu_mlp import fused_gelu_mul_dropout, glu_linear
from kernels.fused_layernorm import fused_add_layernorm, fused_layernorm
from kernels.weight_pack import packed_weight
from kernels.varlen_attention import (qkv_rope_projection, token_positions, varlen_from_positions,
                                      varlen_rope_attention, varlen_rope_attention_krot)

MASK_TOKEN_ID = 50284


@dataclass
class ModernBertLayerWeights:
    wqkv: torch.Tensor       # [3 * hidden, hidden]
    wo: torch.Tensor         # [hidden, hidden]
    wi: torch.Tensor         # [2 * inter, hidden] (input rows, then gate rows)
    wo_mlp: torch.Tensor     # [hidden, inter]
    attn_norm: Optional[torch.Tensor]   # [hidden]; None in layer 0 (Identity)
    mlp_norm: torch.Tensor   # [hidden]


@dataclass
class ModernBertWeights:
    hidden: int
    heads: int
    inter: int
    emb: torch.Tensor        # [vocab, hidden]
    emb_norm: torch.Tensor
    layers: List[ModernBertLayerWeights] = field(default_factory=list)
    final_norm: Optional[torch.Tensor] = None
    global_every: int = 3
    window: int = 64
    theta_global: float = 160000.0
    theta_local: float = 10000.0
    eps: float = 1e-5

    def to(self, device=None, dtype=None) -> "ModernBertWeights":
        def mv(t):
            return None if t is None else t.to(device=device, dtype=dtype)
        return ModernBertWeights(
            self.hidden, self.heads, self.inter, mv(self.emb), mv(self.emb_norm),
            [ModernBertLayerWeights(mv(l.wqkv), mv(l.wo), mv(l.wi), mv(l.wo_mlp), mv(l.attn_norm),
                                    mv(l.mlp_norm)) for l in self.layers],
            mv(self.final_norm), self.global_every, self.window, self.theta_global,
            self.theta_local, self.eps)


def random_weights(num_layers: int = 22, hidden: int = 768, heads: int = 12, inter: int = 1152,
                   vocab: int = 50368, seed: int = 1005, std: float = 0.02,
                   dtype=torch.bfloat16) -> ModernBertWeights:
    """Random-init weights ~ N(0, std) (CPU, seeded), LayerNorm weights 1."""
    g = torch.Generator().manual_seed(seed)

    def rnd(*shape):
        return (torch.randn(*shape, generator=g) * std).to(dtype)

    ones = torch.ones(hidden, dtype=dtype)
    layers = [ModernBertLayerWeights(rnd(3 * hidden, hidden), rnd(hidden, hidden),
                                     rnd(2 * inter, hidden), rnd(hidden, inter),
                                     None if i == 0 else ones.clone(), ones.clone())
              for i in range(num_layers)]
    return ModernBertWeights(hidden, heads, inter, rnd(vocab, hidden), ones.clone(), layers,
                             ones.clone())


def _glu_fusable(wi: torch.Tensor, h: torch.Tensor) -> bool:
    """Whether the Wi projection and GELU gate run as one kernel (glu_linear:
    16-bit weights, hidden a multiple of 64, intermediate of 8)."""
    return (wi.dtype in (torch.bfloat16, torch.float16) and h.dtype == wi.dtype
            and wi.shape[1] % 64 == 0 and (wi.shape[0] // 2) % 8 == 0)


def _qkv_fusable(wqkv: torch.Tensor, h: torch.Tensor, head_dim: int) -> bool:
    """Whether the Wqkv projection and the rotary step of k run as one kernel
    (qkv_rope_projection: 16-bit weights, head_dim 64, hidden a multiple of
    64)."""
    return (wqkv.dtype in (torch.bfloat16, torch.float16) and h.dtype == wqkv.dtype
            and head_dim == 64 and wqkv.shape[1] % 64 == 0 and h.dim() == 2)


def _dense_ln_fusable(wo: torch.Tensor) -> bool:
    """Wo + residual + mlp_norm as one kernel (dense_add_layernorm with the sum
    output): 16-bit weights, a square projection of width 256..1024."""
    N, K = wo.shape
    return wo.dtype in (torch.bfloat16, torch.float16) and N == K and N in (256, 512, 768, 1024)


def _encode(ids: torch.Tensor, cu_seqlens: torch.Tensor, max_seqlen: int, w: ModernBertWeights,
            num_layers: Optional[int], fuse_qkv_rope: bool = False, fuse_dense_ln: bool = False):
    """Embeddings and layers; returns (pending MLP output or None, residual
    stream) before the final LayerNorm. fuse_qkv_rope: Wqkv and the k rotation
    as one kernel (qkv_rope_projection) where the weights allow it; off by
    default, since hipBLASLt plus the k pass measures about 5 % faster per
    layer at 163 736 tokens. fuse_dense_ln: the attention output's Wo, residual add
    and mlp_norm as one kernel (dense_add_layernorm, which also writes the
    new residual stream) where _dense_ln_fusable allows it; off by default:
    the 22-layer forward at 163 736 tokens takes 52.21 ms with it and
    52.25-52.33 ms without, within the run-to-run spread."""
    T = ids.shape[0]
    d = w.hidden // w.heads
    key_valid = ids != MASK_TOKEN_ID
    x = fused_layernorm(w.emb[ids], w.hidden, w.emb_norm, None, w.eps)
    pending = None  # MLP output not yet added to the residual stream x
    n = len(w.layers) if num_layers is None else num_layers
    positions = None  # rotary position of each token, for the fused q | k | v projection
    for i in range(n):
        lw = w.layers[i]
        if pending is None:
            h = x if lw.attn_norm is None else fused_layernorm(x, w.hidden, lw.attn_norm, None, w.eps)
        else:
            h, x = fused_add_layernorm(pending, x, lw.attn_norm, None, w.eps)
        is_global = i % w.global_every == 0
        window = -1 if is_global else w.window
        theta = w.theta_global if is_global else w.theta_local
        if fuse_qkv_rope and _qkv_fusable(lw.wqkv, h, d):
            # Wqkv with the rotary step of k in the GEMM epilogue; the attention
            # reads the rotated k from its workspace (no k pass)
            if positions is None:
                positions = token_positions(cu_seqlens, T)
            res = qkv_rope_projection(h, lw.wqkv, w.heads, positions, max_seqlen, theta,
                                      1.0 / math.sqrt(d))
            att = varlen_rope_attention_krot(res, cu_seqlens, max_seqlen, window, key_valid)
        else:
            qkv = F.linear(h, lw.wqkv).view(T, 3, w.heads, d)
            att = varlen_rope_attention(qkv[:, 0], qkv[:, 1], qkv[:, 2], cu_seqlens, max_seqlen,
                                        window, theta, 1.0 / math.sqrt(d), key_valid)
        if fuse_dense_ln and _dense_ln_fusable(lw.wo):
            h, x = dense_add_layernorm(att.view(T, w.hidden), None, None, x, lw.mlp_norm, None,
                                       w.eps, packed_weight=packed_weight(lw.wo), return_sum=True)
        else:
            o = F.linear(att.view(T, w.hidden), lw.wo)
            h, x = fused_add_layernorm(o, x, lw.mlp_norm, None, w.eps)
        if _glu_fusable(lw.wi, h):
            g = glu_linear(h, lw.wi, "gelu")
        else:
            y = F.linear(h, lw.wi)
            g = fused_gelu_mul_dropout(y[:, :w.inter], y[:, w.inter:], "gelu")
        pending = F.linear(g, lw.wo_mlp)
    return pending, x


def modernbert_forward(ids: torch.Tensor, cu_seqlens: torch.Tensor, max_seqlen: int,
                       w: ModernBertWeights, num_layers: Optional[int] = None,
                       fuse_qkv_rope: bool = False, fuse_dense_ln: bool = False) -> torch.Tensor:
    """ids [T] (device, int64), cu_seqlens int32 [n + 1] -> last hidden state [T, hidden]."""
    pending, x = _encode(ids, cu_seqlens, max_seqlen, w, num_layers, fuse_qkv_rope, fuse_dense_ln)
    if pending is None:
        return fused_layernorm(x, w.hidden, w.final_norm, None, w.eps)
    out, _ = fused_add_layernorm(pending, x, w.final_norm, None, w.eps)
    return out


def modernbert_colbert_forward(ids: torch.Tensor, cu_seqlens: torch.Tensor, max_seqlen: int,
                               w: ModernBertWeights, proj_weight: torch.Tensor,
                               proj_bias: Optional[torch.Tensor] = None,
                               num_layers: Optional[int] = None) -> torch.Tensor:
    """ModernBERT + ColBERT head (plugins/moderncolbert/model.py:220-267 with a
    single Dense layer): the last residual add, the final LayerNorm, the
    projection [colbert_dim, hidden] and the L2 normalisation in one kernel
    (kernels.colbert_head). Returns [T, colbert_dim] unit-norm embeddings."""
    pending, x = _encode(ids, cu_seqlens, max_seqlen, w, num_layers)
    return colbert_head(x, proj_weight, proj_bias, w.final_norm, None, w.eps, residual=pending)


def modernbert_forward_positions(input_ids: torch.Tensor, position_ids: torch.Tensor,
                                 w: ModernBertWeights,
                                 num_layers: Optional[int] = None) -> torch.Tensor:
    """The reference's flat vLLM call (models/modernbert/modernbert_encoder.py:430-480:
    input_ids and position_ids of the packed stream): sequence boundaries come
    from the position resets on the device (varlen_from_positions) instead of
    [T, T] masks."""
    cu, max_len = varlen_from_positions(position_ids)
    return modernbert_forward(input_ids.reshape(-1), cu, max_len, w, num_layers)
