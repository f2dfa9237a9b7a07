"""Attention restatements (oracle; test infrastructure only).

All three attentions are written as explicit matrix softmax in `dtype`
(default fp32) over dense per-(batch, head) score matrices.

Pinned by (tests/test_oracle_attention.py):
  * zero bias / no mask -> torch.nn.functional.scaled_dot_product_attention (CPU);
  * brute-force Python loops over every (query, key) on tiny inputs;
  * DeBERTa: the gather formulation here == the bmm formulation of the
    model's own _disentangled_att_bias (both restated, compared), and zero
    position projections reduce it to plain attention with scale 1/sqrt(3d);
  * varlen: window >= length equals global; packing order equivariance; RoPE
    cos/sin equal transformers' ModernBertRotaryEmbedding;
  * rows of the probability matrix sum to one (V = ones -> ones);
  * committed vectors tests/golden/attn_*.pt.
"""
from __future__ import annotations

import math
from typing import Optional

import torch

from .buckets import make_log_bucket_position, t5_bucket_matrix


def t5_rpb_bias(rpb_table: torch.Tensor, q_len: int, k_len: int, bidirectional: bool,
                num_buckets: int, max_distance: int) -> torch.Tensor:
    """models/mt5/mt5_encoder.py:150-164: table [num_buckets, H] -> bias [1, H, q, k]."""
    buckets = t5_bucket_matrix(q_len, k_len, bidirectional, num_buckets, max_distance)
    values = rpb_table[buckets]            # (q, k, H) -- nn.Embedding lookup
    return values.permute(2, 0, 1).unsqueeze(0)


def rpb_attention(q, k, v, rpb_table: Optional[torch.Tensor], num_buckets: int,
                  max_distance: int, is_decoder: bool,
                  padding_mask: Optional[torch.Tensor] = None,
                  softmax_scale: float = 1.0, dtype=torch.float32) -> torch.Tensor:
    """T5 self-attention with relative-position bias.

    Eager path: mt5_encoder.py:285-320 (dense bias = RPB + additive padding mask,
    _make_contiguous_additive_bias :75-110, then SDPA with scale=softmax_scale).
    Causal mode (is_decoder) follows the kernel contract of
    kernels/flash_attention_rpb.py:120-124, :176-178 (keys after the query get
    -inf) with unidirectional buckets (:315-321).
    q [B,H,Lq,D], k/v [B,H,Lk,D]. Returns `dtype`.
    """
    q, k, v = (t.to(dtype) for t in (q, k, v))
    Lq, Lk = q.shape[2], k.shape[2]
    s = torch.matmul(q, k.transpose(-1, -2)) * softmax_scale
    if rpb_table is not None:
        s = s + t5_rpb_bias(rpb_table.to(dtype), Lq, Lk, not is_decoder, num_buckets, max_distance)
    if padding_mask is not None:
        s = s + padding_mask.to(dtype)
    if is_decoder:
        causal = torch.ones(Lq, Lk, dtype=torch.bool).triu(1)
        s = s.masked_fill(causal, float("-inf"))
    p = torch.softmax(s, dim=-1)
    return torch.matmul(p, v)


def deberta_flash_attention(q, k, v, seq_lengths=None, pos_key=None, pos_query=None,
                            sm_scale=None, position_buckets=0, max_relative_distance=0,
                            use_log_bucket=False, causal=False, zero_padded_rows=True,
                            dtype=torch.float32) -> torch.Tensor:
    """Disentangled attention with precomputed position projections.

    kernels/flash_deberta_attention.py:375-448 (_pytorch_flash_deberta_fwd):
      attn = q k^T sm + gather(pos_key, c2p) sm + gather(pos_query, p2c)^T sm,
      keys >= seq_len -> -inf, softmax, @ v.
    With zero_padded_rows, query rows >= seq_len are zero as the reference's GPU
    kernel writes them (flash_deberta_attention.py:334, :298-299).
    """
    q, k, v = (t.to(dtype) for t in (q, k, v))
    B, H, M, D = q.shape
    N = k.shape[2]
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(D)
    att_span = position_buckets if position_buckets > 0 else max_relative_distance
    attn = torch.matmul(q, k.transpose(-1, -2)) * sm_scale
    relative_pos = torch.arange(M)[:, None] - torch.arange(N)[None, :]
    if use_log_bucket and position_buckets > 0 and max_relative_distance > 0:
        bucket_pos = make_log_bucket_position(relative_pos, position_buckets, max_relative_distance)
    else:
        bucket_pos = relative_pos.float()
    if pos_key is not None:
        c2p_idx = torch.clamp(bucket_pos + att_span, 0, att_span * 2 - 1).long()
        c2p_idx = c2p_idx.unsqueeze(0).unsqueeze(0).expand(B, H, M, N)
        attn = attn + torch.gather(pos_key.to(dtype), dim=-1, index=c2p_idx) * sm_scale
    if pos_query is not None:
        p2c_idx = torch.clamp(-bucket_pos + att_span, 0, att_span * 2 - 1).long()
        p2c_idx = p2c_idx.unsqueeze(0).unsqueeze(0).expand(B, H, N, N)
        p2c = torch.gather(pos_query.to(dtype), dim=-1, index=p2c_idx)
        attn = attn + p2c.transpose(-1, -2) * sm_scale
    if seq_lengths is not None:
        keep = torch.arange(N)[None, :] < seq_lengths.cpu()[:, None]
        attn = attn.masked_fill(~keep[:, None, None, :], float("-inf"))
    if causal:
        attn = attn.masked_fill(~torch.ones(M, N, dtype=torch.bool).tril(), float("-inf"))
    out = torch.matmul(torch.softmax(attn, dim=-1), v)
    if zero_padded_rows and seq_lengths is not None:
        rows = torch.arange(M)[None, :] < seq_lengths.cpu()[:, None]
        out = out * rows[:, None, :, None].to(dtype)
    return out


def deberta_position_projections(q, k, key_rel, query_rel, dtype=torch.float32):
    """models/deberta_v2/deberta_v2_encoder.py:275-286 (share_att_key):
    pos_key = q @ key_rel^T, pos_query = k @ query_rel^T, key_rel/query_rel
    given per head as [H, 2S, D]."""
    pk = torch.matmul(q.to(dtype), key_rel.to(dtype).unsqueeze(0).transpose(-1, -2))
    pq = torch.matmul(k.to(dtype), query_rel.to(dtype).unsqueeze(0).transpose(-1, -2))
    return pk, pq


def rope_cos_sin(positions: torch.Tensor, theta: float, dim: int = 64):
    """ModernBERT rotary tables in fp32, as transformers' ModernBertRotaryEmbedding
    (default rope) used at models/modernbert/modernbert_encoder.py:236-242:
    inv_freq = 1 / theta^(arange(0, dim, 2)/dim); emb = cat(f, f)."""
    inv_freq = 1.0 / (theta ** (torch.arange(0, dim, 2, dtype=torch.int64).float() / dim))
    freqs = positions.float()[:, None] * inv_freq[None, :]
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos(), emb.sin()


def rotate_half(x):
    """modernbert_encoder.py:277-281."""
    x1 = x[..., : x.shape[-1] // 2]
    x2 = x[..., x.shape[-1] // 2:]
    return torch.cat((-x2, x1), dim=-1)


def apply_rope(x, cos, sin):
    """modernbert_encoder.py:262-275: x * cos + rotate_half(x) * sin (x [..., S, H, D])."""
    return x * cos.unsqueeze(-2) + rotate_half(x) * sin.unsqueeze(-2)


def varlen_attention(q, k, v, cu_seqlens, window: int = -1, rope_theta: float = 0.0,
                     key_valid: Optional[torch.Tensor] = None,
                     softmax_scale: Optional[float] = None, dtype=torch.float32) -> torch.Tensor:
    """ModernBERT attention over a packed stream, one sequence at a time.

    Follows models/modernbert/modernbert_encoder.py:214-260 (Wqkv -> RoPE -> SDPA)
    with the masks of :491-550: keys attend only inside their sequence (position
    resets), key j is hidden when key_valid[j] is False (token id 50284,
    :456-460), and local layers keep |i - j| <= window (:539-549).
    q/k/v [T, H, D]; cu_seqlens [n+1]. Rows that see no key are returned as 0
    (the dense reference would average over the whole packed stream there).
    """
    q, k, v = (t.to(dtype) for t in (q, k, v))
    T, H, D = q.shape
    scale = softmax_scale if softmax_scale is not None else 1.0 / math.sqrt(D)
    out = torch.zeros(T, H, D, dtype=dtype)
    cu = [int(x) for x in cu_seqlens.tolist()]
    for s in range(len(cu) - 1):
        a, b = cu[s], cu[s + 1]
        n = b - a
        if n == 0:
            continue
        qs, ks, vs = q[a:b], k[a:b], v[a:b]
        if rope_theta > 0:
            cos, sin = rope_cos_sin(torch.arange(n), rope_theta, D)
            cos, sin = cos.to(dtype), sin.to(dtype)
            qs, ks = apply_rope(qs, cos, sin), apply_rope(ks, cos, sin)
        sc = torch.einsum("ihd,jhd->hij", qs, ks) * scale
        vis = torch.ones(n, n, dtype=torch.bool)
        if window >= 0:
            idx = torch.arange(n)
            vis &= (idx[:, None] - idx[None, :]).abs() <= window
        if key_valid is not None:
            vis &= key_valid[a:b].bool()[None, :]
        sc = sc.masked_fill(~vis[None], float("-inf"))
        p = torch.softmax(sc, dim=-1)
        p = torch.nan_to_num(p, nan=0.0)  # rows with no visible key
        out[a:b] = torch.einsum("hij,jhd->ihd", p, vs)
    return out
