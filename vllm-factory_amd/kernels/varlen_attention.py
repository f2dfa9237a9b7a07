"""Packed (varlen) local/global attention with in-kernel RoPE, for ModernBERT.

No reference kernel exists for this op: the reference runs
F.scaled_dot_product_attention over the whole packed stream with dense [T, T]
block-diagonal and sliding-window masks
(models/modernbert/modernbert_encoder.py:236-255, :491-550). This op computes
the same attention per sequence from cu_seqlens:

  * token t of sequence s has position t - cu_seqlens[s] (positions restart at
    0 per sequence, which is what the reference's block mask keys on);
  * window < 0: global layer; window = w: key j visible iff |i - j| <= w
    (ModernBERT local layers use w = local_attention // 2 = 64);
  * rope_theta > 0: q and k are rotated with the HF ModernBertRotaryEmbedding
    frequencies (non-interleaved halves): k once by a pre-pass into a
    workspace, q inside the attention kernel (inputs are never written);
  * key_valid[t] == 0 hides key t (the reference's token-id 50284 mask).

Rows that see no key at all are returned as zeros.
"""
from __future__ import annotations

import math
from typing import Dict, Optional, Tuple

import torch

from . import _lib
from .packing import seq_metadata, varlen_from_positions  # noqa: F401  (re-exported)

_ROPE_TABLES: Dict[Tuple[float, int, torch.device], torch.Tensor] = {}


def rope_table(theta: float, positions: int, device: torch.device) -> torch.Tensor:
    """fp32 [positions, 32, 2] (cos, sin) table of the HF rotary embedding
    (vfk_rope_table), cached per (theta, size bucket, device) the way the HF
    rotary module caches its tables."""
    n = max(256, 1 << (max(positions, 1) - 1).bit_length())
    key = (float(theta), n, torch.device(device))
    t = _ROPE_TABLES.get(key)
    if t is None:
        t = torch.empty(n, 32, 2, dtype=torch.float32, device=device)
        _lib.on_device("vfk_rope_table", torch.device(device), float(theta), int(n), t.data_ptr())
        _ROPE_TABLES[key] = t
    return t


def varlen_rope_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                          cu_seqlens: torch.Tensor, max_seqlen: int, window: int = -1,
                          rope_theta: float = 0.0, softmax_scale: Optional[float] = None,
                          key_valid: Optional[torch.Tensor] = None,
                          out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """q, k, v: [T, H, 64] (any token/head strides, e.g. views of a fused qkv
    projection); cu_seqlens: int32 [num_seqs + 1] on the device. Returns [T, H, 64]."""
    dev = _lib.require_gpu(q, k, v, cu_seqlens, key_valid)
    if q.dim() != 3 or k.shape != q.shape or v.shape != q.shape:
        raise ValueError("q, k, v must all be [T, H, D]")
    if cu_seqlens.dtype != torch.int32 or cu_seqlens.dim() != 1:
        raise ValueError("cu_seqlens must be a 1-D int32 tensor")
    if not cu_seqlens.is_contiguous():
        cu_seqlens = cu_seqlens.contiguous()
    qq, kk, vv = (_lib.rows_aligned(t) for t in (q, k, v))
    if out is None:
        out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    kv_ptr = None
    if key_valid is not None:
        if key_valid.numel() != q.shape[0]:
            raise ValueError("key_valid must have one entry per token")
        key_valid = key_valid.to(torch.uint8).contiguous()
        kv_ptr = key_valid.data_ptr()
    scale = softmax_scale if softmax_scale is not None else 1.0 / math.sqrt(q.shape[-1])
    tab_ptr, tab_n = None, 0
    rope = bool(rope_theta and rope_theta > 0)
    if rope:
        tab = rope_table(rope_theta, int(max_seqlen), dev)
        tab_ptr, tab_n = tab.data_ptr(), tab.shape[0]
    ws_bytes = int(_lib.load().vfk_varlen_attn_workspace_bytes(
        _lib.dtype_code(q.dtype), int(q.shape[0]), int(q.shape[1]), int(rope),
        int(cu_seqlens.numel() - 1), int(max_seqlen)))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device) if ws_bytes else None
    _lib.on_device(
        "vfk_varlen_attn_fwd", dev,
        _lib.ref(_lib.desc(qq)), _lib.ref(_lib.desc(kk)), _lib.ref(_lib.desc(vv)),
        cu_seqlens.data_ptr(), int(cu_seqlens.numel() - 1), int(max_seqlen),
        int(window), tab_ptr, int(tab_n), kv_ptr, float(scale),
        ws.data_ptr() if ws is not None else None, ws_bytes,
        _lib.ref(_lib.desc(out)),
    )
    return out
