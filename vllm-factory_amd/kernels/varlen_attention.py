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
from typing import Dict, NamedTuple, Optional, Tuple

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


def token_positions(cu_seqlens: torch.Tensor, total_tokens: int) -> torch.Tensor:
    """int32 [T]: t - cu_seqlens[s] for token t of sequence s (the rotary
    position varlen_rope_attention gives it), computed on the device."""
    t = torch.arange(total_tokens, dtype=torch.int32, device=cu_seqlens.device)
    s = torch.searchsorted(cu_seqlens[1:].contiguous(), t, right=True)
    return (t - cu_seqlens.index_select(0, s)).to(torch.int32)


class RotatedQKV(NamedTuple):
    """Output of qkv_rope_projection: q and v [T, H, 64] as projected, and the
    workspace holding k rotated, scaled by softmax_scale * log2(e) and laid out
    head-major, with per-head norm bounds of each 32-token block."""
    q: torch.Tensor
    v: torch.Tensor
    krot: torch.Tensor
    rope_theta: float
    softmax_scale: float


def qkv_rope_projection(x: torch.Tensor, wqkv: torch.Tensor, num_heads: int,
                        positions: torch.Tensor, max_seqlen: int, rope_theta: float,
                        softmax_scale: Optional[float] = None) -> RotatedQKV:
    """The Wqkv linear of models/modernbert/modernbert_encoder.py:236-242 with the
    rotary step of k in the GEMM epilogue (vfk_qkv_rope_linear_fwd): x [T, K],
    wqkv [3 H 64, K] (q, k, v rows) in bf16 / fp16, positions int32 [T] (the
    rotary position of each token, < max_seqlen). The projection sums stay in
    fp32 through the rotation and are rounded once. Use the result with
    varlen_rope_attention_krot."""
    dev = _lib.require_gpu(x, wqkv, positions)
    T, K = x.shape
    if wqkv.shape != (3 * num_heads * 64, K) or wqkv.dtype != x.dtype:
        raise ValueError(f"qkv_rope_projection: wqkv must be [{3 * num_heads * 64}, {K}] {x.dtype}")
    if positions.dtype != torch.int32 or positions.shape != (T,):
        raise ValueError("qkv_rope_projection: positions must be int32 [T]")
    scale = softmax_scale if softmax_scale is not None else 1.0 / math.sqrt(64)
    tab = rope_table(rope_theta, int(max_seqlen), dev)
    x2 = _lib.rows_aligned(x)
    w2 = _lib.rows_aligned(wqkv)
    q = torch.empty(T, num_heads, 64, dtype=x.dtype, device=x.device)
    v = torch.empty_like(q)
    ws_bytes = int(_lib.load().vfk_qkv_rope_workspace_bytes(int(T), int(num_heads)))
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=x.device)
    _lib.on_device("vfk_qkv_rope_linear_fwd", dev, _lib.ref(_lib.desc(x2)), _lib.ref(_lib.desc(w2)),
                   positions.contiguous().data_ptr(), tab.data_ptr(), int(tab.shape[0]),
                   int(num_heads), float(scale), _lib.ref(_lib.desc(q)), _lib.ref(_lib.desc(v)),
                   ws.data_ptr(), ws_bytes)
    return RotatedQKV(q, v, ws, float(rope_theta), float(scale))


def varlen_rope_attention_krot(qkv: RotatedQKV, cu_seqlens: torch.Tensor, max_seqlen: int,
                               window: int = -1, key_valid: Optional[torch.Tensor] = None,
                               out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """varlen_rope_attention for the output of qkv_rope_projection (k already
    rotated: no k pass); positions t - cu_seqlens[s] must be the ones the
    projection was given. Returns [T, H, 64]."""
    q, v = qkv.q, qkv.v
    dev = _lib.require_gpu(q, v, qkv.krot, cu_seqlens, key_valid)
    if cu_seqlens.dtype != torch.int32 or cu_seqlens.dim() != 1:
        raise ValueError("cu_seqlens must be a 1-D int32 tensor")
    if not cu_seqlens.is_contiguous():
        cu_seqlens = cu_seqlens.contiguous()
    if out is None:
        out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    kv_ptr = None
    if key_valid is not None:
        if key_valid.numel() != q.shape[0]:
            raise ValueError("key_valid must have one entry per token")
        key_valid = key_valid.to(torch.uint8).contiguous()
        kv_ptr = key_valid.data_ptr()
    tab = rope_table(qkv.rope_theta, int(max_seqlen), dev)
    _lib.on_device(
        "vfk_varlen_attn_krot_fwd", dev, _lib.ref(_lib.desc(q)), _lib.ref(_lib.desc(v)),
        qkv.krot.data_ptr(), int(qkv.krot.numel()), cu_seqlens.data_ptr(),
        int(cu_seqlens.numel() - 1), int(max_seqlen), int(window), tab.data_ptr(),
        int(tab.shape[0]), kv_ptr, float(qkv.softmax_scale), _lib.ref(_lib.desc(out)))
    return out
