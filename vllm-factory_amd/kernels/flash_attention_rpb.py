"""T5 relative-position-bias flash attention on gfx950.

Drop-in for kernels/flash_attention_rpb.py:296-412 (`flash_attention_rpb_final`):
same signature, defaults and return value (a new tensor shaped like `q`).
Buckets follow the eager formula of models/mt5/mt5_encoder.py:124-148
bit-exactly; the bias table keeps the HF [num_buckets, num_heads] layout
(mt5_encoder.py:546-566) and any strides.
"""
from __future__ import annotations

from typing import Optional

import torch

from . import _lib


def flash_attention_rpb_final(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    rpb_table: Optional[torch.Tensor],
    num_buckets: int,
    max_distance: int,
    is_decoder: bool,
    padding_mask: Optional[torch.Tensor] = None,
    dropout_p: float = 0.0,
    softmax_scale: float = 1.0,
    use_autotune: bool = True,
    out: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """out = softmax(q k^T * softmax_scale + rpb[bucket(k - q)] + padding_mask) v.

    q [B,H,Lq,D], k/v [B,H,Lk,D] (D = 64, any strides); padding_mask is an
    additive mask broadcastable to [B,H,Lq,Lk] (typically [B,1,1,Lk]).
    `use_autotune` is accepted for signature compatibility; tiles are fixed.
    `out` (an addition to the reference's signature): a [B,H,Lq,D] tensor of
    q's dtype with a contiguous last dim and 16-byte aligned rows, written in
    place (e.g. a [B,Lq,H,D] buffer viewed through transpose(1, 2)).
    """
    if dropout_p != 0.0:
        raise NotImplementedError("flash_attention_rpb_final: dropout is not supported (inference only)")
    dev = _lib.require_gpu(q, k, v, rpb_table, padding_mask)
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError("q, k, v must be 4-D [B, H, L, D]")
    if k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError("q, k, v must share a dtype")
    qq, kk, vv = (_lib.rows_aligned(t) for t in (q, k, v))
    if out is None:
        out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    elif out.shape != q.shape or out.dtype != q.dtype or out.device != q.device:
        raise ValueError("out must match q's shape, dtype and device")
    mask = padding_mask
    if mask is not None:
        while mask.dim() < 4:
            mask = mask.unsqueeze(0)
    _lib.on_device(
        "vfk_flash_rpb_fwd", dev,
        _lib.ref(_lib.desc(qq)), _lib.ref(_lib.desc(kk)), _lib.ref(_lib.desc(vv)),
        _lib.ref(_lib.desc(rpb_table)),
        int(num_buckets), int(max_distance), int(bool(is_decoder)),
        _lib.ref(_lib.desc(mask)), float(softmax_scale),
        _lib.ref(_lib.desc(out)),
    )
    return out



def flash_attention_rpb_varlen(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    cu_seqlens: torch.Tensor,
    max_seqlen: int,
    rpb_table: Optional[torch.Tensor],
    num_buckets: int,
    max_distance: int,
    is_decoder: bool = False,
    softmax_scale: float = 1.0,
    out: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """flash_attention_rpb_final over packed sequences, without padding.

    q, k, v [T, H, 64] (bf16 / fp16, any token and head strides with a
    contiguous last dim); sequence s is rows cu_seqlens[s] .. cu_seqlens[s+1]
    - 1 (int32 on the device) and attends to its own rows only, relative
    positions counted inside the sequence. Equals the padded call with the
    reference's [B, 1, 1, L] key mask on the valid rows. max_seqlen must be
    >= every sequence length. Returns [T, H, 64] (or writes `out`)."""
    dev = _lib.require_gpu(q, k, v, cu_seqlens, rpb_table)
    if q.dim() != 3 or k.shape != q.shape or v.shape != q.shape:
        raise ValueError("q, k, v must be [T, H, D] of one shape")
    if k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError("q, k, v must share a dtype")
    qq, kk, vv = (_lib.rows_aligned(t) for t in (q, k, v))
    if out is None:
        out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    elif out.shape != q.shape or out.dtype != q.dtype or out.device != q.device:
        raise ValueError("out must match q's shape, dtype and device")
    cu = cu_seqlens.to(torch.int32).contiguous()
    _lib.on_device(
        "vfk_flash_rpb_varlen_fwd", dev,
        _lib.ref(_lib.desc(qq)), _lib.ref(_lib.desc(kk)), _lib.ref(_lib.desc(vv)),
        cu.data_ptr(), int(cu.numel() - 1), int(max_seqlen),
        _lib.ref(_lib.desc(rpb_table)), int(num_buckets), int(max_distance), int(bool(is_decoder)),
        float(softmax_scale), _lib.ref(_lib.desc(out)),
    )
    return out
