"""DeBERTa-v2/v3 disentangled flash attention on gfx950.

Drop-in for kernels/flash_deberta_attention.py:455-507: `flash_deberta_attention`
with the same signature, defaults and output convention (a new [B, H, M, D]
tensor whose rows >= seq_lengths[b] are zero), plus `clear_config_cache` and
`HAS_TRITON` (true: the reference's models gate their flash path on it).
Scores follow
    s(i, j) = (q_i.k_j + pos_key[i, c(i-j)] + pos_query[j, c(i-j)]) * sm_scale,
    c(d) = clamp(bucket(d) + att_span, 0, 2 att_span - 1),
with the log bucket of models/deberta_v2/deberta_v2_encoder.py:70-89 evaluated
bit-exactly.

`flash_deberta_attention_fused` (no reference counterpart) takes the per-head
relative-position projections key_rel = key_proj(rel_emb), query_rel =
query_proj(rel_emb) ([H, 2S, D]) instead of the [B, H, L, 2S] pos_key /
pos_query tensors the reference materialises with two batched matmuls
(deberta_v2_encoder.py:275-286).
"""
from __future__ import annotations

import functools
import math
from typing import Optional

import torch

from . import _lib

# The reference's DeBERTa models read this flag as "the flash kernel is
# available" (models/deberta_v2/deberta_v2_encoder.py:39-42, :201, :230;
# models/deberta/deberta_encoder.py:35-38, :202, :227) and take their eager
# [B*H, L, L] path when it is false. The flash kernel here is the HIP one, so
# the flag is true: with this package on the import path those models call
# flash_deberta_attention. (There is no Triton code in this package.)
HAS_TRITON = True


def clear_config_cache() -> None:
    """Kept for API compatibility: tile shapes are fixed at build time."""
    return None


@functools.lru_cache(maxsize=64)
def unit_steps(position_buckets: int, max_relative_distance: int, use_log_bucket: bool,
               max_len: int) -> bool:
    """Whether c(d) = clamp(bucket(d) + att_span, 0, 2 att_span - 1) moves by at
    most 1 per unit of distance for |d| <= max_len. The fused kernel needs it;
    the log bucket of deberta_v2_encoder.py:70-89 breaks it when
    max_relative_positions is small against position_buckets (e.g. 256 / 256)."""
    rc = _lib.load().vfk_deberta_unit_steps(int(position_buckets), int(max_relative_distance),
                                            int(bool(use_log_bucket)), int(max_len))
    if rc < 0:
        _lib.call("vfk_deberta_unit_steps", int(position_buckets), int(max_relative_distance),
                  int(bool(use_log_bucket)), int(max_len))
    return rc == 1


def _seq_lengths(seq_lengths: Optional[torch.Tensor], B: int, dev) -> Optional[torch.Tensor]:
    if seq_lengths is None:
        return None
    sl = seq_lengths.to(device=dev, dtype=torch.int32).contiguous()
    if sl.numel() != B:
        raise ValueError(f"seq_lengths must have {B} entries")
    return sl


def flash_deberta_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    seq_lengths: Optional[torch.Tensor] = None,
    pos_key: Optional[torch.Tensor] = None,
    pos_query: Optional[torch.Tensor] = None,
    causal: bool = False,
    sm_scale: Optional[float] = None,
    position_buckets: int = 0,
    max_relative_distance: int = 0,
    use_log_bucket: bool = False,
) -> torch.Tensor:
    """Flash attention with DeBERTa disentangled relative position bias.

    q (B, H, M, D), k/v (B, H, N, D); pos_key (B, H, M, 2*ATT_SPAN),
    pos_query (B, H, N, 2*ATT_SPAN); seq_lengths (B,) int32 or None.
    """
    dev = _lib.require_gpu(q, k, v, pos_key, pos_query)
    B, H, M, D = q.shape
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(D)
    qq, kk, vv = (_lib.rows_aligned(t) for t in (q, k, v))
    pk = pos_key.to(q.dtype) if pos_key is not None else None
    pq = pos_query.to(q.dtype) if pos_query is not None else None
    sl = _seq_lengths(seq_lengths, B, dev)
    out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    _lib.on_device(
        "vfk_flash_deberta_fwd", dev,
        _lib.ref(_lib.desc(qq)), _lib.ref(_lib.desc(kk)), _lib.ref(_lib.desc(vv)),
        sl.data_ptr() if sl is not None else None,
        _lib.ref(_lib.desc(pk)), _lib.ref(_lib.desc(pq)),
        int(bool(causal)), float(sm_scale), int(position_buckets), int(max_relative_distance),
        int(bool(use_log_bucket)), _lib.ref(_lib.desc(out)),
    )
    return out


def rel_chunk_major(rel: torch.Tensor, att_span: int) -> torch.Tensor:
    """A per-head relative table [H, >= 2 att_span, 64] in the fused kernels'
    chunk-major layout [H, 8, 2 att_span, 8] (chunk c holds k = 8c .. 8c + 7
    of every row), so that each wave's operand load reads contiguous runs.
    A 4-D table is returned as given."""
    if rel.dim() == 4:
        return rel
    H, R, D = rel.shape
    if D != 64 or R < 2 * att_span:
        raise ValueError(f"expected [H, >= {2 * att_span}, 64], got {tuple(rel.shape)}")
    return rel[:, :2 * att_span].reshape(H, 2 * att_span, 8, 8).permute(0, 2, 1, 3).contiguous()


def _rel_tables(key_rel, query_rel, dtype, att_span, chunk_major):
    """Both tables in one layout: chunk-major (16-bit types, by default; the
    [H, 2S, 64] tables of a call are converted by one
    vfk_deberta_rel_chunk_major launch) or [H, 2S, 64] rows with aligned
    rows."""
    tabs = [None if t is None else t.to(dtype) for t in (key_rel, query_rel)]
    if chunk_major and dtype != torch.float32:
        todo = [t is not None and t.dim() == 3 for t in tabs]
        if any(todo):
            src = [_lib.rows_aligned(t) if c else None for t, c in zip(tabs, todo)]
            dst = [torch.empty(t.shape[0], 8, 2 * att_span, 8, dtype=dtype, device=t.device) if c else None
                   for t, c in zip(tabs, todo)]
            dev = _lib.require_gpu(*[t for t in src if t is not None])
            _lib.on_device("vfk_deberta_rel_chunk_major", dev, _lib.ref(_lib.desc(src[0])),
                           _lib.ref(_lib.desc(dst[0])), _lib.ref(_lib.desc(src[1])),
                           _lib.ref(_lib.desc(dst[1])), int(att_span))
            tabs = [d if c else t for t, d, c in zip(tabs, dst, todo)]
        return tabs
    if any(t is not None and t.dim() == 4 for t in tabs):
        raise ValueError("a chunk-major table needs a 16-bit dtype and chunk_major=True")
    return [None if t is None else _lib.rows_aligned(t) for t in tabs]


def flash_deberta_attention_fused(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    seq_lengths: Optional[torch.Tensor],
    key_rel: Optional[torch.Tensor],
    query_rel: Optional[torch.Tensor],
    sm_scale: float,
    position_buckets: int = 256,
    max_relative_distance: int = 512,
    use_log_bucket: bool = True,
    out: Optional[torch.Tensor] = None,
    chunk_major: bool = True,
) -> torch.Tensor:
    """Disentangled attention with c2p / p2c computed inside the kernel.

    key_rel, query_rel: [H, 2*ATT_SPAN, D] per-head projections of the
    relative-position embeddings, or the same in the chunk-major layout of
    `rel_chunk_major` (which the kernel reads with contiguous loads; 3-D
    tables are converted unless chunk_major is False). Equivalent to
    flash_deberta_attention with
    pos_key = q @ key_rel^T and pos_query = k @ query_rel^T. Raises
    NotImplementedError where `unit_steps` is False (flash_deberta_attention
    covers those bucket settings). `out` may be a
    strided [B, H, M, D] view (e.g. of a [B, M, H, D] buffer) with contiguous
    16-byte-aligned rows; it is written in place and returned.
    """
    dev = _lib.require_gpu(q, k, v, key_rel, query_rel)
    B = q.shape[0]
    qq, kk, vv = (_lib.rows_aligned(t) for t in (q, k, v))
    span = position_buckets if position_buckets > 0 else max_relative_distance
    kr, qr = _rel_tables(key_rel, query_rel, q.dtype, span, chunk_major)
    sl = _seq_lengths(seq_lengths, B, dev)
    if out is None:
        out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    elif (out.shape != q.shape or out.dtype != q.dtype or out.device != q.device
          or _lib.rows_aligned(out) is not out):
        raise ValueError("out must match q's shape, dtype and device, with contiguous 16-byte rows")
    _lib.on_device(
        "vfk_deberta_fused_fwd", dev,
        _lib.ref(_lib.desc(qq)), _lib.ref(_lib.desc(kk)), _lib.ref(_lib.desc(vv)),
        sl.data_ptr() if sl is not None else None,
        _lib.ref(_lib.desc(kr)), _lib.ref(_lib.desc(qr)), float(sm_scale),
        int(position_buckets), int(max_relative_distance), int(bool(use_log_bucket)),
        _lib.ref(_lib.desc(out)),
    )
    return out


def flash_deberta_attention_varlen(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    cu_seqlens: torch.Tensor,
    max_seqlen: int,
    key_rel: Optional[torch.Tensor],
    query_rel: Optional[torch.Tensor],
    sm_scale: float,
    position_buckets: int = 256,
    max_relative_distance: int = 512,
    use_log_bucket: bool = True,
    out: Optional[torch.Tensor] = None,
    chunk_major: bool = True,
) -> torch.Tensor:
    """flash_deberta_attention_fused over packed sequences, without padding.

    q, k, v [T, H, 64] (bf16 / fp16, any token and head strides with a
    contiguous last dim); sequence s is rows cu_seqlens[s] .. cu_seqlens[s+1]
    - 1 (int32 on the device) and attends to its own rows only, relative
    positions counted inside the sequence: the padded call with seq_lengths
    on the valid rows. max_seqlen must be >= every sequence length; bucket
    steps must be unit (`unit_steps`). Returns [T, H, 64] (or writes `out`)."""
    dev = _lib.require_gpu(q, k, v, cu_seqlens, key_rel, query_rel)
    if q.dim() != 3 or k.shape != q.shape or v.shape != q.shape:
        raise ValueError("q, k, v must be [T, H, D] of one shape")
    qq, kk, vv = (_lib.rows_aligned(t) for t in (q, k, v))
    span = position_buckets if position_buckets > 0 else max_relative_distance
    kr, qr = _rel_tables(key_rel, query_rel, q.dtype, span, chunk_major)
    if out is None:
        out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    elif (out.shape != q.shape or out.dtype != q.dtype or out.device != q.device
          or _lib.rows_aligned(out) is not out):
        raise ValueError("out must match q's shape, dtype and device, with contiguous 16-byte rows")
    cu = cu_seqlens.to(torch.int32).contiguous()
    _lib.on_device(
        "vfk_deberta_fused_varlen_fwd", dev,
        _lib.ref(_lib.desc(qq)), _lib.ref(_lib.desc(kk)), _lib.ref(_lib.desc(vv)),
        cu.data_ptr(), int(cu.numel() - 1), int(max_seqlen),
        _lib.ref(_lib.desc(kr)), _lib.ref(_lib.desc(qr)), float(sm_scale),
        int(position_buckets), int(max_relative_distance), int(bool(use_log_bucket)),
        _lib.ref(_lib.desc(out)),
    )
    return out


__all__ = ["flash_deberta_attention", "flash_deberta_attention_fused",
           "flash_deberta_attention_varlen", "rel_chunk_major", "unit_steps",
           "clear_config_cache", "HAS_TRITON"]
