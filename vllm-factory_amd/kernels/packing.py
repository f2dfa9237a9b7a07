"""Packed-stream plumbing on the device: sequence boundaries from vLLM's flat
position ids, and flat <-> padded row copies for the padded encoders.

No reference kernel exists for these steps; they replace host-side and dense
constructions around the hot path:

  * seq_metadata / varlen_from_positions: the boundary detection of
    models/modernbert/modernbert_encoder.py:491-516 (_build_seq_block_mask,
    rule "reset": a sequence starts wherever the position does not increase)
    and of plugins/deberta_gliner/model.py:166-170 (rule "zero": a sequence
    starts at every position 0);
  * pad_packed / unpad_packed / batch_from_flat: the per-row copy loop of
    plugins/deberta_gliner/model.py:171-200 (batched ids with pad_id,
    positions with 0, attention mask, and the torch.cat of the valid rows of
    the encoder output).

Shapes that depend on the data (number of sequences, longest sequence) are
read back once, 16 bytes, as the reference reads its start list with .tolist().
"""
from __future__ import annotations

from typing import Tuple

import torch

from . import _lib

_RULES = {"reset": _lib.SEQ_RESET, "zero": _lib.SEQ_ZERO}


def seq_metadata(position_ids: torch.Tensor,
                 rule: str = "reset") -> Tuple[torch.Tensor, torch.Tensor]:
    """Device-side packed-sequence metadata from flat position ids.

    position_ids: int32/int64 [T] or [1, T] on the device. rule "reset"
    (ModernBERT): token 0 starts a sequence, and so does every token whose
    position does not exceed its predecessor's; rule "zero" (GLiNER plugins):
    token 0 and every token at position 0. Returns (cu_seqlens int32 [T + 1],
    meta int32 [4]) on the device, nothing read back: cu_seqlens[0..n] hold
    the n sequence starts and T, meta = (n, longest sequence, breaks in the
    run of positions, T); the break count (a start whose position is not 0, or
    a step other than +1) is 0 exactly when every token's position is
    t - cu_seqlens[s]."""
    if rule not in _RULES:
        raise ValueError(f"rule must be one of {sorted(_RULES)}, got {rule!r}")
    dev = _lib.require_gpu(position_ids)
    pos = position_ids.reshape(-1)
    if pos.dtype not in (torch.int32, torch.int64):
        raise ValueError("position_ids must be int32 or int64")
    T = pos.numel()
    if T == 0:
        raise ValueError("position_ids is empty")
    pos = pos.contiguous()
    cu = torch.empty(T + 1, dtype=torch.int32, device=dev)
    meta = torch.empty(4, dtype=torch.int32, device=dev)
    ws_bytes = int(_lib.load().vfk_varlen_meta_workspace_bytes(T))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    _lib.on_device("vfk_varlen_meta", dev, pos.data_ptr(), pos.element_size(), T, _RULES[rule],
                   cu.data_ptr(), meta.data_ptr(), ws.data_ptr(), ws_bytes)
    return cu, meta


def read_metadata(cu: torch.Tensor, meta: torch.Tensor) -> Tuple[torch.Tensor, int, int, int]:
    """(cu_seqlens [n + 1] view, n, longest sequence, breaks), one read-back."""
    n, max_len, bad, _ = (int(x) for x in meta.cpu())
    return cu[:n + 1], n, max_len, bad


def varlen_from_positions(position_ids: torch.Tensor,
                          require_restart: bool = True) -> Tuple[torch.Tensor, int]:
    """(cu_seqlens int32 [n + 1] on the device, max_seqlen) for
    varlen_rope_attention, from the reference's position ids (rule "reset");
    one 16-byte read back. require_restart: raise if some token's position is
    not its offset in its sequence (the reference would rotate it by its own
    position id, the varlen op by its offset)."""
    cu, n, max_len, bad = read_metadata(*seq_metadata(position_ids, "reset"))
    if require_restart and bad:
        raise ValueError(f"position ids do not count up from 0 within their sequence "
                         f"({bad} breaks)")
    return cu, max_len


def _fill_bits(t: torch.Tensor, fill) -> int:
    v = torch.tensor([fill], dtype=t.dtype)
    raw = v.view(torch.uint8).tolist()
    return sum(b << (8 * i) for i, b in enumerate(raw))


def pad_packed(x: torch.Tensor, cu_seqlens: torch.Tensor, num_seqs: int, max_len: int,
               fill=0) -> Tuple[torch.Tensor, torch.Tensor]:
    """x [T, ...] (flat rows) -> (padded [num_seqs, max_len, ...] with `fill`
    beyond each sequence, seq_lengths int32 [num_seqs]), on x's device."""
    dev = _lib.require_gpu(x, cu_seqlens)
    if x.dim() < 1:
        raise ValueError("x needs a token dimension")
    x = x.contiguous()
    cu = cu_seqlens.to(torch.int32).contiguous()
    if cu.numel() < num_seqs + 1:
        raise ValueError("cu_seqlens needs num_seqs + 1 entries")
    row_bytes = x[0].numel() * x.element_size() if x.shape[0] else x.element_size()
    out = torch.empty((num_seqs, max_len) + tuple(x.shape[1:]), dtype=x.dtype, device=dev)
    lens = torch.empty(num_seqs, dtype=torch.int32, device=dev)
    _lib.on_device("vfk_pad_rows", dev, x.data_ptr(), row_bytes, cu.data_ptr(), int(num_seqs),
                   int(max_len), x.element_size(), _fill_bits(x, fill), out.data_ptr(),
                   lens.data_ptr())
    return out, lens


def unpad_packed(padded: torch.Tensor, cu_seqlens: torch.Tensor, total_tokens: int) -> torch.Tensor:
    """padded [num_seqs, max_len, ...] -> flat [total_tokens, ...] of the
    valid rows, in sequence order."""
    dev = _lib.require_gpu(padded, cu_seqlens)
    if padded.dim() < 2:
        raise ValueError("padded needs [num_seqs, max_len, ...]")
    padded = padded.contiguous()
    cu = cu_seqlens.to(torch.int32).contiguous()
    B, L = padded.shape[:2]
    if cu.numel() < B + 1:
        raise ValueError("cu_seqlens needs num_seqs + 1 entries")
    row_bytes = padded[0, 0].numel() * padded.element_size()
    out = torch.empty((total_tokens,) + tuple(padded.shape[2:]), dtype=padded.dtype, device=dev)
    _lib.on_device("vfk_unpad_rows", dev, padded.data_ptr(), row_bytes, cu.data_ptr(), int(B),
                   int(L), out.data_ptr())
    return out


def batch_from_flat(input_ids: torch.Tensor, positions: torch.Tensor, pad_id: int = 0):
    """The padded batch plugins/deberta_gliner/model.py:166-191 builds from a
    flat vLLM call, on the device: returns (batched_ids [B, L] padded with
    pad_id, batched_positions [B, L] padded with 0, attention_mask [B, L]
    int64, cu_seqlens int32 [B + 1], seq_lengths int32 [B])."""
    cu, n, max_len, _ = read_metadata(*seq_metadata(positions, "zero"))
    ids, lens = pad_packed(input_ids.reshape(-1), cu, n, max_len, pad_id)
    pos, _ = pad_packed(positions.reshape(-1).to(input_ids.device), cu, n, max_len, 0)
    mask = (torch.arange(max_len, device=ids.device)[None, :] < lens[:, None]).to(torch.int64)
    return ids, pos, mask, cu, lens
