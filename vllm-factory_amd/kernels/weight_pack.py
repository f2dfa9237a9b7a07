"""Projection weights in MFMA operand order (vfk_pack_weight_mfma32).

Kernels that stream a whole [N, K] weight per workgroup (the dense +
LayerNorm block, the ColBERT head) read it as [N/32, K/16, 64, 8]: block
(f, s) holds rows 32 f .. +32 and k = 16 s .. +16 in the order one wave's
32x32x16 operand load takes them, so each such load is one contiguous KiB.

`packed_weight` keeps one packed copy per live weight tensor: the entry is
keyed by the tensor object (a weak reference) and its version counter, so an
in-place update of the weight, or a new tensor at the same address,
re-packs. Tensors made under torch.inference_mode() (vLLM runs its forward
there) have no version counter: their entry is keyed by the object alone, so
an in-place update of such a weight inside inference mode is not seen; call
`clear_cache()` after one.
"""
from __future__ import annotations

import weakref

import torch

from . import _lib


def pack_weight(weight: torch.Tensor) -> torch.Tensor:
    """weight [N, K] (N a multiple of 32, K of 16) -> a new packed
    [N / 32, K / 16, 64, 8] tensor on the same device."""
    dev = _lib.require_gpu(weight)
    if weight.dim() != 2:
        raise ValueError(f"weight must be [N, K], got {tuple(weight.shape)}")
    N, K = weight.shape
    w2 = _lib.rows_aligned(weight)
    packed = torch.empty(max(N // 32, 1), max(K // 16, 1), 64, 8, dtype=weight.dtype,
                         device=weight.device)
    _lib.on_device("vfk_pack_weight_mfma32", dev, _lib.ref(_lib.desc(w2)),
                   _lib.ref(_lib.desc(packed)))
    return packed


_CACHE: dict = {}


def _version(weight: torch.Tensor) -> int:
    # inference tensors carry no version counter (reading it raises)
    return -1 if weight.is_inference() else weight._version


def packed_weight(weight: torch.Tensor) -> torch.Tensor:
    """pack_weight(weight), made once per weight tensor and version."""
    key = id(weight)
    ver = _version(weight)
    hit = _CACHE.get(key)
    if hit is not None and hit[0]() is weight and hit[1] == ver:
        return hit[2]
    packed = pack_weight(weight.detach())
    _CACHE[key] = (weakref.ref(weight, lambda _r, k=key: _CACHE.pop(k, None)), ver, packed)
    return packed


def clear_cache() -> None:
    """Drops every packed copy (e.g. after an in-place update of a weight
    made under inference mode, which has no version counter)."""
    _CACHE.clear()


__all__ = ["pack_weight", "packed_weight", "clear_cache"]
