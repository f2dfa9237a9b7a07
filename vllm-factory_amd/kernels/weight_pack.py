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

The ColBERT head's folded weight (`folded_colbert_weight`) is cached the same
way, per projection weight, and also follows the LayerNorm weight and bias
and the projection bias it was made from.
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


_FOLDED: dict = {}


def fold_colbert_weight(weight: torch.Tensor, norm_weight=None, norm_bias=None, bias=None):
    """The ColBERT head's folded constants (vfk_colbert_fold_weight): the
    LayerNorm weight gamma multiplied into the projection weight, packed in
    operand order, plus fp32 G = row sums of that product and
    C = W beta + b. Returns (folded, G, C)."""
    dev = _lib.require_gpu(weight, norm_weight, norm_bias, bias)
    if weight.dim() != 2:
        raise ValueError(f"weight must be [N, D], got {tuple(weight.shape)}")
    N, D = weight.shape
    w2 = _lib.rows_aligned(weight.detach())
    folded = torch.empty(max(N // 32, 1), max(D // 16, 1), 64, 8, dtype=weight.dtype, device=dev)
    g = torch.empty(N, dtype=torch.float32, device=dev)
    c = torch.empty(N, dtype=torch.float32, device=dev)
    vec = lambda t: None if t is None else t.detach().contiguous()
    _lib.on_device("vfk_colbert_fold_weight", dev, _lib.ref(_lib.desc(w2)),
                   _lib.ref(_lib.desc(vec(norm_weight))), _lib.ref(_lib.desc(vec(norm_bias))),
                   _lib.ref(_lib.desc(vec(bias))), _lib.ref(_lib.desc(folded)),
                   _lib.ref(_lib.desc(g)), _lib.ref(_lib.desc(c)))
    return folded, g, c


def folded_colbert_weight(weight: torch.Tensor, norm_weight=None, norm_bias=None, bias=None):
    """fold_colbert_weight(...), made once per weight tensor: the entry is
    keyed by the projection weight (one entry each) and remembers the
    LayerNorm weight, LayerNorm bias and bias objects and the versions of
    all four; any change re-folds."""
    parts = (weight, norm_weight, norm_bias, bias)
    sig = tuple((None, 0) if t is None else (id(t), _version(t)) for t in parts)
    key = id(weight)
    hit = _FOLDED.get(key)
    if (hit is not None and hit[0]() is weight and hit[1] == sig
            and all(t is None or r() is t for t, r in zip(parts[1:], hit[2]))):
        return hit[3]
    val = fold_colbert_weight(weight, norm_weight, norm_bias, bias)
    refs = tuple(None if t is None else weakref.ref(t) for t in parts[1:])
    _FOLDED[key] = (weakref.ref(weight, lambda _r, k=key: _FOLDED.pop(k, None)), sig, refs, val)
    return val


def clear_cache() -> None:
    """Drops every packed and folded copy (e.g. after an in-place update of a
    weight made under inference mode, which has no version counter)."""
    _CACHE.clear()
    _FOLDED.clear()


__all__ = ["pack_weight", "packed_weight", "fold_colbert_weight", "folded_colbert_weight",
           "clear_cache"]
