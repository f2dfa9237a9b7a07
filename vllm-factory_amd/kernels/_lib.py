"""ctypes binding of libvfk.so (the gfx950 kernel library, C ABI in include/vfk.h).

Every public op in this package goes through `call()`: tensors are described by
`VfkTensor` (pointer, dtype code, sizes, element strides) and kernels run on the
caller's current torch stream. There is no CPU or alternative GPU path: a
missing library or a non-GPU tensor raises.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional, Sequence

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.normpath(os.path.join(_HERE, "..", "lib", "libvfk.so"))

F32, BF16, F16 = 0, 1, 2
OK, ERR_INVALID, ERR_UNSUPPORTED = 0, -1, -2
SEQ_RESET, SEQ_ZERO = 0, 1
ACT_GELU_ERF, ACT_GELU_TANH, ACT_SILU, ACT_RELU = 0, 1, 2, 3

_DTYPE_CODE = {torch.float32: F32, torch.bfloat16: BF16, torch.float16: F16}


class VfkTensor(ctypes.Structure):
    _fields_ = [
        ("data", ctypes.c_void_p),
        ("dtype", ctypes.c_int32),
        ("ndim", ctypes.c_int32),
        ("size", ctypes.c_int64 * 4),
        ("stride", ctypes.c_int64 * 4),
    ]


_P = ctypes.POINTER(VfkTensor)
_vp = ctypes.c_void_p
_i32 = ctypes.c_int32
_f32 = ctypes.c_float
_i64 = ctypes.c_int64

# name -> argtypes (restype int unless listed in _RESTYPES)
_SIGNATURES = {
    "vfk_abi_version": [],
    "vfk_t5_bucket": [_vp, _vp, ctypes.c_int64, _i32, _i32, _i32],
    "vfk_deberta_bucket": [_vp, _vp, ctypes.c_int64, _i32, _i32],
    "vfk_deberta_unit_steps": [_i32, _i32, _i32, _i32],
    "vfk_flash_rpb_fwd": [_P, _P, _P, _P, _i32, _i32, _i32, _P, _f32, _P, _vp],
    "vfk_flash_rpb_varlen_fwd": [_P, _P, _P, _vp, _i32, _i32, _P, _i32, _i32, _i32, _f32, _P, _vp],
    "vfk_flash_deberta_fwd": [_P, _P, _P, _vp, _P, _P, _i32, _f32, _i32, _i32, _i32, _P, _vp],
    "vfk_deberta_fused_fwd": [_P, _P, _P, _vp, _P, _P, _f32, _i32, _i32, _i32, _P, _vp],
    "vfk_deberta_fused_varlen_fwd": [_P, _P, _P, _vp, _i32, _i32, _P, _P, _f32, _i32, _i32, _i32, _P,
                                     _vp],
    "vfk_varlen_attn_fwd": [_P, _P, _P, _vp, _i32, _i32, _i32, _vp, _i32, _vp, _f32, _vp, _i64,
                            _P, _vp],
    "vfk_varlen_attn_workspace_bytes": [_i32, _i64, _i32, _i32, _i32, _i32],
    "vfk_rope_table": [_f32, _i32, _vp, _vp],
    "vfk_varlen_meta": [_vp, _i32, _i64, _i32, _vp, _vp, _vp, _i64, _vp],
    "vfk_varlen_meta_noalloc": [_vp, _i32, _i64, _i32, _vp, _vp, _vp],
    "vfk_pad_rows": [_vp, _i64, _vp, _i32, _i32, _i32, ctypes.c_uint64, _vp, _vp, _vp],
    "vfk_unpad_rows": [_vp, _i64, _vp, _i32, _i32, _vp, _vp],
    "vfk_varlen_meta_workspace_bytes": [_i64],
    "vfk_gliner_class_workspace_bytes": [_i64],
    "vfk_gliner_class_index": [_vp, _i64, _i64, _i32, _vp, _i32, _vp, _vp, _vp, _vp, _vp, _i64,
                               _vp],
    "vfk_gliner_prompt_rows": [_vp, _i64, _i64, _vp, _vp, _i32, _i64, _vp, _vp],
    "vfk_gliner_word_index": [_vp, _i64, _vp, _i32, _vp, _vp, _vp, _vp],
    "vfk_gliner_word_rows": [_vp, _i64, _i64, _vp, _i64, _vp, _vp],
    "vfk_gliner_span_rows": [_vp, _vp, _i64, _i64, _i32, _vp, _i32, _vp, _vp, _vp, _i64, _vp, _vp],
    "vfk_gliner_span_hidden": [_vp, _vp, _vp, _i64, _i64, _i32, _vp, _i32, _vp, _vp, _vp, _i64, _vp,
                               _vp],
    "vfk_rope_fwd": [_P, _P, _P, _P, _vp],
    "vfk_rope_qk_fwd": [_P, _P, _P, _P, _P, _P, _vp],
    "vfk_layernorm_fwd": [_P, _P, _P, _P, _f32, _P, _P, _vp],
    "vfk_rmsnorm_fwd": [_P, _P, _P, _f32, _P, _P, _vp],
    "vfk_glu_fwd": [_i32, _P, _P, _P, _vp],
    "vfk_glu_linear_fwd": [_i32, _P, _P, _P, _vp],
    "vfk_dense_residual_layernorm_fwd": [_P, _P, _P, _P, _P, _P, _f32, _P, _P, _vp],
    "vfk_pack_weight_mfma32": [_P, _P, _vp],
    "vfk_deberta_rel_chunk_major": [_P, _P, _P, _P, _i32, _vp],
    "vfk_qkv_rope_linear_fwd": [_P, _P, _vp, _vp, _i32, _i32, _f32, _P, _P, _vp, _i64, _vp],
    "vfk_qkv_rope_workspace_bytes": [_i64, _i32],
    "vfk_varlen_attn_krot_fwd": [_P, _P, _vp, _i64, _vp, _i32, _i32, _i32, _vp, _i32, _vp, _f32,
                                 _P, _vp],
    "vfk_act_fwd": [_i32, _P, _P, _vp],
    "vfk_residual_add": [_P, _P, _P, _vp],
    "vfk_colbert_head_fwd": [_P, _P, _P, _P, _f32, _P, _P, _P, _P, _vp],
    "vfk_colbert_fold_weight": [_P, _P, _P, _P, _P, _P, _P, _vp],
    "vfk_colbert_head_folded_fwd": [_P, _P, _P, _P, _P, _f32, _P, _vp],
}

_RESTYPES = {"vfk_varlen_attn_workspace_bytes": ctypes.c_int64,
             "vfk_qkv_rope_workspace_bytes": ctypes.c_int64,
             "vfk_varlen_meta_workspace_bytes": ctypes.c_int64,
             "vfk_gliner_class_workspace_bytes": ctypes.c_int64}

_lib: Optional[ctypes.CDLL] = None


def load() -> ctypes.CDLL:
    """Loads libvfk.so once (after torch, so both share one HIP runtime)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"libvfk.so is not built ({LIB_PATH}); run "
            "`python vllm-factory_amd/build.py` or __graft_entry__.build()"
        )
    lib = ctypes.CDLL(LIB_PATH)
    missing = [n for n in _SIGNATURES if not hasattr(lib, n)]
    if missing:
        raise RuntimeError(f"libvfk.so lacks symbols {missing}; rebuild it")
    for name, argtypes in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = _RESTYPES.get(name, ctypes.c_int)
    lib.vfk_last_error.argtypes = []
    lib.vfk_last_error.restype = ctypes.c_char_p
    _lib = lib
    return lib


def dtype_code(dt: torch.dtype) -> int:
    try:
        return _DTYPE_CODE[dt]
    except KeyError:
        raise NotImplementedError(f"dtype {dt} is not supported by libvfk") from None


def desc(t: Optional[torch.Tensor], shape: Optional[Sequence[int]] = None,
         strides: Optional[Sequence[int]] = None) -> Optional[VfkTensor]:
    """Describes a tensor (optionally with an overriding view shape/strides)."""
    if t is None:
        return None
    shape = list(t.shape) if shape is None else list(shape)
    strides = list(t.stride()) if strides is None else list(strides)
    if len(shape) > 4:
        raise ValueError(f"libvfk tensors have at most 4 dims, got {len(shape)}")
    d = VfkTensor()
    d.data = t.data_ptr()
    d.dtype = dtype_code(t.dtype)
    d.ndim = len(shape)
    for i in range(4):
        d.size[i] = shape[i] if i < len(shape) else 1
        d.stride[i] = strides[i] if i < len(strides) else 0
    return d


def ref(d: Optional[VfkTensor]):
    return ctypes.byref(d) if d is not None else None


def require_gpu(*tensors: Optional[torch.Tensor]) -> torch.device:
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError(
                "libvfk kernels run on the GPU only; got a tensor on "
                f"{t.device} (no CPU path exists in this package)"
            )
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"tensors on different devices: {dev} vs {t.device}")
    if dev is None:
        raise RuntimeError("no tensor arguments")
    return dev


def stream_of(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def call(name: str, *args) -> None:
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc == OK:
        return
    msg = (lib.vfk_last_error() or b"").decode(errors="replace")
    if rc == ERR_UNSUPPORTED:
        raise NotImplementedError(f"{name}: {msg}")
    if rc == ERR_INVALID:
        raise ValueError(f"{name}: {msg}")
    raise RuntimeError(f"{name}: HIP error {rc}: {msg}")


def on_device(fn_name: str, device: torch.device, *args) -> None:
    """Calls a GPU entry point with `device` current and its current stream."""
    with torch.cuda.device(device):
        call(fn_name, *args, stream_of(device))


def rows_aligned(t: torch.Tensor) -> torch.Tensor:
    """Returns t, or a contiguous copy, so that the last dim is contiguous and
    every row starts on a 16-byte boundary (what the vector paths need)."""
    el = t.element_size()
    ok = (t.stride(-1) == 1 and t.data_ptr() % 16 == 0
          and all((s * el) % 16 == 0 for s in t.stride()[:-1]))
    if ok:
        return t
    c = t.contiguous()
    if c.data_ptr() % 16 != 0:
        c = c.clone()
    return c
