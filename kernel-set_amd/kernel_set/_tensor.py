"""Tensor-like -> (device pointer, dtype, stream) resolution for the op wrappers.

Same contract as the reference's ``bindings/python/kernel_set/_tensor.py:142-235``:
an argument may be a torch device tensor (must be contiguous), a raw ``int``
device address, anything exposing ``data_ptr()``, or ``None`` where optional.
Streams default to torch's current stream for the tensor's device, so launches
are ordered with the caller's torch work.
"""
from __future__ import annotations

from typing import Optional, Union

from . import _lib

TensorLike = Union[int, object, None]

try:
    import torch as _torch
except Exception:  # pragma: no cover
    _torch = None


def _is_tensor(obj) -> bool:
    return _torch is not None and isinstance(obj, _torch.Tensor)


def _dtype_pairs():
    if _torch is None:
        return []
    names = [("float32", _lib.KS_DTYPE_F32), ("float16", _lib.KS_DTYPE_F16),
             ("bfloat16", _lib.KS_DTYPE_BF16), ("float64", _lib.KS_DTYPE_F64),
             ("int64", _lib.KS_DTYPE_I64), ("int32", _lib.KS_DTYPE_I32),
             ("int8", _lib.KS_DTYPE_I8), ("uint8", _lib.KS_DTYPE_U8),
             ("float8_e4m3fn", _lib.KS_DTYPE_F8E4M3),
             ("float8_e5m2", _lib.KS_DTYPE_F8E5M2)]
    return [(getattr(_torch, a), k) for a, k in names if hasattr(_torch, a)]


TORCH_TO_KS = {t: k for t, k in _dtype_pairs()}
KS_TO_TORCH = {}
for _t, _k in _dtype_pairs():
    KS_TO_TORCH.setdefault(_k, _t)


def dtype_to_ks(torch_dtype) -> int:
    try:
        return TORCH_TO_KS[torch_dtype]
    except KeyError:
        raise ValueError(f"torch dtype {torch_dtype!r} has no kernel_set equivalent") from None


def ks_to_torch_dtype(ks_dtype: int):
    try:
        return KS_TO_TORCH[int(ks_dtype)]
    except KeyError:
        raise ValueError(f"ks dtype {int(ks_dtype)} has no torch equivalent") from None


def ptr(obj: TensorLike, *, name: str = "tensor", allow_none: bool = True) -> int:
    if obj is None:
        if allow_none:
            return 0
        raise ValueError(f"{name} must not be None")
    if isinstance(obj, int):
        return obj
    if _is_tensor(obj):
        if not obj.is_cuda:
            raise ValueError(f"{name} must be a device tensor (got {obj.device}); "
                             "kernel_set operates on device memory")
        if not obj.is_contiguous():
            raise ValueError(f"{name} must be contiguous; call .contiguous() first")
        return obj.data_ptr()
    dp = getattr(obj, "data_ptr", None)
    if callable(dp):
        return int(dp())
    raise TypeError(f"{name} must be a torch.Tensor, an int device pointer, or expose "
                    f"data_ptr(); got {type(obj).__name__}")


def stream_ptr(stream) -> int:
    if stream is None:
        return 0
    if isinstance(stream, int):
        return stream
    if isinstance(stream, str) and stream == "current":
        if _torch is None:
            raise RuntimeError("stream='current' requires torch")
        return _torch.cuda.current_stream().cuda_stream
    cs = getattr(stream, "cuda_stream", None)
    if cs is not None:
        return int(cs)
    raise TypeError(f"stream must be None, an int, 'current' or a torch stream; "
                    f"got {type(stream).__name__}")


def default_stream(stream, reference: TensorLike = None) -> int:
    if stream is not None:
        return stream_ptr(stream)
    if _is_tensor(reference) and reference.is_cuda:
        return _torch.cuda.current_stream(reference.device).cuda_stream
    return 0


def infer_dtype(reference: TensorLike, dtype: Optional[int]) -> int:
    if dtype is not None:
        return int(dtype)
    if _is_tensor(reference):
        return dtype_to_ks(reference.dtype)
    raise ValueError("dtype could not be inferred from a raw pointer; pass dtype=DType.*")
