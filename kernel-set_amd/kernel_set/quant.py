"""Quantizers and weight-format helpers (``include/kernel_set/quant.h``).

Same names, argument order and defaults as the reference's
``bindings/python/kernel_set/quant.py:35-215`` (``quantize_nvfp4`` excluded).
"""
from __future__ import annotations

from ctypes import POINTER, c_float, cast
from typing import Optional

from ._lib import check, lib
from ._tensor import TensorLike, default_stream, infer_dtype, ptr
from .enums import DType, QuantMode

__all__ = ["quantize_fp8", "quantize_fp8_group", "dequantize_fp8", "quantize_int8",
           "dequantize_int8", "dequantize_int4", "repack_int4"]

_F32P = POINTER(c_float)


def _f32(obj, *, name, allow_none=False):
    raw = ptr(obj, name=name, allow_none=allow_none)
    return cast(raw, _F32P) if raw else _F32P()


def quantize_fp8(out, scale, input, rows: int, cols: int, in_dtype: Optional[int] = None,
                 fp8_dtype: int = DType.F8E4M3, mode: int = QuantMode.PER_TENSOR,
                 stream: TensorLike = None):
    """Dynamic fp8 quant; ``scale`` fp32 ``[1]`` (per-tensor) or ``[rows]``."""
    dt = infer_dtype(input, in_dtype)
    check(lib.ks_quantize_fp8(ptr(out, name="out"), _f32(scale, name="scale"),
                              ptr(input, name="input"), int(rows), int(cols), dt,
                              int(fp8_dtype), int(mode), default_stream(stream, input)),
          "ks_quantize_fp8")
    return out, scale


def quantize_fp8_group(out, scale, input, rows: int, cols: int, group_size: int = 128,
                       in_dtype: Optional[int] = None, fp8_dtype: int = DType.F8E4M3,
                       stream: TensorLike = None):
    """Per-token-group (1 x group_size) fp8 quant; ``scale [rows, ceil(cols/gs)]``."""
    dt = infer_dtype(input, in_dtype)
    check(lib.ks_quantize_fp8_group(ptr(out, name="out"), _f32(scale, name="scale"),
                                    ptr(input, name="input"), int(rows), int(cols),
                                    int(group_size), dt, int(fp8_dtype),
                                    default_stream(stream, input)),
          "ks_quantize_fp8_group")
    return out, scale


def dequantize_fp8(out, input, scale, rows: int, cols: int, out_dtype: Optional[int] = None,
                   fp8_dtype: int = DType.F8E4M3, mode: int = QuantMode.PER_TENSOR,
                   stream: TensorLike = None):
    dt = infer_dtype(out, out_dtype)
    check(lib.ks_dequantize_fp8(ptr(out, name="out"), ptr(input, name="input"),
                                _f32(scale, name="scale"), int(rows), int(cols), dt,
                                int(fp8_dtype), int(mode), default_stream(stream, out)),
          "ks_dequantize_fp8")
    return out


def quantize_int8(out, scale, input, rows: int, cols: int, in_dtype: Optional[int] = None,
                  mode: int = QuantMode.PER_TOKEN, stream: TensorLike = None):
    """Dynamic symmetric int8 quant; returns ``(out, scale)``."""
    dt = infer_dtype(input, in_dtype)
    check(lib.ks_quantize_int8(ptr(out, name="out"), _f32(scale, name="scale"),
                               ptr(input, name="input"), int(rows), int(cols), dt,
                               int(mode), default_stream(stream, input)),
          "ks_quantize_int8")
    return out, scale


def dequantize_int8(out, input, scale, rows: int, cols: int, out_dtype: Optional[int] = None,
                    mode: int = QuantMode.PER_TOKEN, stream: TensorLike = None):
    dt = infer_dtype(out, out_dtype)
    check(lib.ks_dequantize_int8(ptr(out, name="out"), ptr(input, name="input"),
                                 _f32(scale, name="scale"), int(rows), int(cols), dt,
                                 int(mode), default_stream(stream, out)),
          "ks_dequantize_int8")
    return out


def dequantize_int4(out, qweight_packed, scales, zeros, k: int, n: int, group_size: int,
                    out_dtype: Optional[int] = None, stream: TensorLike = None):
    """int32 ``[k/8, n]`` (code of row k in nibble k % 8) -> ``[k, n]``."""
    dt = infer_dtype(out, out_dtype)
    check(lib.ks_dequantize_int4(ptr(out, name="out"), ptr(qweight_packed, name="qweight_packed"),
                                 ptr(scales, name="scales"), ptr(zeros, name="zeros"),
                                 int(k), int(n), int(group_size), dt,
                                 default_stream(stream, out)),
          "ks_dequantize_int4")
    return out


def repack_int4(out_packed, qweight, perm, size_k: int, size_n: int, num_bits: int = 4,
                stream: TensorLike = None):
    """int32 ``[K/8, N]`` -> uint8 ``[K/2, N]`` (the ``gemm_w4a16`` layout).
    ``perm`` (int32 ``[K]`` or None): output row k takes input row ``perm[k]``."""
    check(lib.ks_repack_int4(ptr(out_packed, name="out_packed"), ptr(qweight, name="qweight"),
                             ptr(perm, name="perm", allow_none=True), int(size_k), int(size_n),
                             int(num_bits), default_stream(stream, out_packed)),
          "ks_repack_int4")
    return out_packed
