"""Quantized GEMMs (``include/kernel_set/gemm.h``).

Same function names, argument order and defaults as the reference's
``bindings/python/kernel_set/gemm.py:151-362`` for the four quantized GEMMs.
"""
from __future__ import annotations

from ctypes import POINTER, c_float, cast
from typing import Optional

from ._lib import check, lib
from ._tensor import TensorLike, _is_tensor, default_stream, dtype_to_ks, infer_dtype, ptr
from .enums import QuantMode

__all__ = ["gemm_w8a8", "gemm_w4a16", "gemm_w4a16_noalloc", "gemm_fp8", "gemm_fp8_blockwise"]

_F32P = POINTER(c_float)


def _f32(obj, *, name, allow_none=False):
    raw = ptr(obj, name=name, allow_none=allow_none)
    return cast(raw, _F32P) if raw else _F32P()


def _out_dtype(out, out_dtype, fn):
    if out_dtype is not None:
        return int(out_dtype)
    if _is_tensor(out):
        return dtype_to_ks(out.dtype)
    raise ValueError(f"out_dtype is required for {fn}")


def gemm_w8a8(c: TensorLike, a_i8: TensorLike, b_i8: TensorLike, a_scale: TensorLike,
              b_scale: TensorLike, m: int, n: int, k: int, bias: TensorLike = None,
              a_mode: int = QuantMode.PER_TOKEN, b_mode: int = QuantMode.PER_CHANNEL,
              out_dtype: int = None, stream: TensorLike = None) -> TensorLike:
    """int8 ``A [M,K]`` x int8 ``B [K,N]`` -> ``C [M,N]`` in ``out_dtype``;
    exact int32 accumulation then ``(acc * a_scale) * b_scale (+ bias)``."""
    odt = _out_dtype(c, out_dtype, "ks_gemm_w8a8")
    check(lib.ks_gemm_w8a8(
        ptr(c, name="c"), ptr(a_i8, name="a_i8"), ptr(b_i8, name="b_i8"),
        _f32(a_scale, name="a_scale"), _f32(b_scale, name="b_scale"),
        ptr(bias, name="bias"), int(m), int(n), int(k), int(a_mode), int(b_mode), odt,
        default_stream(stream, c if not isinstance(c, int) else a_i8)), "ks_gemm_w8a8")
    return c


def gemm_w8a8_fused_quant(c: TensorLike, a: TensorLike, b_i8: TensorLike,
                          b_scale: TensorLike, m: int, n: int, k: int,
                          bias: TensorLike = None, a_mode: int = QuantMode.PER_TOKEN,
                          b_mode: int = QuantMode.PER_CHANNEL, a_dtype: int = None,
                          out_dtype: int = None, stream: TensorLike = None) -> TensorLike:
    """Extension (no reference counterpart): ``c = gemm_w8a8(quantize_int8(a,
    a_mode), b_i8, b_scale, bias)`` with the same bits as that two-call
    sequence. ``a`` is bf16/f16/f32 ``[M, K]``; decode shapes (M <= 4) run as
    a single pass."""
    adt = infer_dtype(a, a_dtype)
    odt = _out_dtype(c, out_dtype, "ks_gemm_w8a8_fused_quant")
    check(lib.ks_gemm_w8a8_fused_quant(
        ptr(c, name="c"), ptr(a, name="a"), ptr(b_i8, name="b_i8"),
        _f32(b_scale, name="b_scale"), ptr(bias, name="bias"), int(m), int(n), int(k),
        int(a_mode), int(b_mode), adt, odt,
        default_stream(stream, c if not isinstance(c, int) else a)),
        "ks_gemm_w8a8_fused_quant")
    return c


def gemm_w4a16(c: TensorLike, a: TensorLike, b_packed: TensorLike, scales: TensorLike,
               zeros: TensorLike, m: int, n: int, k: int, group_size: int,
               bias: TensorLike = None, dtype: Optional[int] = None,
               stream: TensorLike = None) -> TensorLike:
    """f16/bf16 ``A [M,K]`` x int4 ``B`` (uint8 ``[K/2,N]``, even k in the low
    nibble) with ``[K/group_size, N]`` scales/zeros."""
    dt = infer_dtype(a, dtype)
    check(lib.ks_gemm_w4a16(
        ptr(c, name="c"), ptr(a, name="a"), ptr(b_packed, name="b_packed"),
        ptr(scales, name="scales"), ptr(zeros, name="zeros"), ptr(bias, name="bias"),
        int(m), int(n), int(k), int(group_size), dt, default_stream(stream, a)),
        "ks_gemm_w4a16")
    return c


def gemm_w4a16_noalloc(c: TensorLike, a: TensorLike, b_packed: TensorLike, scales: TensorLike,
                       zeros: TensorLike, m: int, n: int, k: int, group_size: int,
                       bias: TensorLike = None, dtype: Optional[int] = None,
                       stream: TensorLike = None) -> TensorLike:
    """Extension (no reference counterpart): :func:`gemm_w4a16` with the same
    bits, for callers that cannot allocate. Split-K partials use a fixed
    16 MiB per-device array; larger needs raise ``KS_ERROR_INVALID_ARGUMENT``.
    Calls that overlap on one device race on that array."""
    dt = infer_dtype(a, dtype)
    check(lib.ks_gemm_w4a16_noalloc(
        ptr(c, name="c"), ptr(a, name="a"), ptr(b_packed, name="b_packed"),
        ptr(scales, name="scales"), ptr(zeros, name="zeros"), ptr(bias, name="bias"),
        int(m), int(n), int(k), int(group_size), dt, default_stream(stream, a)),
        "ks_gemm_w4a16_noalloc")
    return c


def gemm_fp8(out: TensorLike, a_fp8: TensorLike, b_fp8: TensorLike, a_scale: TensorLike,
             b_scale: TensorLike, m: int, n: int, k: int,
             a_mode: int = QuantMode.PER_TOKEN, b_mode: int = QuantMode.PER_CHANNEL,
             fp8_dtype: int = None, out_dtype: int = None,
             stream: TensorLike = None) -> TensorLike:
    """fp8 ``A [M,K]`` x fp8 ``B [K,N]`` -> ``C [M,N]`` in ``out_dtype``: fp32
    accumulation, then ``(acc * a_scale) * b_scale`` (reference gemm.py:228-280).
    ``fp8_dtype`` is inferred from ``a_fp8`` and ``out_dtype`` from ``out``."""
    fdt = infer_dtype(a_fp8, fp8_dtype)
    odt = _out_dtype(out, out_dtype, "ks_gemm_fp8")
    check(lib.ks_gemm_fp8(
        ptr(out, name="out"), ptr(a_fp8, name="a_fp8"), ptr(b_fp8, name="b_fp8"),
        _f32(a_scale, name="a_scale"), _f32(b_scale, name="b_scale"),
        int(m), int(n), int(k), int(a_mode), int(b_mode), fdt, odt,
        default_stream(stream, out if not isinstance(out, int) else a_fp8)), "ks_gemm_fp8")
    return out


def gemm_fp8_blockwise(out: TensorLike, a_fp8: TensorLike, b_fp8: TensorLike,
                       a_scale: TensorLike, b_scale: TensorLike, m: int, n: int, k: int,
                       block_n: int = 128, block_k: int = 128, fp8_dtype: int = None,
                       out_dtype: int = None, stream: TensorLike = None) -> TensorLike:
    """fp8 ``A [M,K]`` x fp8 ``B [K,N]`` with ``a_scale [M, ceil(K/bk)]`` and
    ``b_scale [ceil(K/bk), ceil(N/bn)]``, two-level fp32 accumulation."""
    fdt = infer_dtype(a_fp8, fp8_dtype)
    odt = _out_dtype(out, out_dtype, "ks_gemm_fp8_blockwise")
    check(lib.ks_gemm_fp8_blockwise(
        ptr(out, name="out"), ptr(a_fp8, name="a_fp8"), ptr(b_fp8, name="b_fp8"),
        _f32(a_scale, name="a_scale"), _f32(b_scale, name="b_scale"),
        int(m), int(n), int(k), int(block_n), int(block_k), fdt, odt,
        default_stream(stream, out if not isinstance(out, int) else a_fp8)),
        "ks_gemm_fp8_blockwise")
    return out


def gemm_fp8_blockwise_fused_quant(out: TensorLike, a: TensorLike, b_fp8: TensorLike,
                                   b_scale: TensorLike, m: int, n: int, k: int,
                                   block_n: int = 128, block_k: int = 128,
                                   a_dtype: int = None, fp8_dtype: int = None,
                                   out_dtype: int = None, stream: TensorLike = None) -> TensorLike:
    """Extension (no reference counterpart): ``out = gemm_fp8_blockwise(
    quantize_fp8_group(a, group_size=block_k, fp8_dtype), b_fp8, b_scale)``
    with the same bits as that two-call sequence. ``a`` is bf16/f16/f32
    ``[M, K]``; decode shapes (M <= 8) run as a single pass."""
    adt = infer_dtype(a, a_dtype)
    fdt = infer_dtype(b_fp8, fp8_dtype)
    odt = _out_dtype(out, out_dtype, "ks_gemm_fp8_blockwise_fused_quant")
    check(lib.ks_gemm_fp8_blockwise_fused_quant(
        ptr(out, name="out"), ptr(a, name="a"), ptr(b_fp8, name="b_fp8"),
        _f32(b_scale, name="b_scale"), int(m), int(n), int(k), int(block_n), int(block_k),
        adt, fdt, odt, default_stream(stream, out if not isinstance(out, int) else a)),
        "ks_gemm_fp8_blockwise_fused_quant")
    return out
