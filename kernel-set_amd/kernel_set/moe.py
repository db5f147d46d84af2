"""Grouped W4A16 GEMM for Mixture-of-Experts (extension, ``moe_w4a16.h``).

The reference has no quantized grouped GEMM; this follows the argument order of
its dense ``grouped_gemm`` (``bindings/python/kernel_set/moe.py:189-217``) with
the weight replaced by the ``gemm_w4a16`` format.
"""
from __future__ import annotations

from ctypes import POINTER, c_int32, cast
from typing import Optional

from ._lib import check, lib
from ._tensor import TensorLike, default_stream, infer_dtype, ptr

__all__ = ["grouped_gemm_w4a16"]


def grouped_gemm_w4a16(c: TensorLike, a: TensorLike, b_packed: TensorLike,
                       scales: TensorLike, zeros: TensorLike, expert_offsets: TensorLike,
                       num_experts: int, total_rows: int, n: int, k: int,
                       group_size: int = 128, dtype: Optional[int] = None,
                       stream: TensorLike = None) -> TensorLike:
    """For each expert e: ``C[off_e:off_{e+1}] = A[off_e:off_{e+1}] @ dequant(B_e)``.

    a ``[total_rows, k]``; b_packed uint8 ``[E, k/2, n]``; scales/zeros
    ``[E, k/group_size, n]`` (zeros may be None); expert_offsets int32 ``[E+1]``."""
    dt = infer_dtype(a, dtype)
    offs = cast(ptr(expert_offsets, name="expert_offsets", allow_none=False), POINTER(c_int32))
    check(lib.ks_moe_grouped_gemm_w4a16(
        ptr(c, name="c"), ptr(a, name="a"), ptr(b_packed, name="b_packed"),
        ptr(scales, name="scales"), ptr(zeros, name="zeros"), offs, int(num_experts),
        int(total_rows), int(n), int(k), int(group_size), dt, default_stream(stream, a)),
        "ks_moe_grouped_gemm_w4a16")
    return c
