"""``ks.dispatch`` entry points for the quantized-inference ops.

Signatures follow the reference's ``bindings/python/kernel_set/dispatch.py``
(``fp8_gemm`` :321-324, ``int8_gemm`` :327-331, ``w4a16`` :334-337, ``fp8_gemm_blockwise`` :377-384,
``per_token_group_quant`` :387-391, ``moe`` :539-543) and the output allocation
of its kernel-set adapters (``backends/_registry.py:464-492,723-731,1204-1218``).
There is exactly one provider, the native gfx950 library: no routing, no
fallback. Introspection helpers report that single provider.
"""
from __future__ import annotations

import weakref

import torch

from . import gemm as _gemm
from . import moe as _moe
from . import quant as _quant
from ._tensor import dtype_to_ks
from .enums import DType

PROVIDER = "kernel-set"
_OPS = ("w4a16", "int8_gemm", "fp8_gemm", "fp8_gemm_blockwise", "per_token_group_quant", "moe")

__all__ = list(_OPS) + ["which", "available", "providers", "chain", "ops"]


def w4a16(a, b_packed, scales, zeros, *, group_size=128, **kw):
    """W4A16 GEMM; ``n = scales.shape[1]``, output dtype = ``a.dtype``."""
    m, k = a.shape
    n = scales.shape[1]
    c = torch.empty(m, n, device=a.device, dtype=a.dtype)
    _gemm.gemm_w4a16(c, a, b_packed, scales, zeros, m=m, n=n, k=k, group_size=group_size,
                     bias=kw.get("bias"))
    return c


def int8_gemm(a8, b8, a_scale, b_scale, *, out_dtype=None, **kw):
    """W8A8 scaled GEMM; B is ``[K, N]``; per-token ``a_scale`` and per-channel
    ``b_scale`` (a one-element scale selects per-tensor); default bf16 out."""
    m, k = a8.shape
    n = b8.shape[1]
    out = torch.empty(m, n, device=a8.device, dtype=out_dtype or torch.bfloat16)
    from .enums import QuantMode
    a_mode = QuantMode.PER_TOKEN if a_scale.numel() == m and m != 1 else QuantMode.PER_TENSOR
    b_mode = QuantMode.PER_CHANNEL if b_scale.numel() == n and n != 1 else QuantMode.PER_TENSOR
    if m == 1 and a_scale.numel() == 1:
        a_mode = QuantMode.PER_TOKEN
    if n == 1 and b_scale.numel() == 1:
        b_mode = QuantMode.PER_CHANNEL
    _gemm.gemm_w8a8(out, a8, b8, a_scale, b_scale, m=m, n=n, k=k, bias=kw.get("bias"),
                    a_mode=a_mode, b_mode=b_mode, out_dtype=dtype_to_ks(out.dtype))
    return out


# [N, K] fp8 weight -> its [K, N] copy, made once per weight tensor: keyed on
# the tensor's identity (the entry is dropped when the weight is freed) and
# revalidated against its storage pointer, shape, strides and in-place version.
_KN_CACHE: dict = {}


def _weight_kn(b8):
    key = (b8.data_ptr(), tuple(b8.shape), tuple(b8.stride()), b8._version)
    ent = _KN_CACHE.get(id(b8))
    if ent is not None and ent[2]() is b8 and ent[0] == key:
        return ent[1]
    kn = b8.t().contiguous()
    ident = id(b8)
    _KN_CACHE[ident] = (key, kn, weakref.ref(b8, lambda _r, i=ident: _KN_CACHE.pop(i, None)))
    return kn


def fp8_gemm(a8, b8, a_scale, b_scale, *, out_dtype=None, **kw):
    """Scaled fp8 GEMM ``C = (a_scale (x) b_scale) * (a8 @ b8.T)``. ``b8`` is
    ``[N, K]`` (the NT weight layout of the reference's fp8_gemm providers,
    ``backends/_registry.py:427-442``); ``a_scale`` is ``[M]``/``[M,1]`` or one
    element, ``b_scale`` ``[N]``/``[1,N]`` or one element; default bf16 out.
    ``ks_gemm_fp8`` takes B as ``[K, N]``; the transposed copy is made on the
    first call with a given weight tensor and reused while that tensor lives
    unmodified, so steady-state calls move no extra weight bytes."""
    m, k = a8.shape
    n = b8.shape[0]
    out = torch.empty(m, n, device=a8.device, dtype=out_dtype or torch.bfloat16)
    from .enums import QuantMode
    a_mode = QuantMode.PER_TENSOR if a_scale.numel() == 1 else QuantMode.PER_TOKEN
    b_mode = QuantMode.PER_TENSOR if b_scale.numel() == 1 else QuantMode.PER_CHANNEL
    if a_mode == QuantMode.PER_TOKEN and a_scale.numel() != m:
        raise ValueError(f"fp8_gemm: a_scale must have 1 or M={m} elements")
    if b_mode == QuantMode.PER_CHANNEL and b_scale.numel() != n:
        raise ValueError(f"fp8_gemm: b_scale must have 1 or N={n} elements")
    b_kn = _weight_kn(b8)
    _gemm.gemm_fp8(out, a8, b_kn, a_scale.contiguous(), b_scale.contiguous(), m=m, n=n, k=k,
                   a_mode=a_mode, b_mode=b_mode, out_dtype=dtype_to_ks(out.dtype))
    return out


def fp8_gemm_blockwise(a8, b8, a_scale, b_scale, *, block_n=128, block_k=128,
                       out_dtype=None, **kw):
    """fp8 blockwise GEMM (1 x block_k activation tiles, block_k x block_n weight
    blocks); B is ``[K, N]``; default bf16 out."""
    m, k = a8.shape
    n = b8.shape[1]
    out = torch.empty(m, n, device=a8.device, dtype=out_dtype or torch.bfloat16)
    _gemm.gemm_fp8_blockwise(out, a8, b8, a_scale, b_scale, m=m, n=n, k=k,
                             block_n=block_n, block_k=block_k)
    return out


def per_token_group_quant(x, *, group_size=128, fp8_dtype=None, **kw):
    """1 x group_size dynamic fp8 quant -> ``(fp8 [rows, cols], fp32 scale)``."""
    rows, cols = x.shape
    ng = (cols + group_size - 1) // group_size
    fdt = DType.F8E4M3 if fp8_dtype is None else int(fp8_dtype)
    tdt = torch.float8_e4m3fn if fdt == DType.F8E4M3 else torch.float8_e5m2
    out = torch.empty(rows, cols, device=x.device, dtype=tdt)
    scale = torch.empty(rows, ng, device=x.device, dtype=torch.float32)
    _quant.quantize_fp8_group(out, scale, x, rows=rows, cols=cols, group_size=group_size,
                              fp8_dtype=fdt)
    return out, scale


def moe(a, b, expert_offsets, *, num_experts, n, k, scales=None, zeros=None,
        group_size=128, **kw):
    """Grouped expert GEMM over CSR ``expert_offsets``.

    Dense form (the reference's kernel-set provider, ``_registry.py:1040-1046``):
    ``b`` is ``[E, k, n]`` of ``a``'s dtype, ``scales`` is None. W4A16 form
    (extension): ``b`` is uint8 ``[E, k/2, n]`` with ``scales``/``zeros``
    ``[E, k/group_size, n]``. Returns ``C [total_rows, n]`` of ``a``'s dtype;
    rows outside every expert's range are left as ``torch.empty`` made them."""
    total_rows = a.shape[0]
    c = torch.empty(total_rows, n, device=a.device, dtype=a.dtype)
    if scales is None:
        _moe.grouped_gemm(c, a, b, expert_offsets, num_experts, total_rows, n, k)
    else:
        _moe.grouped_gemm_w4a16(c, a, b, scales, zeros, expert_offsets, num_experts,
                                total_rows, n, k, group_size=group_size)
    return c


def ops():
    return list(_OPS)


def providers(op=None):
    return [PROVIDER]


def chain(op):
    if op not in _OPS:
        raise KeyError(op)
    return [PROVIDER]


def available(op):
    return op in _OPS


def which(op, *args, **kwargs):
    if op not in _OPS:
        raise KeyError(op)
    return PROVIDER
