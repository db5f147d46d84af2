"""ctypes loader for ``libkernel_set.so`` (the gfx950 HIP build).

Mirrors the reference loader (``bindings/python/kernel_set/_lib.py:210-340``):
``KERNEL_SET_LIB`` (full path) or ``KERNEL_SET_LIB_DIR`` override the search,
otherwise the library next to this package is used. Symbols are declared with
exact argtypes; a symbol the library lacks is recorded in ``_MISSING`` and only
fails when called. Non-zero statuses raise :class:`KernelSetError` carrying the
symbolic status name and ``ks_last_error_string()``.

torch (when installed) is imported before the library is opened, so the HIP
runtime torch ships is the one both use: one process, one HIP runtime.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_char_p, c_float, c_int, c_int32, c_int64, c_size_t, c_void_p
from typing import Optional

try:  # share torch's HIP runtime when torch is present
    import torch as _torch  # noqa: F401
except Exception:  # pragma: no cover
    _torch = None

KS_SUCCESS = 0
KS_ERROR_INVALID_ARGUMENT = 1
KS_ERROR_UNSUPPORTED_DTYPE = 2
KS_ERROR_UNSUPPORTED_SHAPE = 3
KS_ERROR_CUDA = 4
KS_ERROR_NOT_IMPLEMENTED = 5
KS_ERROR_OUT_OF_MEMORY = 6
KS_ERROR_ARCH_UNSUPPORTED = 7
KS_ERROR_INTERNAL = 8

KS_DTYPE_F32 = 0
KS_DTYPE_F16 = 1
KS_DTYPE_BF16 = 2
KS_DTYPE_F8E4M3 = 3
KS_DTYPE_F8E5M2 = 4
KS_DTYPE_F64 = 5
KS_DTYPE_I64 = 6
KS_DTYPE_I32 = 7
KS_DTYPE_I8 = 8
KS_DTYPE_U8 = 9
KS_DTYPE_I4 = 10

KS_QUANT_PER_TENSOR = 0
KS_QUANT_PER_TOKEN = 1
KS_QUANT_PER_CHANNEL = 2
KS_QUANT_GROUPWISE = 3


class KernelSetError(RuntimeError):
    """A kernel-set entry point returned a status other than KS_SUCCESS."""

    def __init__(self, status: int, name: str, backend_message: str = "",
                 func: Optional[str] = None):
        self.status = int(status)
        self.status_name = name
        self.backend_message = backend_message
        self.func = func
        msg = f"{func}: {name}" if func else name
        if backend_message:
            msg += f": {backend_message}"
        super().__init__(msg)


class ks_device_properties_t(ctypes.Structure):
    _fields_ = [
        ("name", ctypes.c_char * 256),
        ("compute_major", c_int),
        ("compute_minor", c_int),
        ("multiprocessor_count", c_int),
        ("max_threads_per_block", c_int),
        ("max_shared_memory_per_block", c_int),
        ("warp_size", c_int),
        ("total_global_memory", c_size_t),
        ("supports_bf16", c_int),
        ("supports_fp8", c_int),
        ("supports_tf32", c_int),
    ]


HERE = os.path.dirname(os.path.abspath(__file__))
LIB_NAME = "libkernel_set.so"


def library_path() -> str:
    explicit = os.environ.get("KERNEL_SET_LIB")
    if explicit:
        return os.path.expanduser(explicit)
    d = os.environ.get("KERNEL_SET_LIB_DIR")
    if d:
        return os.path.join(os.path.expanduser(d), LIB_NAME)
    return os.path.join(HERE, LIB_NAME)


def _load() -> ctypes.CDLL:
    path = library_path()
    if not os.path.isfile(path):
        raise OSError(
            f"kernel_set: {path} not found. Build it with "
            "`python kernel-set_amd/build.py` (or __graft_entry__.build()); "
            "there is no fallback implementation.")
    return ctypes.CDLL(path)


lib: ctypes.CDLL = _load()

_VP = c_void_p
_I64 = c_int64
_I = c_int
_F32P = POINTER(c_float)
_I32P = POINTER(c_int32)
_MISSING: list = []


def _decl(name, argtypes, restype=c_int):
    try:
        fn = getattr(lib, name)
    except AttributeError:
        _MISSING.append(name)
        return
    fn.argtypes = argtypes
    fn.restype = restype


# runtime.h
_decl("ks_version", [], c_char_p)
_decl("ks_status_string", [_I], c_char_p)
_decl("ks_dtype_size_bits", [_I], _I)
_decl("ks_dtype_name", [_I], c_char_p)
_decl("ks_backend_name", [], c_char_p)
_decl("ks_last_error_string", [], c_char_p)
_decl("ks_device_count", [POINTER(c_int)])
_decl("ks_set_device", [_I])
_decl("ks_get_device", [POINTER(c_int)])
_decl("ks_get_device_properties", [_I, POINTER(ks_device_properties_t)])
_decl("ks_stream_create", [POINTER(c_void_p)])
_decl("ks_stream_destroy", [_VP])
_decl("ks_stream_synchronize", [_VP])
_decl("ks_malloc_device", [POINTER(c_void_p), c_size_t])
_decl("ks_free_device", [_VP])
_decl("ks_memcpy", [_VP, _VP, c_size_t, _I, _VP])
_decl("ks_memset_device", [_VP, _I, c_size_t, _VP])
# gemm.h
_decl("ks_gemm_w8a8", [_VP, _VP, _VP, _F32P, _F32P, _VP, _I64, _I64, _I64, _I, _I, _I, _VP])
_decl("ks_gemm_w4a16", [_VP, _VP, _VP, _VP, _VP, _VP, _I64, _I64, _I64, _I, _I, _VP])
_decl("ks_gemm_w4a16_noalloc", [_VP, _VP, _VP, _VP, _VP, _VP, _I64, _I64, _I64, _I, _I, _VP])
_decl("ks_gemm_fp8", [_VP, _VP, _VP, _F32P, _F32P, _I64, _I64, _I64, _I, _I, _I, _I, _VP])
_decl("ks_gemm_fp8_blockwise",
      [_VP, _VP, _VP, _F32P, _F32P, _I64, _I64, _I64, _I, _I, _I, _I, _VP])
# extension of this build (no reference counterpart)
_decl("ks_gemm_fp8_blockwise_fused_quant",
      [_VP, _VP, _VP, _F32P, _I64, _I64, _I64, _I, _I, _I, _I, _I, _VP])
_decl("ks_gemm_w8a8_fused_quant",
      [_VP, _VP, _VP, _F32P, _VP, _I64, _I64, _I64, _I, _I, _I, _I, _VP])
# quant.h
_decl("ks_quantize_fp8", [_VP, _F32P, _VP, _I64, _I64, _I, _I, _I, _VP])
_decl("ks_dequantize_fp8", [_VP, _VP, _F32P, _I64, _I64, _I, _I, _I, _VP])
_decl("ks_quantize_fp8_group", [_VP, _F32P, _VP, _I64, _I64, _I, _I, _I, _VP])
_decl("ks_quantize_int8", [_VP, _F32P, _VP, _I64, _I64, _I, _I, _VP])
_decl("ks_dequantize_int8", [_VP, _VP, _F32P, _I64, _I64, _I, _I, _VP])
_decl("ks_dequantize_int4", [_VP, _VP, _VP, _VP, _I64, _I64, _I, _I, _VP])
_decl("ks_repack_int4", [_VP, _VP, _VP, _I64, _I64, _I, _VP])
# moe.h (routing)
_decl("ks_moe_gate_softmax_topk", [_F32P, _I32P, _VP, _I64, _I, _I, _I, _I, _VP])
_decl("ks_moe_gate_sigmoid_group_topk",
      [_F32P, _I32P, _VP, _VP, _I64, _I, _I, _I, _I, _I, c_float, _I, _VP])
_decl("ks_moe_compute_permutation", [_I32P, _I32P, _I32P, _I64, _I, _I, _VP])
_decl("ks_moe_permute", [_VP, _VP, _I32P, _I64, _I, _I64, _I, _VP])
_decl("ks_moe_unpermute", [_VP, _VP, _I32P, _F32P, _I64, _I, _I64, _I, _VP])
_decl("ks_moe_grouped_gemm", [_VP, _VP, _VP, _I32P, _I, _I64, _I64, _I64, _I, _VP])
# moe_w4a16.h (extension)
_decl("ks_moe_grouped_gemm_w4a16",
      [_VP, _VP, _VP, _VP, _VP, _I32P, _I, _I64, _I64, _I64, _I, _I, _VP])
# testing.h (test hook, not reference ABI)
_decl("ks_testing_gemm_w8a8_i32", [_I32P, _VP, _VP, _I64, _I64, _I64, _VP])
_decl("ks_testing_round_bits", [_VP, ctypes.c_uint32, _I64, _I, _VP])


def status_string(status: int) -> str:
    raw = lib.ks_status_string(int(status))
    return raw.decode() if raw else f"status {status}"


def last_error_string() -> str:
    raw = lib.ks_last_error_string()
    return raw.decode("utf-8", "replace") if raw else ""


def check(status: int, func: Optional[str] = None) -> None:
    if status == KS_SUCCESS:
        return
    raise KernelSetError(status, status_string(status), last_error_string(), func)
