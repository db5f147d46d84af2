"""kernel_set -- MI355X-native (gfx950) quantized-inference operators.

Drop-in for the quantized-inference subset of cklxx/kernel-set's Python
package: ``kernel_set.gemm``, ``kernel_set.quant``, ``kernel_set.dispatch``
keep the reference's function names and signatures and call the hand-written
HIP library ``libkernel_set.so`` through its C ABI. There is no fallback: if the
library is missing, importing this package raises.
"""
from __future__ import annotations

from . import _lib
from ._lib import KernelSetError, check, last_error_string, lib, library_path, status_string
from ._tensor import dtype_to_ks, ks_to_torch_dtype
from .enums import Activation, DType, MemcpyKind, QuantMode, Status

__version__ = _lib.lib.ks_version().decode()

from . import gemm, moe, quant, runtime  # noqa: E402

try:
    from . import dispatch  # noqa: E402  (needs torch)
except ImportError:  # pragma: no cover
    dispatch = None

__all__ = ["gemm", "quant", "moe", "runtime", "dispatch", "KernelSetError", "check",
           "status_string", "last_error_string", "library_path", "dtype_to_ks",
           "ks_to_torch_dtype", "DType", "QuantMode", "Status", "Activation", "MemcpyKind",
           "lib"]
