"""IntEnum mirrors of the C ABI enums (``include/kernel_set/types.h``,
``runtime.h``); same names and values as the reference's
``bindings/python/kernel_set/enums.py:15-69``."""
from __future__ import annotations

from enum import IntEnum

__all__ = ["Status", "DType", "Activation", "QuantMode", "MemcpyKind"]


class Status(IntEnum):
    SUCCESS = 0
    ERROR_INVALID_ARGUMENT = 1
    ERROR_UNSUPPORTED_DTYPE = 2
    ERROR_UNSUPPORTED_SHAPE = 3
    ERROR_CUDA = 4
    ERROR_NOT_IMPLEMENTED = 5
    ERROR_OUT_OF_MEMORY = 6
    ERROR_ARCH_UNSUPPORTED = 7
    ERROR_INTERNAL = 8


class DType(IntEnum):
    F32 = 0
    F16 = 1
    BF16 = 2
    F8E4M3 = 3
    F8E5M2 = 4
    F64 = 5
    I64 = 6
    I32 = 7
    I8 = 8
    U8 = 9
    I4 = 10


class Activation(IntEnum):
    NONE = 0
    RELU = 1
    GELU = 2
    GELU_TANH = 3
    SILU = 4


class QuantMode(IntEnum):
    PER_TENSOR = 0
    PER_TOKEN = 1
    PER_CHANNEL = 2
    GROUPWISE = 3


class MemcpyKind(IntEnum):
    HOST_TO_DEVICE = 0
    DEVICE_TO_HOST = 1
    DEVICE_TO_DEVICE = 2
