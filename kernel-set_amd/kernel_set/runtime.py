"""Device / stream / memory helpers over ``runtime.h`` (reference
``bindings/python/kernel_set/runtime.py``)."""
from __future__ import annotations

import ctypes

from ._lib import check, ks_device_properties_t, lib

__all__ = ["version", "backend_name", "device_count", "set_device", "get_device",
           "device_properties", "synchronize"]


def version() -> str:
    return lib.ks_version().decode()


def backend_name() -> str:
    return lib.ks_backend_name().decode()


def device_count() -> int:
    n = ctypes.c_int(0)
    check(lib.ks_device_count(ctypes.byref(n)), "ks_device_count")
    return n.value


def set_device(device: int) -> None:
    check(lib.ks_set_device(int(device)), "ks_set_device")


def get_device() -> int:
    d = ctypes.c_int(0)
    check(lib.ks_get_device(ctypes.byref(d)), "ks_get_device")
    return d.value


def device_properties(device: int = 0) -> dict:
    p = ks_device_properties_t()
    check(lib.ks_get_device_properties(int(device), ctypes.byref(p)), "ks_get_device_properties")
    return {f: (getattr(p, f).decode() if f == "name" else getattr(p, f))
            for f, _ in ks_device_properties_t._fields_}


def synchronize(stream: int = 0) -> None:
    check(lib.ks_stream_synchronize(ctypes.c_void_p(stream)), "ks_stream_synchronize")
