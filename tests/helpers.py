"""Shared helpers for the parity tests: numpy <-> torch device tensors with
exact bit patterns, seeded input builders matching the BASELINE configs."""
from __future__ import annotations

import numpy as np

import oracle as O

try:
    import torch
except Exception:  # pragma: no cover
    torch = None


def dev():
    return torch.device("cuda:0")


def to_dev_bf16(x_f32):
    """fp32 numpy values (already bf16-representable or not) -> bf16 device
    tensor holding round_bf16(x); returns (tensor, exact fp32 values)."""
    bits = O.f32_to_bf16_bits(x_f32)
    t = torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).to(dev())
    return t, O.bf16_bits_to_f32(bits)


def to_dev_f16(x_f32):
    h = np.ascontiguousarray(x_f32, np.float32).astype(np.float16)
    return torch.from_numpy(h).to(dev()), h.astype(np.float32)


def to_dev(x_f32, dtype: str):
    if dtype == "bf16":
        return to_dev_bf16(x_f32)
    if dtype == "f16":
        return to_dev_f16(x_f32)
    x = np.ascontiguousarray(x_f32, np.float32)
    return torch.from_numpy(x).to(dev()), x


def from_dev_f32(t) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def u8(t) -> np.ndarray:
    return t.detach().contiguous().view(torch.uint8).cpu().numpy()


def np_u8_dev(a):
    return torch.from_numpy(np.ascontiguousarray(a, np.uint8)).to(dev())


def np_i8_dev(a):
    return torch.from_numpy(np.ascontiguousarray(a, np.int8)).to(dev())


def np_f32_dev(a):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(dev())


def np_i32_dev(a):
    return torch.from_numpy(np.ascontiguousarray(a, np.int32)).to(dev())


def torch_dtype(name: str):
    return {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}[name]


# ---- config builders (seeded) ----------------------
def w4a16_inputs(m, k, n, gs=128, zero_mode="fixed8", seed=0):
    """Activations ~N(0,1); codes U[0,15]; scales U[0.002,0.02]; zeros fixed 8
    (config 1) or integer-valued U{6..9} (config 2)."""
    rng = np.random.default_rng(seed)
    a = rng.standard_normal((m, k), dtype=np.float32)
    codes = rng.integers(0, 16, (k, n), dtype=np.uint8)
    ng = k // gs
    scales = rng.uniform(0.002, 0.02, (ng, n)).astype(np.float32)
    if zero_mode == "fixed8":
        zeros = np.full((ng, n), 8.0, np.float32)
    elif zero_mode == "int69":
        zeros = rng.integers(6, 10, (ng, n)).astype(np.float32)
    else:
        zeros = None
    return a, codes, scales, zeros
