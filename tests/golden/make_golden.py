"""Regenerate the committed golden fixtures from the CPU oracle.

The reference repository commits no golden vectors for this path (its only
kernel-level quant test, kernels/tests/test_quant.cu:34-139, compares int8
codes within +-1 of a division-based host reference). These fixtures freeze the
oracle's outputs on small seeded inputs so that (a) the oracle itself cannot
drift silently and (b) GPU tests have byte-exact expectations that travel to
the GPU box without the oracle build. The oracle is pinned independently in
tests/test_oracle.py (torch's fp8 casts, closed forms, brute force).

Run: python tests/golden/make_golden.py
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
import oracle as O  # noqa: E402


def quant_int8_refcase():
    # test_quant.cu:34-40: rows=6, cols=130, xorshift32 seed 11, range +-5,
    # inputs narrowed to the storage dtype (test_common.cuh:112-121).
    x = O.xorshift32_uniform(6 * 130, 11, -5.0, 5.0).reshape(6, 130)
    out = {"x_f32": x}
    for dt in ("f32", "f16", "bf16"):
        xs = O.round_to(x, dt)
        q, s = O.quant_row(xs, O.INT8)
        out[f"{dt}_tok_q"], out[f"{dt}_tok_s"] = q, s
        q, s = O.quant_tensor(xs, O.INT8)
        out[f"{dt}_ten_q"], out[f"{dt}_ten_s"] = q, s
    return out


def quant_fp8_group():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((8, 300)).astype(np.float32)
    idx = rng.choice(x.size, 6, replace=False)
    x.flat[idx] *= 50.0
    x[5] = 0.0  # all-zero row -> scale 1e-12, codes 0
    xb = O.round_bf16(x)
    out = {"x_bf16_vals": xb}
    for name, fmt in (("e4m3", O.E4M3), ("e5m2", O.E5M2)):
        q, s = O.quant_group(xb, 128, fmt)
        out[f"{name}_q"], out[f"{name}_s"] = q, s
        q, s = O.quant_row(xb, fmt)
        out[f"{name}_tok_q"], out[f"{name}_tok_s"] = q, s
    return out


def w4a16_small():
    rng = np.random.default_rng(5)
    m, k, n, gs = 3, 256, 64, 64
    a = O.round_bf16(rng.standard_normal((m, k)).astype(np.float32))
    codes = rng.integers(0, 16, (k, n), dtype=np.uint8)
    b = O.pack_k2_uint8(codes)
    s = O.round_bf16(rng.uniform(0.002, 0.02, (k // gs, n)).astype(np.float32))
    z = O.round_bf16(rng.integers(6, 10, (k // gs, n)).astype(np.float32))
    bias = O.round_bf16(rng.standard_normal(n).astype(np.float32))
    c = O.w4a16_scalar(a, b, s, z, gs, bias)
    return {"a": a, "b_packed": b, "scales": s, "zeros": z, "bias": bias,
            "c_f32": c, "gs": np.int32(gs)}


def fp8_blockwise_small():
    rng = np.random.default_rng(7)
    m, n, k, bn, bk = 40, 72, 200, 64, 64
    a8, a_s = O.quant_group(rng.standard_normal((m, k)).astype(np.float32), bk, O.E4M3)
    w = (rng.standard_normal((k, n)) * 0.02).astype(np.float32)
    nkb, nnb = -(-k // bk), -(-n // bn)
    b_s = np.empty((nkb, nnb), np.float32)
    b8 = np.empty((k, n), np.uint8)
    for i in range(nkb):
        for j in range(nnb):
            blk = w[i * bk:(i + 1) * bk, j * bn:(j + 1) * bn]
            sc = np.float32(max(np.float32(np.abs(blk).max()) / np.float32(448.0), np.float32(1e-12)))
            b_s[i, j] = sc
            b8[i * bk:(i + 1) * bk, j * bn:(j + 1) * bn] = O.fp8_encode(blk * (np.float32(1) / sc))
    c = O.fp8_blockwise_scalar(a8, b8, a_s, b_s, bn, bk)
    return {"a8": a8, "b8": b8, "a_scale": a_s, "b_scale": b_s, "c_f32": c,
            "bn": np.int32(bn), "bk": np.int32(bk)}


def w8a8_small():
    rng = np.random.default_rng(9)
    m, n, k = 33, 47, 100
    a = rng.integers(-127, 128, (m, k)).astype(np.int8)
    b = rng.integers(-127, 128, (k, n)).astype(np.int8)
    a_s = rng.uniform(0.01, 0.03, m).astype(np.float32)
    b_s = rng.uniform(0.01, 0.03, n).astype(np.float32)
    acc = O.w8a8_acc_scalar(a, b)
    c = O.w8a8_epilogue(acc, a_s, b_s)
    return {"a": a, "b": b, "a_scale": a_s, "b_scale": b_s, "acc": acc, "c_f32": c}


FIXTURES = {
    "quant_int8_refcase": quant_int8_refcase,
    "quant_fp8_group": quant_fp8_group,
    "w4a16_small": w4a16_small,
    "fp8_blockwise_small": fp8_blockwise_small,
    "w8a8_small": w8a8_small,
}


def main():
    for name, fn in FIXTURES.items():
        path = os.path.join(HERE, name + ".npz")
        np.savez_compressed(path, **fn())
        print(path, os.path.getsize(path))


if __name__ == "__main__":
    main()
