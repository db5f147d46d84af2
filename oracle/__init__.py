"""CPU oracle for the quantized-inference path -- TEST INFRASTRUCTURE ONLY.

Restates the arithmetic of cklxx/kernel-set's reference kernels and of its
benchmark references so the HIP library can be checked against it:

* scalar C (``ks_oracle.c``, built by ``oracle/build.py``): fp8 codec,
  quantizers, int4 repack/dequant, and scalar GEMMs in the reference kernels'
  operation order;
* NumPy: the "dequantize, then fp32 matmul" references of
  ``benchmarks/bench.py:1228-1235,1274-1285,1434-1470`` that the GEMM
  tolerances are stated against, plus small helpers (bf16 rounding, packing,
  the reference tests' xorshift32 generator).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this package, and only as the checker.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libks_oracle.so")

E4M3, E5M2, INT8 = 0, 1, 2  # quantizer targets (fp8 formats share 0/1)
QMAX = {E4M3: 448.0, E5M2: 57344.0, INT8: 127.0}

_lib = None


def lib() -> ctypes.CDLL:
    """Load (building if needed) the scalar C oracle."""
    global _lib
    if _lib is None:
        if not os.path.isfile(_LIB_PATH):
            from . import build as _b
            _b.build()
        L = ctypes.CDLL(_LIB_PATH)
        P = ctypes.c_void_p
        I64 = ctypes.c_int64
        I = ctypes.c_int
        sig = {
            "oracle_fp8_encode": [P, P, I64, I],
            "oracle_fp8_decode": [P, P, I64, I],
            "oracle_quant_group": [P, P, P, I64, I64, I64, I],
            "oracle_quant_row": [P, P, P, I64, I64, I],
            "oracle_quant_tensor": [P, P, P, I64, I],
            "oracle_repack_int4": [P, P, P, I64, I64],
            "oracle_dequant_int4": [P, P, P, P, I64, I64, I64],
            "oracle_w4a16": [P, P, P, P, P, P, I64, I64, I64, I64],
            "oracle_fp8_blockwise": [P, P, P, P, P, I64, I64, I64, I64, I64, I],
            "oracle_fp8_gemm": [P, P, P, P, P, I64, I64, I64, I, I, I],
            "oracle_w8a8_acc": [P, P, P, I64, I64, I64],
            "oracle_w8a8_epilogue": [P, P, P, P, P, I64, I64, I, I],
            "oracle_grouped_gemm": [P, P, P, I, P, I64, I64, I64],
        }
        for name, args in sig.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = None
        _lib = L
    return _lib


def _p(arr):
    return None if arr is None else arr.ctypes.data


def _c(arr, dtype):
    return np.ascontiguousarray(arr, dtype=dtype)


# ---------------------------------------------------------------------------
# 16-bit float helpers
# ---------------------------------------------------------------------------
def f32_to_bf16_bits(x) -> np.ndarray:
    """fp32 -> bf16 bit patterns, round to nearest even (NaN -> quiet NaN)."""
    u = _c(x, np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(_c(x, np.float32))
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_bits_to_f32(h) -> np.ndarray:
    return (_c(h, np.uint16).astype(np.uint32) << 16).view(np.float32)


def round_bf16(x) -> np.ndarray:
    """Round fp32 values to the nearest bf16 value, returned as fp32."""
    return bf16_bits_to_f32(f32_to_bf16_bits(x))


def round_f16(x) -> np.ndarray:
    return _c(x, np.float32).astype(np.float16).astype(np.float32)


def round_to(x, dtype: str) -> np.ndarray:
    if dtype == "bf16":
        return round_bf16(x)
    if dtype == "f16":
        return round_f16(x)
    return _c(x, np.float32)


# ---------------------------------------------------------------------------
# fp8 / int8 quantization (scalar C)
# ---------------------------------------------------------------------------
def fp8_encode(x, fmt: int = E4M3) -> np.ndarray:
    x = _c(x, np.float32)
    out = np.empty(x.shape, np.uint8)
    lib().oracle_fp8_encode(_p(x), _p(out), x.size, fmt)
    return out


def fp8_decode(c, fmt: int = E4M3) -> np.ndarray:
    c = _c(c, np.uint8)
    out = np.empty(c.shape, np.float32)
    lib().oracle_fp8_decode(_p(c), _p(out), c.size, fmt)
    return out


def quant_group(x, group_size: int, target: int = E4M3):
    """Per-(row, 1 x group_size) dynamic quant (quant_fp8_group.cu:74-107).

    Returns (codes uint8 [rows, cols], scale fp32 [rows, ceil(cols/gs)])."""
    x = _c(x, np.float32)
    rows, cols = x.shape
    ng = (cols + group_size - 1) // group_size
    out = np.empty((rows, cols), np.uint8)
    sc = np.empty((rows, ng), np.float32)
    lib().oracle_quant_group(_p(x), _p(out), _p(sc), rows, cols, group_size, target)
    return out, sc


def quant_row(x, target: int = E4M3):
    """Per-token dynamic quant (quant_fp8.cu:42-66, quant_int8.cu:23-47)."""
    x = _c(x, np.float32)
    rows, cols = x.shape
    out = np.empty((rows, cols), np.uint8)
    sc = np.empty((rows,), np.float32)
    lib().oracle_quant_row(_p(x), _p(out), _p(sc), rows, cols, target)
    return out, sc


def quant_tensor(x, target: int = E4M3):
    """Per-tensor dynamic quant (quant_fp8.cu:69-100, quant_int8.cu:50-83)."""
    x = _c(x, np.float32)
    out = np.empty(x.shape, np.uint8)
    sc = np.empty((1,), np.float32)
    lib().oracle_quant_tensor(_p(x), _p(out), _p(sc), x.size, target)
    return out, sc


def dequant(codes, scale, target: int, per_token: bool) -> np.ndarray:
    """float(code) * scale in fp32 (quant_fp8.cu:103-115, quant_int8.cu:86-99)."""
    if target == INT8:
        v = _c(codes, np.uint8).view(np.int8).astype(np.float32)
    else:
        v = fp8_decode(codes, target)
    s = _c(scale, np.float32)
    s = s.reshape(-1, 1) if per_token else s.reshape(1, 1)
    return (v * s).astype(np.float32)


# ---------------------------------------------------------------------------
# int4 weight formats
# ---------------------------------------------------------------------------
def pack_k8_int32(codes) -> np.ndarray:
    """codes uint8 [K, N] in 0..15 -> int32 [K/8, N], code k in nibble k % 8."""
    q = _c(codes, np.uint32)
    k, n = q.shape
    q = q.reshape(k // 8, 8, n)
    w = np.zeros((k // 8, n), np.uint32)
    for j in range(8):
        w |= q[:, j, :] << np.uint32(4 * j)
    return w.view(np.int32)


def pack_k2_uint8(codes) -> np.ndarray:
    """codes [K, N] -> uint8 [K/2, N]: even k in bits 0-3, odd k in bits 4-7
    (gemm_w4a16.cu:6-13)."""
    q = _c(codes, np.uint8)
    return (q[0::2] & 0xF) | ((q[1::2] & 0xF) << 4)


def unpack_k2_uint8(b) -> np.ndarray:
    b = _c(b, np.uint8)
    kp, n = b.shape
    out = np.empty((2 * kp, n), np.uint8)
    out[0::2] = b & 0xF
    out[1::2] = b >> 4
    return out


def repack_int4(qweight, perm=None) -> np.ndarray:
    """repack_int4.cu:10-34 (+ act-order perm: output row k <- input row perm[k])."""
    q = _c(qweight, np.int32).view(np.uint32)
    k8, n = q.shape
    out = np.empty((k8 * 4, n), np.uint8)
    pp = None if perm is None else _c(perm, np.int32)
    lib().oracle_repack_int4(_p(q), _p(pp), _p(out), k8 * 8, n)
    return out


def dequant_int4(qweight, scales, zeros, group_size: int) -> np.ndarray:
    """dequant_int4.cu:47-58 in fp32 (caller rounds to the output dtype)."""
    q = _c(qweight, np.int32).view(np.uint32)
    k8, n = q.shape
    s = _c(scales, np.float32)
    z = _c(zeros, np.float32)
    out = np.empty((k8 * 8, n), np.float32)
    lib().oracle_dequant_int4(_p(q), _p(s), _p(z), _p(out), k8 * 8, n, group_size)
    return out


# ---------------------------------------------------------------------------
# GEMM references
# ---------------------------------------------------------------------------
def w4a16_scalar(a, b_packed, scales, zeros, group_size, bias=None) -> np.ndarray:
    """gemm_w4a16.cu:74-129 order, fp32 result (before rounding to dtype)."""
    a = _c(a, np.float32)
    b = _c(b_packed, np.uint8)
    m, k = a.shape
    n = b.shape[1]
    s = _c(scales, np.float32)
    z = None if zeros is None else _c(zeros, np.float32)
    bb = None if bias is None else _c(bias, np.float32)
    out = np.empty((m, n), np.float32)
    lib().oracle_w4a16(_p(a), _p(b), _p(s), _p(z), _p(bb), _p(out), m, n, k, group_size)
    return out


def w4a16_dequant_weight(b_packed, scales, zeros, group_size, dtype="bf16") -> np.ndarray:
    """bench.py:1274-1284: codes -> (codes - z) * s in fp32, rounded to dtype."""
    codes = unpack_k2_uint8(b_packed).astype(np.float32)
    k = codes.shape[0]
    g = np.arange(k) // group_size
    z = 0.0 if zeros is None else _c(zeros, np.float32)[g]
    w = (codes - z) * _c(scales, np.float32)[g]
    return round_to(w, dtype)


def w4a16_ref(a, b_packed, scales, zeros, group_size, dtype="bf16", bias=None,
              weight=None) -> np.ndarray:
    """bench.py:1274-1285: a.float() @ dequant(weight).float() (+ bias), fp32."""
    if weight is None:
        weight = w4a16_dequant_weight(b_packed, scales, zeros, group_size, dtype)
    out = _c(a, np.float32) @ weight
    if bias is not None:
        out = out + _c(bias, np.float32)[None, :]
    return out.astype(np.float32)


def fp8_blockwise_scalar(a8, b8, a_scale, b_scale, block_n, block_k, fmt=E4M3):
    """gemm_fp8_blockwise.cu:107-161 (two-level fp32 accumulation)."""
    a8 = _c(a8, np.uint8)
    b8 = _c(b8, np.uint8)
    m, k = a8.shape
    n = b8.shape[1]
    out = np.empty((m, n), np.float32)
    lib().oracle_fp8_blockwise(_p(a8), _p(b8), _p(_c(a_scale, np.float32)),
                               _p(_c(b_scale, np.float32)), _p(out), m, n, k,
                               block_n, block_k, fmt)
    return out


def fp8_blockwise_dequant(a8, b8, a_scale, b_scale, block_n, block_k, fmt=E4M3):
    """bench.py:1460-1470: dequantize both operands with their block scales."""
    a = fp8_decode(a8, fmt)
    b = fp8_decode(b8, fmt)
    m, k = a.shape
    n = b.shape[1]
    kb = np.arange(k) // block_k
    nb = np.arange(n) // block_n
    a_deq = a * _c(a_scale, np.float32)[:, kb]
    b_deq = b * _c(b_scale, np.float32)[kb][:, nb]
    return a_deq.astype(np.float32), b_deq.astype(np.float32)


def fp8_blockwise_ref(a8, b8, a_scale, b_scale, block_n=128, block_k=128, fmt=E4M3):
    """bench.py:1502: a_deq @ b_deq in fp32."""
    a_deq, b_deq = fp8_blockwise_dequant(a8, b8, a_scale, b_scale, block_n, block_k, fmt)
    return (a_deq @ b_deq).astype(np.float32)


def fp8_gemm_scalar(a8, b8, a_scale, b_scale, a_per_token=True, b_per_channel=True,
                    fmt=E4M3) -> np.ndarray:
    """gemm_fp8.cu:98-157 in the reference's operation order (scalar C)."""
    a8 = _c(a8, np.uint8)
    b8 = _c(b8, np.uint8)
    m, k = a8.shape
    n = b8.shape[1]
    out = np.empty((m, n), np.float32)
    lib().oracle_fp8_gemm(_p(a8), _p(b8), _p(_c(a_scale, np.float32)),
                          _p(_c(b_scale, np.float32)), _p(out), m, n, k,
                          int(a_per_token), int(b_per_channel), fmt)
    return out


def fp8_gemm_ref(a8, b8, a_scale, b_scale, a_per_token=True, b_per_channel=True,
                 fmt=E4M3) -> np.ndarray:
    """gemm.h:60-70 closed form C = (a_scale (x) b_scale) * (A_fp8 @ B_fp8):
    decode both operands exactly, fp32 matmul, then scale."""
    a = fp8_decode(a8, fmt).astype(np.float32)
    b = fp8_decode(b8, fmt).astype(np.float32)
    acc = (a @ b).astype(np.float32)
    m, n = acc.shape
    asv = _c(a_scale, np.float32).reshape(-1)
    bsv = _c(b_scale, np.float32).reshape(-1)
    col_a = asv[:m].reshape(m, 1) if a_per_token else asv[0]
    row_b = bsv[:n].reshape(1, n) if b_per_channel else bsv[0]
    return ((acc * col_a).astype(np.float32) * row_b).astype(np.float32)


def w8a8_acc(a_i8, b_i8) -> np.ndarray:
    """Exact int32 accumulators A @ B (bench.py:1228 does it in fp64: every
    |partial sum| < 2^53, so fp64 BLAS is exact)."""
    a = _c(a_i8, np.int8).astype(np.float64)
    b = _c(b_i8, np.int8).astype(np.float64)
    acc = a @ b
    return acc.astype(np.int64).astype(np.int32)


def w8a8_acc_scalar(a_i8, b_i8) -> np.ndarray:
    a = _c(a_i8, np.int8)
    b = _c(b_i8, np.int8)
    m, k = a.shape
    n = b.shape[1]
    out = np.empty((m, n), np.int32)
    lib().oracle_w8a8_acc(_p(a), _p(b), _p(out), m, n, k)
    return out


def w8a8_epilogue(acc, a_scale, b_scale, bias=None, a_per_token=True,
                  b_per_channel=True) -> np.ndarray:
    """gemm_w8a8.cu:134-141: (float(acc) * a_s) * b_s (+ bias), fp32."""
    acc = _c(acc, np.int32)
    m, n = acc.shape
    out = np.empty((m, n), np.float32)
    bb = None if bias is None else _c(bias, np.float32)
    lib().oracle_w8a8_epilogue(_p(acc), _p(_c(a_scale, np.float32)),
                               _p(_c(b_scale, np.float32)), _p(bb), _p(out), m, n,
                               int(a_per_token), int(b_per_channel))
    return out


# ---------------------------------------------------------------------------
# misc
# ---------------------------------------------------------------------------
def xorshift32_uniform(n: int, seed: int, lo: float = -2.0, hi: float = 2.0) -> np.ndarray:
    """The reference tests' deterministic generator (test_common.cuh:205-220),
    computed in fp32 like the C++ it restates."""
    s = seed if seed else 0x9E3779B9
    out = np.empty(n, np.float32)
    lo32, span = np.float32(lo), np.float32(hi) - np.float32(lo)
    for i in range(n):
        s ^= (s << 13) & 0xFFFFFFFF
        s ^= s >> 17
        s ^= (s << 5) & 0xFFFFFFFF
        u = np.float32(s) / np.float32(4294967295.0)
        out[i] = lo32 + u * span
    return out


def rel_err(out, ref) -> float:
    """max |out - ref| / max |ref| (bench.py:847-852), in fp64."""
    o = np.asarray(out, np.float64)
    r = np.asarray(ref, np.float64)
    denom = max(float(np.abs(r).max()) if r.size else 0.0, 1e-6)
    return float(np.abs(o - r).max()) / denom if r.size else 0.0


# ---------------------------------------------------------------------------
# MoE routing helpers (fixture construction for the grouped GEMM)
# ---------------------------------------------------------------------------
def moe_topk_ids(logits, top_k: int) -> np.ndarray:
    """Top-k experts per token (moe_gate.cu:88-105): softmax is monotonic, so
    the selection is the k largest logits, the lowest expert id winning ties."""
    lg = _c(logits, np.float32)
    order = np.argsort(-lg, axis=1, kind="stable")  # stable: lower id first on ties
    return order[:, :top_k].astype(np.int32)


def moe_group_rows(ids, num_experts: int, pad: int = 1):
    """Rows grouped by expert for the grouped GEMM (moe_permute.cu:57-101 with a
    fixed intra-expert order: increasing (token, slot)). Each expert's block is
    padded to a multiple of `pad` rows. Returns (row_src, offsets): row_src[r] is
    the flat (token*top_k + slot) index feeding row r, or -1 for padding;
    offsets is int32 [E+1] over the padded rows."""
    flat = _c(ids, np.int32).reshape(-1)
    rows, offs = [], [0]
    for e in range(num_experts):
        src = np.nonzero(flat == e)[0]
        padded = -(-len(src) // pad) * pad
        rows.append(np.concatenate([src, np.full(padded - len(src), -1)]))
        offs.append(offs[-1] + padded)
    return np.concatenate(rows).astype(np.int64), np.array(offs, np.int32)


def moe_w4a16_ref(a, b_packed, scales, zeros, offsets, group_size, dtype="bf16"):
    """Per expert e: C[off_e:off_{e+1}] = A[off_e:off_{e+1}] @ dequant(B_e)
    (moe_grouped_gemm.cu:99-124 composed with bench.py:1274-1285), fp32."""
    a = _c(a, np.float32)
    E = len(offsets) - 1
    n = b_packed.shape[2]
    out = np.zeros((a.shape[0], n), np.float32)
    for e in range(E):
        r0, r1 = int(offsets[e]), int(offsets[e + 1])
        if r1 > r0:
            w = w4a16_dequant_weight(b_packed[e], scales[e],
                                     None if zeros is None else zeros[e], group_size, dtype)
            out[r0:r1] = a[r0:r1] @ w
    return out


def grouped_gemm_scalar(a, b, offsets, init=None) -> np.ndarray:
    """Dense grouped GEMM in the reference kernel's order (moe_grouped_gemm.cu:
    68-127, scalar C): a ``[rows, k]``, b ``[E, k, n]`` (fp32 values of the
    storage dtype), offsets ``[E+1]``. Rows outside every expert's range keep
    ``init`` (zeros by default). Returns fp32 before the output rounding."""
    a = _c(a, np.float32)
    b = _c(b, np.float32)
    offs = _c(offsets, np.int32)
    rows, k = a.shape
    E, _, n = b.shape
    out = np.zeros((rows, n), np.float32) if init is None else _c(init, np.float32).copy()
    lib().oracle_grouped_gemm(_p(a), _p(b), _p(offs), E, _p(out), rows, n, k)
    return out


def grouped_gemm_ref(a, b, offsets, init=None) -> np.ndarray:
    """The same grouped product as one fp32 matmul per expert (the closed form
    the GEMM tolerance is stated against), for sizes the scalar loop is too
    slow for."""
    a = _c(a, np.float32)
    b = _c(b, np.float32)
    rows = a.shape[0]
    out = np.zeros((rows, b.shape[2]), np.float32) if init is None else _c(init, np.float32).copy()
    for e in range(b.shape[0]):
        r0 = min(max(int(offsets[e]), 0), rows)
        r1 = min(int(offsets[e + 1]), rows)
        if r1 > r0:
            out[r0:r1] = a[r0:r1] @ b[e]
    return out


# ---------------------------------------------------------------------------
# MoE routing (gates, permutation, permute, unpermute)
# ---------------------------------------------------------------------------
_NEG_MAX = np.float32(-3.4028235e38)


def gate_softmax_topk_ref(logits, top_k: int, renormalize: bool = True):
    """moe_gate.cu:42-117: fp32 softmax (max-shifted), then top_k picks by a
    strict '>' scan in increasing expert id (lowest id wins ties); the chosen
    probabilities are divided by their sum (summed in pick order) when
    renormalize is set. Returns (weights fp32 [T, k], indices int32 [T, k])."""
    x = _c(logits, np.float32)
    T, E = x.shape
    w = np.zeros((T, top_k), np.float32)
    idx = np.zeros((T, top_k), np.int32)
    for t in range(T):
        p = np.exp(x[t] - x[t].max()).astype(np.float32)
        s = np.float32(0)
        for v in p:
            s = np.float32(s + v)
        prob = (p * np.float32(np.float32(1) / s)).astype(np.float32)
        order = np.argsort(-prob, kind="stable")[:top_k]
        renorm = np.float32(0)
        for v in prob[order]:
            renorm = np.float32(renorm + v)
        scale = np.float32(1) / renorm if (renormalize and renorm > 0) else np.float32(1)
        w[t] = prob[order] * scale
        idx[t] = order
    return w, idx


def _sigmoid32(x):
    x = np.float32(x)
    if x >= 0:
        return np.float32(np.float32(1) / (np.float32(1) + np.float32(np.exp(-x))))
    z = np.float32(np.exp(x))
    return np.float32(z / (np.float32(1) + z))


def gate_sigmoid_group_topk_ref(logits, bias, n_group: int, topk_group: int, top_k: int,
                                renormalize: bool = True, routed_scaling_factor: float = 1.0):
    """moe_gate.cu:119-236 (DeepSeek-V3 grouped top-k), restated as the
    reference's sequential loops: group score = sum of the group's two best
    biased scores, the topk_group best groups survive (strict '>' in group
    order), top_k experts of the survivors by biased score (strict '>', expert
    order); weights are the unbiased sigmoid scores, renormalized, times the
    routed scaling factor. Missing picks get id 0 and weight 0."""
    x = _c(logits, np.float32)
    T, E = x.shape
    b = None if bias is None else _c(bias, np.float32)
    epg = E // n_group
    w = np.zeros((T, top_k), np.float32)
    idx = np.zeros((T, top_k), np.int32)
    for t in range(T):
        score = np.array([_sigmoid32(v) for v in x[t]], np.float32)
        sel = score.copy() if b is None else (score + b).astype(np.float32)
        gsc = []
        for g in range(n_group):
            m1 = m2 = _NEG_MAX
            for v in sel[g * epg:(g + 1) * epg]:
                if v > m1:
                    m1, m2 = v, m1
                elif v > m2:
                    m2 = v
            gsc.append(np.float32(m1 + m2) if epg >= 2 else m1)
        keep = [False] * n_group
        tmp = list(gsc)
        for _ in range(min(topk_group, n_group)):
            best, bg = _NEG_MAX, -1
            for g in range(n_group):
                if tmp[g] > best:
                    best, bg = tmp[g], g
            if bg < 0:
                break
            keep[bg] = True
            tmp[bg] = _NEG_MAX
        renorm = np.float32(0)
        for k in range(top_k):
            best, be = _NEG_MAX, -1
            for e in range(E):
                if keep[e // epg] and sel[e] > best:
                    best, be = sel[e], e
            if be < 0:
                continue
            w[t, k], idx[t, k] = score[be], be
            renorm = np.float32(renorm + score[be])
            sel[be] = _NEG_MAX
        norm = np.float32(1) / renorm if (renormalize and renorm > 0) else np.float32(1)
        w[t] = (w[t] * norm * np.float32(routed_scaling_factor)).astype(np.float32)
    return w, idx


def compute_permutation_ref(topk_ids, num_experts: int):
    """moe_permute.cu:58-101 as a stable counting sort: pairs (token*top_k+k)
    grouped by expert in increasing pair id; out-of-range ids are dropped.
    Returns (sorted_ids int32 [valid pairs], offsets int32 [E+1])."""
    flat = _c(topk_ids, np.int32).reshape(-1)
    ok = (flat >= 0) & (flat < num_experts)
    pairs = np.nonzero(ok)[0]
    order = pairs[np.argsort(flat[pairs], kind="stable")]
    counts = np.bincount(flat[pairs], minlength=num_experts)
    offs = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    return order.astype(np.int32), offs


def permute_ref(x, sorted_ids, top_k: int):
    """moe_permute.cu:103-129: row r = x[sorted_ids[r] // top_k], zero when the
    id is out of range."""
    x = np.asarray(x)
    rows = len(sorted_ids)
    out = np.zeros((rows, x.shape[1]), x.dtype)
    for r, pr in enumerate(np.asarray(sorted_ids, np.int64)):
        if 0 <= pr < rows:
            out[r] = x[pr // top_k]
    return out


def unpermute_ref(permuted, sorted_ids, weights, num_tokens: int, top_k: int):
    """moe_permute.cu:131-170: out[t] = sum_k w[t,k] * permuted[inv[t*top_k+k]]
    accumulated in fp32 in increasing k with a fused multiply-add (each step
    rounded once, computed exactly in float64 then rounded), absent pairs
    skipped."""
    p = _c(permuted, np.float32)
    rows = len(sorted_ids)
    inv = np.full(rows, -1, np.int64)
    for r, pr in enumerate(np.asarray(sorted_ids, np.int64)):
        if 0 <= pr < rows:
            inv[pr] = r
    wt = _c(weights, np.float32).reshape(-1)
    out = np.zeros((num_tokens, p.shape[1]), np.float32)
    for t in range(num_tokens):
        acc = np.zeros(p.shape[1], np.float32)
        for k in range(top_k):
            r = inv[t * top_k + k]
            if r < 0:
                continue
            acc = (p[r].astype(np.float64) * np.float64(wt[t * top_k + k])
                   + acc.astype(np.float64)).astype(np.float32)
        out[t] = acc
    return out
