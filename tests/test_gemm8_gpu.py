"""GPU parity: fp8 blockwise GEMM, plain scaled fp8 GEMM and W8A8 int8 GEMM
against the oracle.

fp8 (ks_gemm_fp8): max |out - ref| / max |ref| <= 1e-2 against the closed form
(a_s (x) b_s) * (A @ B) with exactly decoded operands; exact for integer-valued
operands with unit scales; the any-shape fallback is bit-exact against the
scalar oracle (same k order, same (acc * a_s) * b_s epilogue).

fp8 blockwise: max |out - ref| / max |ref| <= 1e-2 against the fp32
dequantize-then-matmul reference (north_star; bench.py:1434-1502 restated);
exact for integer-valued operands with unit scales; the any-shape fallback is
additionally bit-exact against the scalar two-level oracle.
W8A8: int32 accumulators bit-exact (test hook ks_testing_gemm_w8a8_i32), and
outputs bit-exact against the oracle epilogue (float(acc)*a_s)*b_s (+bias).
"""
import ctypes
import os

import numpy as np
import pytest
import torch

import kernel_set as ks
import oracle as O
from kernel_set import _lib
from kernel_set.enums import DType, QuantMode
from tests import helpers as H

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
TOL = 1e-2
FP8 = {O.E4M3: (DType.F8E4M3, torch.float8_e4m3fn), O.E5M2: (DType.F8E5M2, torch.float8_e5m2)}


def block_quant_weight(w, bk, bn, fmt=O.E4M3):
    """bench.py:1434-1461 recipe: per (bk x bn) block scale = max(amax/qmax, 1e-12)."""
    k, n = w.shape
    nkb, nnb = -(-k // bk), -(-n // bn)
    qmax = np.float32(O.QMAX[fmt])
    bs = np.empty((nkb, nnb), np.float32)
    b8 = np.empty((k, n), np.uint8)
    for i in range(nkb):
        for j in range(nnb):
            blk = w[i * bk:(i + 1) * bk, j * bn:(j + 1) * bn]
            sc = np.maximum(np.float32(np.abs(blk).max()) / qmax, np.float32(1e-12))
            bs[i, j] = sc
            b8[i * bk:(i + 1) * bk, j * bn:(j + 1) * bn] = O.fp8_encode(blk * (np.float32(1) / sc), fmt)
    return b8, bs


def run_fp8(a8, b8, a_s, b_s, bn, bk, fmt=O.E4M3, out="bf16"):
    m, k = a8.shape
    n = b8.shape[1]
    fdt, tdt = FP8[fmt]
    o = torch.empty(m, n, device="cuda", dtype=H.torch_dtype(out))
    ks.gemm.gemm_fp8_blockwise(o, H.np_u8_dev(a8).view(tdt), H.np_u8_dev(b8).view(tdt),
                               H.np_f32_dev(a_s), H.np_f32_dev(b_s), m, n, k, block_n=bn,
                               block_k=bk, fp8_dtype=fdt)
    torch.cuda.synchronize()
    return H.from_dev_f32(o)


def fp8_case(m, n, k, bn=128, bk=128, fmt=O.E4M3, seed=0, outliers=0.0):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((m, k)).astype(np.float32)
    if outliers:
        idx = rng.choice(x.size, max(1, int(x.size * outliers)), replace=False)
        x.flat[idx] *= 50.0
    a8, a_s = O.quant_group(O.round_bf16(x), bk, fmt)
    w = (rng.standard_normal((k, n)) * 0.02).astype(np.float32)
    b8, b_s = block_quant_weight(w, bk, bn, fmt)
    return a8, b8, a_s, b_s


@pytest.mark.parametrize("m,n,k", [(128, 128, 128), (256, 384, 512), (130, 208, 384),
                                   (1, 64, 256), (77, 1040, 1056), (512, 512, 7168)])
@pytest.mark.parametrize("out", ["bf16", "f32"])
def test_fp8_blockwise_tiled(m, n, k, out):
    a8, b8, a_s, b_s = fp8_case(m, n, k, seed=m + n + k)
    got = run_fp8(a8, b8, a_s, b_s, 128, 128, out=out)
    ref = O.fp8_blockwise_ref(a8, b8, a_s, b_s, 128, 128)
    assert O.rel_err(got, ref) <= TOL


@pytest.mark.parametrize("bn,bk", [(64, 256), (128, 384), (32, 128)])
def test_fp8_blockwise_other_blocks(bn, bk):
    a8, b8, a_s, b_s = fp8_case(96, 256, 768, bn=bn, bk=bk, seed=bn + bk)
    got = run_fp8(a8, b8, a_s, b_s, bn, bk)
    assert O.rel_err(got, O.fp8_blockwise_ref(a8, b8, a_s, b_s, bn, bk)) <= TOL


def test_fp8_blockwise_e5m2():
    a8, b8, a_s, b_s = fp8_case(128, 256, 512, fmt=O.E5M2, seed=5)
    got = run_fp8(a8, b8, a_s, b_s, 128, 128, fmt=O.E5M2)
    assert O.rel_err(got, O.fp8_blockwise_ref(a8, b8, a_s, b_s, 128, 128, O.E5M2)) <= 2e-2


def test_fp8_blockwise_integer_exact():
    rng = np.random.default_rng(3)
    m, n, k = 160, 192, 640
    ai = rng.integers(-8, 9, (m, k)).astype(np.float32)
    bi = rng.integers(-8, 9, (k, n)).astype(np.float32)
    a_s = np.ones((m, k // 128), np.float32)
    b_s = np.ones((k // 128, n // 128 + 1), np.float32)
    got = run_fp8(O.fp8_encode(ai), O.fp8_encode(bi), a_s, b_s, 128, 128, out="f32")
    assert np.array_equal(got, (ai.astype(np.int64) @ bi.astype(np.int64)).astype(np.float32))


def run_fp8_plain(a8, b8, a_s, b_s, per_tok=True, per_ch=True, fmt=O.E4M3, out="bf16"):
    m, k = a8.shape
    n = b8.shape[1]
    fdt, tdt = FP8[fmt]
    o = torch.empty(m, n, device="cuda", dtype=H.torch_dtype(out))
    ks.gemm.gemm_fp8(o, H.np_u8_dev(a8).view(tdt), H.np_u8_dev(b8).view(tdt),
                     H.np_f32_dev(a_s), H.np_f32_dev(b_s), m, n, k,
                     a_mode=QuantMode.PER_TOKEN if per_tok else QuantMode.PER_TENSOR,
                     b_mode=QuantMode.PER_CHANNEL if per_ch else QuantMode.PER_TENSOR,
                     fp8_dtype=fdt)
    torch.cuda.synchronize()
    return H.from_dev_f32(o)


def fp8_plain_case(m, n, k, fmt=O.E4M3, seed=0):
    """Per-token activations and per-channel weights, both quantized the
    reference way (amax / qmax per row / per output column)."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((m, k)).astype(np.float32)
    a8, a_s = O.quant_row(O.round_bf16(x), fmt)
    w = (rng.standard_normal((k, n)) * 0.02).astype(np.float32)
    wt8, b_s = O.quant_row(w.T.copy(), fmt)
    return a8, np.ascontiguousarray(wt8.T), a_s, b_s


@pytest.mark.parametrize("m,n,k", [(256, 256, 128), (512, 768, 1024), (130, 208, 384),
                                   (1, 64, 256), (77, 1040, 1056), (2048, 512, 7168)])
@pytest.mark.parametrize("out", ["bf16", "f32"])
def test_fp8_plain_shapes(m, n, k, out):
    a8, b8, a_s, b_s = fp8_plain_case(m, n, k, seed=m + 3 * n + k)
    got = run_fp8_plain(a8, b8, a_s, b_s, out=out)
    assert O.rel_err(got, O.fp8_gemm_ref(a8, b8, a_s, b_s)) <= TOL


@pytest.mark.parametrize("per_tok,per_ch", [(False, False), (True, False), (False, True)])
def test_fp8_plain_scale_modes(per_tok, per_ch):
    a8, b8, a_s, b_s = fp8_plain_case(256, 512, 512, seed=9)
    sa = a_s if per_tok else a_s[:1].copy()
    sb = b_s if per_ch else b_s[:1].copy()
    got = run_fp8_plain(a8, b8, sa, sb, per_tok, per_ch)
    assert O.rel_err(got, O.fp8_gemm_ref(a8, b8, sa, sb, per_tok, per_ch)) <= TOL


def test_fp8_plain_e5m2():
    a8, b8, a_s, b_s = fp8_plain_case(256, 256, 512, fmt=O.E5M2, seed=4)
    got = run_fp8_plain(a8, b8, a_s, b_s, fmt=O.E5M2)
    assert O.rel_err(got, O.fp8_gemm_ref(a8, b8, a_s, b_s, fmt=O.E5M2)) <= 2e-2


def test_fp8_plain_integer_exact():
    rng = np.random.default_rng(31)
    for m, n, k in ((256, 256, 640), (160, 192, 640), (33, 40, 70)):  # fast, tiled, scalar
        ai = rng.integers(-8, 9, (m, k)).astype(np.float32)
        bi = rng.integers(-8, 9, (k, n)).astype(np.float32)
        got = run_fp8_plain(O.fp8_encode(ai), O.fp8_encode(bi), np.ones(m, np.float32),
                            np.ones(n, np.float32), out="f32")
        assert np.array_equal(got, (ai.astype(np.int64) @ bi.astype(np.int64)).astype(np.float32))


def test_fp8_plain_fallback_bitexact():
    # K not a multiple of 16 -> the per-element kernel, which keeps the
    # reference's k order and epilogue: bit-exact against the scalar oracle.
    a8, b8, a_s, b_s = fp8_plain_case(19, 23, 45, seed=6)
    got = run_fp8_plain(a8, b8, a_s, b_s, out="f32")
    assert np.array_equal(got, O.fp8_gemm_scalar(a8, b8, a_s, b_s))


def test_fp8_gemm_dispatch_nt_layout():
    # ks.dispatch.fp8_gemm takes the weight as [N, K] (the reference's NT
    # provider layout) and a_scale/b_scale as torch._scaled_mm-style vectors.
    a8, b8, a_s, b_s = fp8_plain_case(128, 256, 384, seed=8)
    tdt = torch.float8_e4m3fn
    out = ks.dispatch.fp8_gemm(H.np_u8_dev(a8).view(tdt),
                               H.np_u8_dev(np.ascontiguousarray(b8.T)).view(tdt),
                               H.np_f32_dev(a_s.reshape(-1, 1)), H.np_f32_dev(b_s.reshape(1, -1)))
    torch.cuda.synchronize()
    assert out.dtype == torch.bfloat16 and tuple(out.shape) == (128, 256)
    assert O.rel_err(H.from_dev_f32(out), O.fp8_gemm_ref(a8, b8, a_s, b_s)) <= TOL


def test_fp8_blockwise_fallback_golden_bitexact():
    # block 64x64 is not a multiple of the 128-deep MFMA step -> scalar path,
    # which follows the reference order and must match the scalar oracle.
    f = np.load(os.path.join(GOLDEN, "fp8_blockwise_small.npz"))
    got = run_fp8(f["a8"], f["b8"], f["a_scale"], f["b_scale"], int(f["bn"]), int(f["bk"]), out="f32")
    assert np.array_equal(got, f["c_f32"])


def test_fp8_config3_end_to_end():
    # x bf16 [2048, 7168] ~N(0,1) with 0.1% outliers x50 ->
    # ks per_token_group_quant (1x128) -> fp8 blockwise GEMM with W [7168,7168]
    # ~N(0,0.02) block-quantized 128x128 on the host -> bf16 out.
    m = n = k = 7168
    m = 2048
    rng = np.random.default_rng(2048)
    x = rng.standard_normal((m, k)).astype(np.float32)
    idx = rng.choice(x.size, int(x.size * 0.001), replace=False)
    x.flat[idx] *= 50.0
    xt, xv = H.to_dev(x, "bf16")
    a8, a_s = ks.dispatch.per_token_group_quant(xt, group_size=128)
    w = (rng.standard_normal((k, n)) * 0.02).astype(np.float32)
    b8, b_s = block_quant_weight(w, 128, 128)
    out = ks.dispatch.fp8_gemm_blockwise(a8, H.np_u8_dev(b8).view(torch.float8_e4m3fn), a_s,
                                         H.np_f32_dev(b_s))
    torch.cuda.synchronize()
    ea8, eas = O.quant_group(xv, 128, O.E4M3)
    assert np.array_equal(H.u8(a8), ea8)
    ref = O.fp8_blockwise_ref(ea8, b8, eas, b_s, 128, 128)
    assert out.dtype == torch.bfloat16 and O.rel_err(H.from_dev_f32(out), ref) <= TOL


# ---------------------------------------------------------------------- W8A8
def w8a8_acc_dev(a, b):
    m, k = a.shape
    n = b.shape[1]
    acc = torch.empty(m, n, device="cuda", dtype=torch.int32)
    at, bt = H.np_i8_dev(a), H.np_i8_dev(b)  # keep both alive until the kernel ran
    ks.check(_lib.lib.ks_testing_gemm_w8a8_i32(
        ctypes.cast(acc.data_ptr(), _lib._I32P), at.data_ptr(), bt.data_ptr(), m, n, k,
        torch.cuda.current_stream().cuda_stream), "ks_testing_gemm_w8a8_i32")
    torch.cuda.synchronize()
    return acc.cpu().numpy()


@pytest.mark.parametrize("m,n,k", [(128, 128, 128), (33, 48, 112), (300, 272, 1008),
                                   (1, 16, 16), (257, 129, 77), (4096, 4096, 4096)])
def test_w8a8_int32_accumulators_bitexact(m, n, k):
    rng = np.random.default_rng(m * n + k)
    a = rng.integers(-127, 128, (m, k)).astype(np.int8)
    b = rng.integers(-127, 128, (k, n)).astype(np.int8)
    a[0, :] = 127
    b[:, 0] = 127  # the largest accumulators the ABI admits
    assert np.array_equal(w8a8_acc_dev(a, b), O.w8a8_acc(a, b))


@pytest.mark.parametrize("out", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("modes", [(QuantMode.PER_TOKEN, QuantMode.PER_CHANNEL),
                                   (QuantMode.PER_TENSOR, QuantMode.PER_TENSOR),
                                   (QuantMode.PER_TOKEN, QuantMode.PER_TENSOR)])
@pytest.mark.parametrize("m,n,k,bias", [(192, 256, 384, False), (33, 47, 100, True),
                                        (96, 128, 256, True)])
def test_w8a8_outputs_bitexact(out, modes, m, n, k, bias):
    rng = np.random.default_rng(m + n + k + modes[0] * 3 + modes[1])
    a = rng.integers(-127, 128, (m, k)).astype(np.int8)
    b = rng.integers(-127, 128, (k, n)).astype(np.int8)
    pt, pc = modes[0] == QuantMode.PER_TOKEN, modes[1] == QuantMode.PER_CHANNEL
    a_s = rng.uniform(0.01, 0.03, m if pt else 1).astype(np.float32)
    b_s = rng.uniform(0.01, 0.03, n if pc else 1).astype(np.float32)
    bias_v = O.round_to(rng.standard_normal(n).astype(np.float32), out) if bias else None
    c = torch.empty(m, n, device="cuda", dtype=H.torch_dtype(out))
    bt = H.to_dev(bias_v, out)[0] if bias else None
    ks.gemm.gemm_w8a8(c, H.np_i8_dev(a), H.np_i8_dev(b), H.np_f32_dev(a_s), H.np_f32_dev(b_s),
                      m, n, k, bias=bt, a_mode=modes[0], b_mode=modes[1])
    torch.cuda.synchronize()
    exp = O.round_to(O.w8a8_epilogue(O.w8a8_acc(a, b), a_s, b_s, bias_v, pt, pc), out)
    assert np.array_equal(H.from_dev_f32(c), exp)


def test_w8a8_golden():
    f = np.load(os.path.join(GOLDEN, "w8a8_small.npz"))
    assert np.array_equal(w8a8_acc_dev(f["a"], f["b"]), f["acc"])
    m, k = f["a"].shape
    n = f["b"].shape[1]
    c = torch.empty(m, n, device="cuda", dtype=torch.float32)
    ks.gemm.gemm_w8a8(c, H.np_i8_dev(f["a"]), H.np_i8_dev(f["b"]), H.np_f32_dev(f["a_scale"]),
                      H.np_f32_dev(f["b_scale"]), m, n, k)
    torch.cuda.synchronize()
    assert np.array_equal(c.cpu().numpy(), f["c_f32"])


def test_w8a8_config4_end_to_end():
    # A bf16 ~N(0,1) per-token int8 via ks_quantize_int8 on
    # the GPU; W ~N(0,0.02) per-output-channel int8 (per-token quant of W^T on
    # the host); bf16 out through ks.dispatch.int8_gemm.
    m = n = k = 4096
    rng = np.random.default_rng(4096)
    x = rng.standard_normal((m, k)).astype(np.float32)
    w = (rng.standard_normal((k, n)) * 0.02).astype(np.float32)
    xt, xv = H.to_dev(x, "bf16")
    a8 = torch.empty(m, k, device="cuda", dtype=torch.int8)
    a_s = torch.empty(m, device="cuda", dtype=torch.float32)
    ks.quant.quantize_int8(a8, a_s, xt, m, k)
    wq_t, b_s = O.quant_row(np.ascontiguousarray(w.T), O.INT8)
    b8 = np.ascontiguousarray(wq_t.view(np.int8).T)
    out = ks.dispatch.int8_gemm(a8, H.np_i8_dev(b8), a_s, H.np_f32_dev(b_s))
    torch.cuda.synchronize()
    ea8, eas = O.quant_row(xv, O.INT8)
    assert np.array_equal(H.u8(a8), ea8) and np.array_equal(a_s.cpu().numpy(), eas)
    exp = O.round_bf16(O.w8a8_epilogue(O.w8a8_acc(ea8.view(np.int8), b8), eas, b_s))
    assert np.array_equal(H.from_dev_f32(out), exp)
    # and the quantized GEMM tracks the full-precision product
    ref = xv @ w
    assert O.rel_err(H.from_dev_f32(out), ref) < 3e-2
