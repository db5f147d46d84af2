"""GPU parity of ks_gemm_fp8_blockwise_fused_quant, the extension that fuses
the 1 x block_k activation quantizer into the fp8 blockwise GEMM.

The entry point is defined as ks_quantize_fp8_group followed by
ks_gemm_fp8_blockwise, so the bar is bit-identity with that two-call sequence
run on the GPU on the same inputs (decode shapes M <= 8 run the one-pass
kernel, which quantizes inside the GEMM; larger M stage through library
scratch). Against the oracle: the quantized codes and scales the two-call path
produces are bit-exact to oracle.quant_group, and the output is within the
GEMM's 1e-2 max-rel tolerance of the closed form on those codes.
"""
import numpy as np
import pytest
import torch

import kernel_set as ks
import oracle as O
from kernel_set.enums import DType
from tests import helpers as H
from tests.test_gemm8_gpu import TOL, block_quant_weight

pytestmark = pytest.mark.gpu
FP8 = {O.E4M3: (DType.F8E4M3, torch.float8_e4m3fn), O.E5M2: (DType.F8E5M2, torch.float8_e5m2)}
ADT = {"bf16": DType.BF16, "f16": DType.F16, "f32": DType.F32}


def case(m, n, k, bn, bk, adt, fmt, seed, outliers=False):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((m, k)).astype(np.float32)
    if outliers:
        x[:, ::37] *= 80.0
    if m > 1:
        x[m // 2, : min(k, 3 * bk)] = 0.0  # all-zero groups: the 1e-12 scale floor
    xt, xv = H.to_dev(x, adt)
    w = (rng.standard_normal((k, n)) * 0.02).astype(np.float32)
    b8, b_s = block_quant_weight(w, bk, bn, fmt)
    return xt, xv, b8, b_s


def two_call(xt, b8t, bst, m, n, k, bn, bk, adt, fmt, out):
    fdt, tdt = FP8[fmt]
    ng = -(-k // bk)
    a8 = torch.empty(m, k, device="cuda", dtype=tdt)
    a_s = torch.empty(m, ng, device="cuda", dtype=torch.float32)
    ks.quant.quantize_fp8_group(a8, a_s, xt, m, k, group_size=bk, fp8_dtype=fdt)
    o = torch.empty(m, n, device="cuda", dtype=H.torch_dtype(out))
    ks.gemm.gemm_fp8_blockwise(o, a8, b8t, a_s, bst, m, n, k, block_n=bn, block_k=bk,
                               fp8_dtype=fdt)
    torch.cuda.synchronize()
    return o, a8, a_s


def fused(xt, b8t, bst, m, n, k, bn, bk, adt, fmt, out):
    fdt, _ = FP8[fmt]
    o = torch.empty(m, n, device="cuda", dtype=H.torch_dtype(out))
    ks.gemm.gemm_fp8_blockwise_fused_quant(o, xt, b8t, bst, m, n, k, block_n=bn, block_k=bk,
                                           a_dtype=ADT[adt], fp8_dtype=fdt)
    torch.cuda.synchronize()
    return o


def check(m, n, k, bn=128, bk=128, adt="bf16", fmt=O.E4M3, out="bf16", seed=0, outliers=False):
    xt, xv, b8, b_s = case(m, n, k, bn, bk, adt, fmt, seed, outliers)
    b8t = H.np_u8_dev(b8).view(FP8[fmt][1])
    bst = H.np_f32_dev(b_s)
    got = fused(xt, b8t, bst, m, n, k, bn, bk, adt, fmt, out)
    ref2, a8, a_s = two_call(xt, b8t, bst, m, n, k, bn, bk, adt, fmt, out)
    assert torch.equal(got, ref2), "fused result differs from quantize + GEMM"
    ea8, eas = O.quant_group(xv, bk, fmt)
    assert np.array_equal(H.u8(a8), ea8) and np.array_equal(a_s.cpu().numpy(), eas)
    ref = O.fp8_blockwise_ref(ea8, b8, eas, b_s, bn, bk, fmt)
    assert O.rel_err(H.from_dev_f32(got), ref) <= (TOL if fmt == O.E4M3 else 2e-2)


@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 6, 7, 8])
@pytest.mark.parametrize("n,k", [(256, 512), (528, 1056), (80, 160), (1024, 4096)])
def test_fused_decode_bitexact(m, n, k):
    check(m, n, k, seed=m * 11 + n + k)


@pytest.mark.parametrize("adt", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("out", ["bf16", "f32"])
def test_fused_dtypes(adt, out):
    check(3, 384, 1536, adt=adt, out=out, seed=5, outliers=True)


@pytest.mark.parametrize("bn,bk", [(128, 32), (64, 64), (16, 256), (128, 384), (96, 128)])
def test_fused_blocks(bn, bk):
    # block_k 384 is outside the one-pass set and stages through scratch
    check(6, 768, 2304, bn=bn, bk=bk, seed=bn + bk)


def test_fused_e5m2():
    check(4, 512, 1024, fmt=O.E5M2, seed=52, outliers=True)


@pytest.mark.parametrize("m", [1, 4])
def test_fused_decode_shape(m):
    check(m, 7168, 7168, seed=m + 7168)


@pytest.mark.parametrize("m,n,k", [(9, 512, 1024), (64, 7168, 2048), (300, 768, 1280)])
def test_fused_staged_bitexact(m, n, k):
    check(m, n, k, seed=m + n)


def test_fused_repeated_calls_and_growth():
    # staging grows between calls (M = 64 then M = 300) and the one-pass path
    # runs in between; every result still equals the two-call sequence
    for m, n, k in ((64, 512, 1024), (2, 512, 1024), (300, 512, 2048), (8, 512, 2048)):
        check(m, n, k, seed=m * 3)
