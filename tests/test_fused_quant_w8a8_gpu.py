"""GPU parity of ks_gemm_w8a8_fused_quant, the extension that fuses the
dynamic int8 activation quantizer (per-token or per-tensor) into W8A8.

The entry point is defined as ks_quantize_int8 followed by ks_gemm_w8a8, so
the bars are (1) bit-identity with that two-call sequence run on the GPU on the
same inputs (decode shapes M <= 4 run the one-pass kernel, which reduces the
row maxima and quantizes inside the GEMM; larger M stage through library
scratch), and (2) bit-identity with the oracle: codes and scales from
oracle.quant_row / quant_tensor (the restatement of quant_int8.cu:23-83),
exact int32 accumulators and the reference's (acc * a_s) * b_s + bias epilogue
(gemm_w8a8.cu:166-217). Against the two-call sequence outputs are compared as
bits; against the oracle as values, with NaN equal to NaN.
"""
import numpy as np
import pytest
import torch

import kernel_set as ks
import oracle as O
from kernel_set.enums import DType, QuantMode
from tests import helpers as H

pytestmark = pytest.mark.gpu
ADT = {"bf16": DType.BF16, "f16": DType.F16, "f32": DType.F32}
PT_PC = (QuantMode.PER_TOKEN, QuantMode.PER_CHANNEL)
PT_PT = (QuantMode.PER_TENSOR, QuantMode.PER_TENSOR)
PT_PTC = (QuantMode.PER_TENSOR, QuantMode.PER_CHANNEL)
TOK_T = (QuantMode.PER_TOKEN, QuantMode.PER_TENSOR)


def bits(t):
    t = t.contiguous()
    return t.view(torch.int32 if t.element_size() == 4 else torch.int16).cpu().numpy()


def make(m, n, k, modes, adt, out, bias, seed, special=False):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[:, ::29] *= 40.0  # outliers set the row scales
    if m > 2:
        x[m // 2] = 0.0  # all-zero row: the 1e-12 scale floor
    if special:
        x[0, 5] = np.nan
        x[0, 9] = -0.0
        x[0, 17] = 3e-39 if adt == "f32" else 0.0  # fp32 subnormal
        if m > 1:
            x[m - 1, 3] = np.inf
    xt, xv = H.to_dev(x, adt)
    b = rng.integers(-127, 128, (k, n)).astype(np.int8)
    pc = modes[1] == QuantMode.PER_CHANNEL
    b_s = rng.uniform(0.005, 0.02, n if pc else 1).astype(np.float32)
    bias_v = O.round_to(rng.standard_normal(n).astype(np.float32), out) if bias else None
    return xt, xv, b, b_s, bias_v


def check(m, n, k, modes=PT_PC, adt="bf16", out="bf16", bias=False, seed=0, special=False):
    xt, xv, b, b_s, bias_v = make(m, n, k, modes, adt, out, bias, seed, special)
    bt, bst = H.np_i8_dev(b), H.np_f32_dev(b_s)
    biast = H.to_dev(bias_v, out)[0] if bias else None
    odt = H.torch_dtype(out)
    got = torch.empty(m, n, device="cuda", dtype=odt)
    ks.gemm.gemm_w8a8_fused_quant(got, xt, bt, bst, m, n, k, bias=biast, a_mode=modes[0],
                                  b_mode=modes[1], a_dtype=ADT[adt])
    # the two-call sequence the extension is defined as
    pt = modes[0] == QuantMode.PER_TOKEN
    a8 = torch.empty(m, k, device="cuda", dtype=torch.int8)
    a_s = torch.empty(m if pt else 1, device="cuda", dtype=torch.float32)
    ks.quant.quantize_int8(a8, a_s, xt, m, k, mode=modes[0])
    ref2 = torch.empty(m, n, device="cuda", dtype=odt)
    ks.gemm.gemm_w8a8(ref2, a8, bt, a_s, bst, m, n, k, bias=biast, a_mode=modes[0],
                      b_mode=modes[1])
    torch.cuda.synchronize()
    assert np.array_equal(bits(got), bits(ref2)), "fused result differs from quantize + GEMM"
    ea8, eas = O.quant_row(xv, O.INT8) if pt else O.quant_tensor(xv, O.INT8)
    assert np.array_equal(H.u8(a8), ea8)
    assert np.array_equal(a_s.cpu().numpy().view(np.int32), eas.view(np.int32))
    with np.errstate(invalid="ignore", over="ignore"):
        exp = O.w8a8_epilogue(O.w8a8_acc(ea8.view(np.int8), b), eas, b_s, bias_v, pt,
                              modes[1] == QuantMode.PER_CHANNEL)
    assert np.array_equal(H.from_dev_f32(got), O.round_to(exp, out), equal_nan=True)


@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 6, 7, 8])
@pytest.mark.parametrize("n,k", [(256, 512), (528, 1056), (80, 160), (1024, 4096)])
def test_fused_w8a8_decode_bitexact(m, n, k):
    check(m, n, k, seed=m * 13 + n + k)


@pytest.mark.parametrize("modes", [PT_PC, PT_PT, PT_PTC, TOK_T])
@pytest.mark.parametrize("m", [1, 5])
def test_fused_w8a8_modes(modes, m):
    check(m, 384, 1536, modes=modes, bias=True, seed=int(modes[0]) * 7 + int(modes[1]) + m)


@pytest.mark.parametrize("adt", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("out", ["bf16", "f16", "f32"])
def test_fused_w8a8_dtypes(adt, out):
    check(3, 320, 1024, adt=adt, out=out, bias=out != "f32", seed=len(adt) + len(out))


@pytest.mark.parametrize("modes", [PT_PC, PT_PT])
def test_fused_w8a8_special_values(modes):
    # NaN is ignored by the amax; an Inf row gets an Inf scale and NaN outputs
    check(4, 256, 512, modes=modes, special=True, seed=91)
    check(2, 256, 512, modes=modes, adt="f32", out="f32", special=True, seed=92)


@pytest.mark.parametrize("m,modes", [(1, PT_PC), (4, PT_PT), (8, PT_PC), (8, PT_PT)])
def test_fused_w8a8_decode_shape(m, modes):
    check(m, 7168, 7168, modes=modes, seed=m + 7168)


@pytest.mark.parametrize("m,k,modes", [(4, 16384, PT_PC), (3, 12288, PT_PT), (1, 40960, PT_PC)])
def test_fused_w8a8_long_rows(m, k, modes):
    # M*K/8 > 4096 pieces: the one-pass row-max prologue runs several batches
    # of 8 loads per thread, the last one ragged (3 x 12288 / 8 = 4608)
    check(m, 256, k, modes=modes, seed=m + k)


@pytest.mark.parametrize("m,n,k,modes", [(9, 512, 1024, PT_PC), (64, 4096, 2048, PT_PC),
                                         (300, 768, 1280, PT_PT), (33, 48, 96, PT_PTC)])
def test_fused_w8a8_staged_bitexact(m, n, k, modes):
    check(m, n, k, modes=modes, bias=True, seed=m + n)


def test_fused_w8a8_unaligned_k_stages():
    # K % 32 != 0 is outside the one-pass kernel: staged through scratch
    check(4, 128, 200, seed=200)


def test_fused_w8a8_repeated_calls_and_growth():
    # the scale stash of the one-pass path and the staged codes share library
    # staging; it grows between calls and every result still matches
    for m, n, k in ((2, 512, 1024), (64, 512, 1024), (8, 512, 2048), (300, 512, 2048),
                    (1, 512, 4096)):
        check(m, n, k, seed=m * 5 + k)
