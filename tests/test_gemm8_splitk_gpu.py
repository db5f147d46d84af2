"""GPU parity of the split-K form of the fast 8-bit GEMM kernel, taken when
the output has fewer tiles than the chip has CUs (e.g. 9 <= M <= 512 at
N = 7168). The row tile follows M: 64 rows for M <= 64, 128 rows for
M <= 384, 256 rows above (all 256 columns wide). Every split writes its raw
accumulators to a partial plane and a second kernel sums them in split order,
then applies the epilogue.

Bars as for the unsplit kernel: fp8 blockwise / plain fp8 max-rel <= 1e-2
against the closed-form oracle and exact on integer-valued operands with unit
scales; W8A8 int32 accumulators and outputs bit-exact.
"""
import numpy as np
import pytest
import torch

import kernel_set as ks
import oracle as O
from kernel_set.enums import QuantMode
from tests import helpers as H
from tests.test_gemm8_gpu import (TOL, fp8_case, fp8_plain_case, run_fp8, run_fp8_plain,
                                  w8a8_acc_dev)

pytestmark = pytest.mark.gpu

SHAPES = [(17, 512, 2048), (100, 1024, 1536), (256, 2048, 4096), (300, 768, 1280),
          (64, 256, 384), (9, 768, 1024), (33, 512, 2560), (65, 512, 1024), (128, 768, 2048)]


@pytest.mark.parametrize("m,n,k", SHAPES)
def test_splitk_fp8_blockwise(m, n, k):
    a8, b8, a_s, b_s = fp8_case(m, n, k, seed=m + n + k)
    got = run_fp8(a8, b8, a_s, b_s, 128, 128)
    assert O.rel_err(got, O.fp8_blockwise_ref(a8, b8, a_s, b_s, 128, 128)) <= TOL


def test_splitk_fp8_blockwise_config3_width():
    a8, b8, a_s, b_s = fp8_case(64, 7168, 7168, seed=647)
    got = run_fp8(a8, b8, a_s, b_s, 128, 128)
    assert O.rel_err(got, O.fp8_blockwise_ref(a8, b8, a_s, b_s, 128, 128)) <= TOL


def test_splitk_fp8_blockwise_integer_exact():
    rng = np.random.default_rng(99)
    m, n, k = 40, 512, 3072
    ai = rng.integers(-8, 9, (m, k)).astype(np.float32)
    bi = rng.integers(-8, 9, (k, n)).astype(np.float32)
    a_s = np.ones((m, k // 128), np.float32)
    b_s = np.ones((k // 128, n // 128), np.float32)
    got = run_fp8(O.fp8_encode(ai), O.fp8_encode(bi), a_s, b_s, 128, 128, out="f32")
    assert np.array_equal(got, (ai.astype(np.int64) @ bi.astype(np.int64)).astype(np.float32))


@pytest.mark.parametrize("m,n,k", SHAPES)
def test_splitk_fp8_plain(m, n, k):
    a8, b8, a_s, b_s = fp8_plain_case(m, n, k, seed=m * n + k)
    got = run_fp8_plain(a8, b8, a_s, b_s, out="f32")
    assert O.rel_err(got, O.fp8_gemm_ref(a8, b8, a_s, b_s)) <= TOL


@pytest.mark.parametrize("m,n,k", SHAPES + [(200, 1024, 4096)])
def test_splitk_w8a8_int32_accumulators_bitexact(m, n, k):
    rng = np.random.default_rng(m * 7 + n + k)
    a = rng.integers(-127, 128, (m, k)).astype(np.int8)
    b = rng.integers(-127, 128, (k, n)).astype(np.int8)
    a[0, :] = 127
    b[:, 0] = 127
    assert np.array_equal(w8a8_acc_dev(a, b), O.w8a8_acc(a, b))


@pytest.mark.parametrize("out", ["bf16", "f32"])
@pytest.mark.parametrize("bias", [False, True])
def test_splitk_w8a8_outputs_bitexact(out, bias):
    m, n, k = 96, 512, 2048
    rng = np.random.default_rng(7 + bias)
    a = rng.integers(-127, 128, (m, k)).astype(np.int8)
    b = rng.integers(-127, 128, (k, n)).astype(np.int8)
    a_s = rng.uniform(0.01, 0.03, m).astype(np.float32)
    b_s = rng.uniform(0.01, 0.03, n).astype(np.float32)
    bias_v = O.round_to(rng.standard_normal(n).astype(np.float32), out) if bias else None
    c = torch.empty(m, n, device="cuda", dtype=H.torch_dtype(out))
    bt = H.to_dev(bias_v, out)[0] if bias else None
    ks.gemm.gemm_w8a8(c, H.np_i8_dev(a), H.np_i8_dev(b), H.np_f32_dev(a_s), H.np_f32_dev(b_s),
                      m, n, k, bias=bt, a_mode=QuantMode.PER_TOKEN, b_mode=QuantMode.PER_CHANNEL)
    torch.cuda.synchronize()
    exp = O.round_to(O.w8a8_epilogue(O.w8a8_acc(a, b), a_s, b_s, bias_v, True, True), out)
    assert np.array_equal(H.from_dev_f32(c), exp)


@pytest.mark.parametrize("m", [24, 64])
def test_fast_64_row_tiles_unsplit(m):
    # M <= 64 runs 64-row tiles; with N / 256 = 130 tiles no K split is taken
    n, k = 33280, 256
    a8, b8, a_s, b_s = fp8_case(m, n, k, seed=m + n)
    got = run_fp8(a8, b8, a_s, b_s, 128, 128)
    assert O.rel_err(got, O.fp8_blockwise_ref(a8, b8, a_s, b_s, 128, 128)) <= TOL
    rng = np.random.default_rng(m)
    a = rng.integers(-127, 128, (m, k)).astype(np.int8)
    b = rng.integers(-127, 128, (k, n)).astype(np.int8)
    assert np.array_equal(w8a8_acc_dev(a, b), O.w8a8_acc(a, b))
