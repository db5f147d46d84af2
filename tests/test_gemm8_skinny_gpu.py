"""GPU parity of the decode-shape (M <= 8) path of the three 8-bit GEMMs
(ks_gemm_fp8_blockwise, ks_gemm_fp8, ks_gemm_w8a8): B streamed once, K split
over workgroups, split partials summed in order by a second kernel. M = 9..16
in the same parametrizations runs the split-K 256x256 kernel (or the tiled
kernel where N is not a multiple of 256) on the same data, to the same bars.

Same bars as the tiled kernels:
  * fp8 blockwise / plain fp8: max |out - ref| / max |ref| <= 1e-2 against the
    closed-form oracle; exact for integer-valued operands with unit scales;
  * W8A8: int32 accumulators and outputs bit-exact (int32 split partials add
    exactly, so the split does not change results).
Shapes cover both fragment counts (M = 1..8 in 4-row fragments), N not a
multiple of the 256-column tile, K with a partial last scale block and with
chunks past K, and block_k down to one 32-row chunk.
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

MS = [1, 2, 3, 4, 5, 7, 8, 9, 12, 13, 16]


@pytest.mark.parametrize("m", MS)
@pytest.mark.parametrize("n,k", [(256, 512), (528, 1056), (80, 160)])
def test_skinny_fp8_blockwise(m, n, k):
    a8, b8, a_s, b_s = fp8_case(m, n, k, seed=m * 7 + n + k)
    got = run_fp8(a8, b8, a_s, b_s, 128, 128)
    assert O.rel_err(got, O.fp8_blockwise_ref(a8, b8, a_s, b_s, 128, 128)) <= TOL


@pytest.mark.parametrize("bn,bk", [(64, 256), (16, 32), (128, 64), (48, 96)])
def test_skinny_fp8_blockwise_blocks(bn, bk):
    a8, b8, a_s, b_s = fp8_case(6, 384, 1344, bn=bn, bk=bk, seed=bn * bk)
    got = run_fp8(a8, b8, a_s, b_s, bn, bk, out="f32")
    assert O.rel_err(got, O.fp8_blockwise_ref(a8, b8, a_s, b_s, bn, bk)) <= TOL


@pytest.mark.parametrize("m", [1, 4, 16])
def test_skinny_fp8_blockwise_decode_shape(m):
    # DeepSeek-V3-style decode projection: N = K = 7168, 1x128 / 128x128 blocks
    a8, b8, a_s, b_s = fp8_case(m, 7168, 7168, seed=m)
    got = run_fp8(a8, b8, a_s, b_s, 128, 128)
    assert O.rel_err(got, O.fp8_blockwise_ref(a8, b8, a_s, b_s, 128, 128)) <= TOL


def test_skinny_fp8_blockwise_e5m2():
    a8, b8, a_s, b_s = fp8_case(5, 512, 1024, fmt=O.E5M2, seed=55)
    got = run_fp8(a8, b8, a_s, b_s, 128, 128, fmt=O.E5M2)
    assert O.rel_err(got, O.fp8_blockwise_ref(a8, b8, a_s, b_s, 128, 128, O.E5M2)) <= 2e-2


@pytest.mark.parametrize("m", [1, 6, 16])
def test_skinny_fp8_blockwise_integer_exact(m):
    rng = np.random.default_rng(m)
    n, k = 272, 2048
    ai = rng.integers(-8, 9, (m, k)).astype(np.float32)
    bi = rng.integers(-8, 9, (k, n)).astype(np.float32)
    a_s = np.ones((m, k // 128), np.float32)
    b_s = np.ones((k // 128, -(-n // 128)), np.float32)
    got = run_fp8(O.fp8_encode(ai), O.fp8_encode(bi), a_s, b_s, 128, 128, out="f32")
    assert np.array_equal(got, (ai.astype(np.int64) @ bi.astype(np.int64)).astype(np.float32))


@pytest.mark.parametrize("m", MS)
@pytest.mark.parametrize("n,k", [(256, 512), (528, 1056)])
def test_skinny_fp8_plain(m, n, k):
    a8, b8, a_s, b_s = fp8_plain_case(m, n, k, seed=m + n + k)
    got = run_fp8_plain(a8, b8, a_s, b_s)
    assert O.rel_err(got, O.fp8_gemm_ref(a8, b8, a_s, b_s)) <= TOL


@pytest.mark.parametrize("per_tok,per_ch", [(False, False), (True, False), (False, True)])
def test_skinny_fp8_plain_scale_modes(per_tok, per_ch):
    a8, b8, a_s, b_s = fp8_plain_case(11, 320, 768, seed=per_tok * 2 + per_ch)
    a_s = a_s if per_tok else a_s[:1].copy()
    b_s = b_s if per_ch else b_s[:1].copy()
    got = run_fp8_plain(a8, b8, a_s, b_s, per_tok, per_ch, out="f32")
    assert O.rel_err(got, O.fp8_gemm_ref(a8, b8, a_s, b_s, per_tok, per_ch)) <= TOL


def test_skinny_fp8_plain_integer_exact():
    rng = np.random.default_rng(17)
    m, n, k = 9, 96, 4096
    ai = rng.integers(-8, 9, (m, k)).astype(np.float32)
    bi = rng.integers(-8, 9, (k, n)).astype(np.float32)
    one = np.ones(1, np.float32)
    got = run_fp8_plain(O.fp8_encode(ai), O.fp8_encode(bi), one, one, False, False, out="f32")
    assert np.array_equal(got, (ai.astype(np.int64) @ bi.astype(np.int64)).astype(np.float32))


@pytest.mark.parametrize("m", MS)
@pytest.mark.parametrize("n,k", [(256, 512), (528, 1056), (4096, 4096)])
def test_skinny_w8a8_int32_accumulators_bitexact(m, n, k):
    rng = np.random.default_rng(m * 31 + n + k)
    a = rng.integers(-127, 128, (m, k)).astype(np.int8)
    b = rng.integers(-127, 128, (k, n)).astype(np.int8)
    a[0, :] = 127
    b[:, 0] = 127  # largest accumulators the ABI admits
    if m > 1:
        a[-1, :] = -127
    assert np.array_equal(w8a8_acc_dev(a, b), O.w8a8_acc(a, b))


@pytest.mark.parametrize("out", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("modes", [(QuantMode.PER_TOKEN, QuantMode.PER_CHANNEL),
                                   (QuantMode.PER_TENSOR, QuantMode.PER_TENSOR)])
@pytest.mark.parametrize("m,bias", [(1, False), (7, True), (16, True)])
def test_skinny_w8a8_outputs_bitexact(out, modes, m, bias):
    n, k = 784, 1536
    rng = np.random.default_rng(m + modes[0] * 3 + modes[1])
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


def test_skinny_matches_split_boundary():
    # M = 8 (skinny) and M = 9 (split-K 256x256 kernel) on the same data: the
    # W8A8 accumulators agree exactly; the fp8 outputs differ only by fp32
    # association (32-row chunk promotion and split sums against 128-row block
    # promotion; ~1.4e-5 of max |out| measured for K = 2048).
    rng = np.random.default_rng(89)
    n, k = 512, 2048
    a = rng.integers(-127, 128, (9, k)).astype(np.int8)
    b = rng.integers(-127, 128, (k, n)).astype(np.int8)
    assert np.array_equal(w8a8_acc_dev(a[:8], b), w8a8_acc_dev(a, b)[:8])
    a8, b8, a_s, b_s = fp8_case(9, n, k, seed=9)
    g9 = run_fp8(a8, b8, a_s, b_s, 128, 128, out="f32")
    g8 = run_fp8(a8[:8].copy(), b8, a_s[:8].copy(), b_s, 128, 128, out="f32")
    assert O.rel_err(g8, g9[:8]) <= 1e-4
