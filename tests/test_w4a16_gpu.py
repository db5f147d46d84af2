"""GPU parity: ks_gemm_w4a16 against the oracle.

Tolerance (north_star): max |out - ref| / max |ref| <= 1e-2 against the fp32
dequant-then-matmul reference (bench.py:1274-1285 restated in oracle.w4a16_ref);
the integer special case (z = 8, s = 1, small integer activations) must be exact.
"""
import os

import numpy as np
import pytest
import torch

import kernel_set as ks
import oracle as O
from kernel_set.enums import DType
from tests import helpers as H

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
TOL = 1e-2


def run_w4a16(a, b_packed, scales, zeros, gs, dt="bf16", bias=None):
    m, k = a.shape
    n = b_packed.shape[1]
    at, av = H.to_dev(a, dt)
    st, sv = H.to_dev(scales, dt)
    zt, zv = (None, None) if zeros is None else H.to_dev(zeros, dt)
    bt, bv = (None, None) if bias is None else H.to_dev(bias, dt)
    c = torch.empty(m, n, device="cuda", dtype=H.torch_dtype(dt))
    ks.gemm.gemm_w4a16(c, at, H.np_u8_dev(b_packed), st, zt, m, n, k, gs, bias=bt)
    torch.cuda.synchronize()
    return H.from_dev_f32(c), (av, sv, zv, bv)


def check(m, k, n, gs, zero_mode="int69", dt="bf16", seed=0, bias=False):
    a, codes, s, z = H.w4a16_inputs(m, k, n, gs, zero_mode, seed)
    b = O.pack_k2_uint8(codes)
    bias_v = np.random.default_rng(seed + 1).standard_normal(n).astype(np.float32) if bias else None
    out, (av, sv, zv, bv) = run_w4a16(a, b, s, z, gs, dt, bias_v)
    ref = O.w4a16_ref(av, b, sv, zv, gs, dt, bias=bv)
    err = O.rel_err(out, ref)
    assert err <= TOL, (m, k, n, gs, err)
    return out, ref


@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 8, 12, 13, 16])
@pytest.mark.parametrize("k,n,gs", [(256, 128, 128), (512, 384, 64), (1024, 272, 32),
                                    (4096, 4096, 128), (2048, 1040, 256),
                                    # K/2 not a multiple of a workgroup's rows, N not of 256
                                    (320, 528, 64), (160, 96, 32)])
def test_gemv_shapes(m, k, n, gs):
    check(m, k, n, gs, seed=m * 7 + k + n)


@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_dtypes_bias_and_null_zeros(dt):
    check(2, 512, 256, 128, dt=dt, bias=True, seed=3)
    check(1, 512, 256, 128, zero_mode=None, dt=dt, seed=4)


@pytest.mark.parametrize("m,k,n,gs", [(3, 100, 30, 50), (2, 96, 50, 6), (1, 64, 7, -1),
                                      (4, 258, 16, 2)])
def test_odd_shapes_fallback(m, k, n, gs):
    eff = gs if gs > 0 else k
    a, codes, s, z = H.w4a16_inputs(m, k, n, eff, "int69", seed=m + k)
    b = O.pack_k2_uint8(codes)
    out, (av, sv, zv, _) = run_w4a16(a, b, s, z, gs)
    ref = O.w4a16_ref(av, b, sv, zv, eff, "bf16")
    assert O.rel_err(out, ref) <= TOL


def test_integer_special_case_exact():
    rng = np.random.default_rng(11)
    m, k, n, gs = 4, 128, 512, 32
    a = rng.integers(-1, 2, (m, k)).astype(np.float32)
    codes = rng.integers(0, 16, (k, n), dtype=np.uint8)
    s = np.ones((k // gs, n), np.float32)
    z = np.full((k // gs, n), 8.0, np.float32)
    out, _ = run_w4a16(a, O.pack_k2_uint8(codes), s, z, gs)
    exact = (a.astype(np.int64) @ (codes.astype(np.int64) - 8)).astype(np.float32)
    assert np.abs(exact).max() < 256  # every value exactly representable in bf16
    assert np.array_equal(out, exact)


def test_golden_fixture():
    f = np.load(os.path.join(GOLDEN, "w4a16_small.npz"))
    out, _ = run_w4a16(f["a"], f["b_packed"], f["scales"], f["zeros"], int(f["gs"]),
                       bias=f["bias"])
    assert O.rel_err(out, O.round_bf16(f["c_f32"])) <= 5e-3


def test_config1_headline_gemv():
    # M=1, K=N=4096, g=128, zeros fixed 8, weights delivered
    # as int32 [K/8, N] and repacked on the device (ks_repack_int4).
    m, k, n, gs = 1, 4096, 4096, 128
    a, codes, s, z = H.w4a16_inputs(m, k, n, gs, "fixed8", seed=2024)
    words = O.pack_k8_int32(codes)
    b = torch.empty(k // 2, n, device="cuda", dtype=torch.uint8)
    ks.quant.repack_int4(b, H.np_i32_dev(words), None, k, n)
    at, av = H.to_dev(a, "bf16")
    st, sv = H.to_dev(s, "bf16")
    zt, zv = H.to_dev(z, "bf16")
    c = ks.dispatch.w4a16(at, b, st, zt, group_size=gs)
    torch.cuda.synchronize()
    ref = O.w4a16_ref(av, O.pack_k2_uint8(codes), sv, zv, gs, "bf16")
    assert c.shape == (1, n) and c.dtype == torch.bfloat16
    assert O.rel_err(H.from_dev_f32(c), ref) <= TOL
    # deterministic: a second call gives identical bits
    c2 = ks.dispatch.w4a16(at, b, st, zt, group_size=gs)
    torch.cuda.synchronize()
    assert torch.equal(c, c2)


@pytest.mark.parametrize("m", [1, 16, 64, 256])
def test_config2_sweep(m):
    # K=4096, N=14336, zeros integer-valued U{6..9}.
    check(m, 4096, 14336, 128, zero_mode="int69", seed=100 + m)


@pytest.mark.parametrize("m", [9, 16, 33, 48, 64, 100, 257])
@pytest.mark.parametrize("k,n,gs", [(1024, 384, 64), (2048, 272, 128), (4096, 512, 256),
                                    (1536, 256, 512), (960, 256, 64), (1024, 200, 32),
                                    (1024, 448, 128)])
def test_batched_shapes(m, k, n, gs):
    # M > 8 runs on MFMA: for M > 64 with N % 64 == 0 the dequantize-to-LDS
    # GEMM (64- or 128-column tiles), otherwise the LDS-ring tile when
    # K % 128 == 0, gs % 64 == 0 and N % 16 == 0 (with N tails, gs = 64
    # half-stage groups and K splits on group boundaries), else the register tile.
    check(m, k, n, gs, seed=m * 3 + k + n + gs)


@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_batched_dtypes_bias_and_null_zeros(dt):
    check(24, 1024, 256, 128, dt=dt, bias=True, seed=5)
    check(40, 1024, 256, 64, zero_mode=None, dt=dt, seed=6)
    check(70, 2048, 384, 128, zero_mode=None, dt=dt, bias=True, seed=7)


@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_dq_split_k(dt):
    # M > 64 on few column tiles: the dequantize-to-LDS GEMM splits K over
    # whole groups and the split reduce adds the bias.
    check(200, 4096, 512, 128, dt=dt, bias=True, seed=11)
    check(65, 8192, 256, 64, zero_mode=None, dt=dt, seed=12)
    check(130, 4096, 1024, 256, dt=dt, bias=True, seed=13)


@pytest.mark.parametrize("m,k,n,gs,zero_mode,dt,bias", [
    (129, 1024, 12288, 128, "int69", "bf16", False),
    (200, 2048, 12288, 64, None, "f16", True),
    (256, 1024, 12288, 256, "int69", "bf16", True),
    (300, 512, 16384, 128, "int69", "f16", False),
    # 96..191 tiles: the role-split kernel splits K (3 uneven splits here)
    (100, 1024, 12288, 128, "int69", "bf16", True),
    (70, 2048, 14336, 64, None, "f16", False),
    (65, 1024, 4096, 128, "int69", "bf16", True),   # 32 tiles
    (200, 2048, 4096, 64, None, "f16", False),      # 64 tiles
    # M >= 384 with >= 192 tiles of 256 x 128: the 256-row role-split tile
    (400, 512, 24576, 128, "int69", "bf16", True),
    (512, 512, 12288, 64, None, "f16", False),
])
def test_dq_role_split_tiles(m, k, n, gs, zero_mode, dt, bias):
    # M > 64 with >= 32 tiles of 128 x 128 (K split below 192 workgroups), or
    # M >= 384 with >= 192 tiles of 256 x 128: the role-split kernel (producer waves copy and dequantize, consumer waves run
    # the MFMAs); M not a multiple of 128 leaves a ragged last row tile.
    check(m, k, n, gs, zero_mode=zero_mode, dt=dt, seed=m + gs, bias=bias)


def test_batched_deterministic():
    a, codes, s, z = H.w4a16_inputs(64, 4096, 1024, 128, "int69", seed=8)
    b = O.pack_k2_uint8(codes)
    o1, _ = run_w4a16(a, b, s, z, 128)
    o2, _ = run_w4a16(a, b, s, z, 128)
    assert np.array_equal(o1, o2)


@pytest.mark.parametrize("m,n", [(16, 1024), (40, 1040), (64, 2048)])
def test_ring_split_reduce_output_alignment(m, n):
    """The ring tile's split reduce stores 4 outputs at a time when C is 8-byte
    aligned and falls back to one output per thread otherwise; both sum the
    splits in the same order, so C must be bit-identical, and within the
    tolerance of the oracle (N = 1024: tiles % 8 == 0, XCD-mapped reduce;
    N = 1040: 65 tiles, linear mapping)."""
    k, gs = 4096, 128
    a, codes, s, z = H.w4a16_inputs(m, k, n, gs, "int69", seed=m + n)
    b = O.pack_k2_uint8(codes)
    at, av = H.to_dev(a, "bf16")
    st, sv = H.to_dev(s, "bf16")
    zt, zv = H.to_dev(z, "bf16")
    bt = H.np_u8_dev(b)
    c0 = torch.empty(m, n, device="cuda", dtype=torch.bfloat16)
    ks.gemm.gemm_w4a16(c0, at, bt, st, zt, m, n, k, gs)
    flat = torch.empty(m * n + 1, device="cuda", dtype=torch.bfloat16)
    c1 = flat[1:].view(m, n)  # 2-byte aligned only
    ks.gemm.gemm_w4a16(c1, at, bt, st, zt, m, n, k, gs)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(c0.view(torch.int16).cpu().numpy(), c1.view(torch.int16).cpu().numpy())
    ref = O.w4a16_ref(av, b, sv, zv, gs, "bf16")
    assert O.rel_err(H.from_dev_f32(c0), ref) <= TOL


def test_dq_256_row_tile_matches_128_row_tile():
    # N = 14336, M = 512 runs the 256 x 128 role-split tile and M = 256 the
    # 128 x 128 one, neither with a K split. Both accumulate each output over
    # the same 64-k stages and 16-k MFMA slices in the same order, so the
    # first 256 rows must agree bit for bit; the rows of the second tile are
    # checked against the oracle on a sample.
    m, k, n, gs = 512, 4096, 14336, 128
    a, codes, s, z = H.w4a16_inputs(m, k, n, gs, "int69", seed=512)
    b = O.pack_k2_uint8(codes)
    out, (av, sv, zv, _) = run_w4a16(a, b, s, z, gs)
    out256, _ = run_w4a16(a[:256], b, s, z, gs)
    assert np.array_equal(out[:256], out256)
    rows = np.array([0, 255, 256, 300, 383, 384, 511])
    ref = O.w4a16_ref(av[rows], b, sv, zv, gs, "bf16")
    assert O.rel_err(out[rows], ref) <= TOL
