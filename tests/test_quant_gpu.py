"""GPU parity: quantizers and int4 weight helpers, bit-exact against the oracle
(codes and fp32 scales compared byte for byte), through the C ABI."""
import os

import numpy as np
import pytest
import torch

import kernel_set as ks
import oracle as O
from kernel_set.enums import DType, QuantMode
from tests import helpers as H

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
KS_DT = {"f32": DType.F32, "f16": DType.F16, "bf16": DType.BF16}
FP8 = {O.E4M3: (DType.F8E4M3, torch.float8_e4m3fn), O.E5M2: (DType.F8E5M2, torch.float8_e5m2)}


def _inputs(rows, cols, dt, seed, outliers=0.001):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((rows, cols)).astype(np.float32)
    if outliers:
        idx = rng.choice(x.size, max(1, int(x.size * outliers)), replace=False)
        x.flat[idx] *= 50.0
    t, xv = H.to_dev(x, dt)
    return t, xv


def _group(t, rows, cols, gs, fmt, dt):
    fdt, tdt = FP8[fmt]
    out = torch.empty(rows, cols, device=t.device, dtype=tdt)
    sc = torch.empty(rows, (cols + gs - 1) // gs, device=t.device, dtype=torch.float32)
    ks.quant.quantize_fp8_group(out, sc, t, rows, cols, group_size=gs, fp8_dtype=fdt)
    torch.cuda.synchronize()
    return H.u8(out), sc.cpu().numpy()


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("fmt", [O.E4M3, O.E5M2])
@pytest.mark.parametrize("rows,cols,gs", [(7, 512, 128), (5, 300, 128), (3, 136, 64),
                                          (4, 100, 100), (2, 130, 7), (9, 1024, 512),
                                          (1, 72, 1024), (6, 256, 16)])
def test_quantize_fp8_group_bitexact(dt, fmt, rows, cols, gs):
    t, xv = _inputs(rows, cols, dt, seed=rows * 1000 + cols + gs)
    q, s = _group(t, rows, cols, gs, fmt, dt)
    eq, es = O.quant_group(xv, gs, fmt)
    assert np.array_equal(s.view(np.uint32), es.view(np.uint32))
    assert np.array_equal(q, eq)


@pytest.mark.parametrize("rows,cols,gs", [(1531, 7168, 128), (777, 4104, 64)])
def test_quantize_fp8_group_persistent_grid_bitexact(rows, cols, gs):
    # More than 2048 workgroups of slots: the persistent kernel, including a
    # trip count that does not divide the grid and a ragged last group.
    t, xv = _inputs(rows, cols, "bf16", seed=rows + cols)
    q, s = _group(t, rows, cols, gs, O.E4M3, "bf16")
    eq, es = O.quant_group(xv, gs, O.E4M3)
    assert np.array_equal(s.view(np.uint32), es.view(np.uint32))
    assert np.array_equal(q, eq)


def test_quantize_fp8_group_golden():
    f = np.load(os.path.join(GOLDEN, "quant_fp8_group.npz"))
    t, _ = H.to_dev(f["x_bf16_vals"], "bf16")
    for name, fmt in (("e4m3", O.E4M3), ("e5m2", O.E5M2)):
        q, s = _group(t, 8, 300, 128, fmt, "bf16")
        assert np.array_equal(q, f[f"{name}_q"]) and np.array_equal(s, f[f"{name}_s"])


def test_quantize_fp8_group_config3_full_size():
    # BASELINE config 3 activations: 2048 x 7168 bf16 ~N(0,1), 0.1% outliers x50.
    rows, cols = 2048, 7168
    t, xv = _inputs(rows, cols, "bf16", seed=33)
    q, s = _group(t, rows, cols, 128, O.E4M3, "bf16")
    eq, es = O.quant_group(xv, 128, O.E4M3)
    assert np.array_equal(s, es) and np.array_equal(q, eq)
    # dispatch entry point returns the same bytes
    q2, s2 = ks.dispatch.per_token_group_quant(t, group_size=128)
    assert q2.dtype == torch.float8_e4m3fn and s2.shape == (rows, 56)
    assert np.array_equal(H.u8(q2), eq) and np.array_equal(s2.cpu().numpy(), es)


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("fmt", [O.E4M3, O.E5M2])
@pytest.mark.parametrize("rows,cols", [(4, 4096), (3, 7168), (2, 130), (2, 20480), (1, 8)])
def test_quantize_fp8_per_token_bitexact(dt, fmt, rows, cols):
    t, xv = _inputs(rows, cols, dt, seed=cols + rows)
    fdt, tdt = FP8[fmt]
    out = torch.empty(rows, cols, device=t.device, dtype=tdt)
    sc = torch.empty(rows, device=t.device, dtype=torch.float32)
    ks.quant.quantize_fp8(out, sc, t, rows, cols, fp8_dtype=fdt, mode=QuantMode.PER_TOKEN)
    torch.cuda.synchronize()
    eq, es = O.quant_row(xv, fmt)
    assert np.array_equal(sc.cpu().numpy(), es) and np.array_equal(H.u8(out), eq)


@pytest.mark.parametrize("dt", ["bf16", "f32"])
@pytest.mark.parametrize("fmt", [O.E4M3, O.E5M2])
def test_quantize_fp8_per_tensor_bitexact(dt, fmt):
    rows, cols = 33, 1000
    t, xv = _inputs(rows, cols, dt, seed=77)
    fdt, tdt = FP8[fmt]
    out = torch.empty(rows, cols, device=t.device, dtype=tdt)
    sc = torch.full((1,), 123.0, device=t.device, dtype=torch.float32)
    for _ in range(2):  # second call must not see the first call's state
        ks.quant.quantize_fp8(out, sc, t, rows, cols, fp8_dtype=fdt, mode=QuantMode.PER_TENSOR)
    torch.cuda.synchronize()
    eq, es = O.quant_tensor(xv, fmt)
    assert np.array_equal(sc.cpu().numpy(), es) and np.array_equal(H.u8(out), eq)


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("mode", [QuantMode.PER_TOKEN, QuantMode.PER_TENSOR])
def test_quantize_int8_reference_case_golden(dt, mode):
    # kernels/tests/test_quant.cu:34-139 inputs; expectation frozen in the fixture.
    f = np.load(os.path.join(GOLDEN, "quant_int8_refcase.npz"))
    xs = O.round_to(f["x_f32"], dt)
    t, _ = H.to_dev(xs, dt)
    out = torch.empty(6, 130, device=t.device, dtype=torch.int8)
    sc = torch.empty(6 if mode == QuantMode.PER_TOKEN else 1, device=t.device, dtype=torch.float32)
    ks.quant.quantize_int8(out, sc, t, 6, 130, mode=mode)
    torch.cuda.synchronize()
    tag = "tok" if mode == QuantMode.PER_TOKEN else "ten"
    assert np.array_equal(H.u8(out), f[f"{dt}_{tag}_q"])
    assert np.array_equal(sc.cpu().numpy(), f[f"{dt}_{tag}_s"])
    # round trip through the dequant partner (reference test's third check)
    deq = torch.empty(6, 130, device=t.device, dtype=H.torch_dtype(dt))
    ks.quant.dequantize_int8(deq, out, sc, 6, 130, mode=mode)
    torch.cuda.synchronize()
    exp = O.round_to(O.dequant(f[f"{dt}_{tag}_q"], f[f"{dt}_{tag}_s"], O.INT8,
                               mode == QuantMode.PER_TOKEN), dt)
    assert np.array_equal(H.from_dev_f32(deq), exp)


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("rows,cols", [(4096, 4096), (3, 130), (2, 20000), (5, 24)])
def test_quantize_int8_per_token_bitexact(dt, rows, cols):
    if rows * cols > 4096 * 4096 // 2 and dt != "bf16":
        pytest.skip("full-size case runs for bf16 only")
    t, xv = _inputs(rows, cols, dt, seed=rows + cols)
    out = torch.empty(rows, cols, device=t.device, dtype=torch.int8)
    sc = torch.empty(rows, device=t.device, dtype=torch.float32)
    ks.quant.quantize_int8(out, sc, t, rows, cols)
    torch.cuda.synchronize()
    eq, es = O.quant_row(xv, O.INT8)
    assert np.array_equal(sc.cpu().numpy(), es) and np.array_equal(H.u8(out), eq)


def test_zero_rows_and_ties():
    x = np.zeros((3, 256), np.float32)
    x[1, :8] = [127, 0.5, 1.5, 2.5, -0.5, -1.5, -127, 126.5]
    t, xv = H.to_dev(x, "f32")
    out = torch.empty(3, 256, device=t.device, dtype=torch.int8)
    sc = torch.empty(3, device=t.device, dtype=torch.float32)
    ks.quant.quantize_int8(out, sc, t, 3, 256)
    torch.cuda.synchronize()
    q = out.cpu().numpy()
    assert sc[0].item() == np.float32(1e-12) and np.all(q[0] == 0)
    assert q[1, :8].tolist() == [127, 0, 2, 2, 0, -2, -127, 126]


@pytest.mark.parametrize("fmt", [O.E4M3, O.E5M2])
def test_dequantize_fp8(fmt):
    rows, cols = 17, 333
    rng = np.random.default_rng(5)
    codes = rng.integers(0, 256, (rows, cols), dtype=np.uint8)
    codes[(codes & 0x7F) == 0x7F] = 0  # avoid NaN codes
    if fmt == O.E5M2:
        codes[(codes & 0x7C) == 0x7C] = 1
    sc = rng.uniform(0.01, 2, rows).astype(np.float32)
    fdt, tdt = FP8[fmt]
    t = H.np_u8_dev(codes).view(tdt)
    out = torch.empty(rows, cols, device=t.device, dtype=torch.float32)
    ks.quant.dequantize_fp8(out, t, H.np_f32_dev(sc), rows, cols, fp8_dtype=fdt,
                            mode=QuantMode.PER_TOKEN)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), O.dequant(codes, sc, fmt, True))


@pytest.mark.parametrize("k,n", [(4096, 4096), (64, 24), (128, 1000)])
def test_repack_int4(k, n):
    rng = np.random.default_rng(k + n)
    codes = rng.integers(0, 16, (k, n), dtype=np.uint8)
    words = O.pack_k8_int32(codes)
    out = torch.empty(k // 2, n, device="cuda", dtype=torch.uint8)
    ks.quant.repack_int4(out, H.np_i32_dev(words), None, k, n)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), O.pack_k2_uint8(codes))
    perm = rng.permutation(k).astype(np.int32)
    ks.quant.repack_int4(out, H.np_i32_dev(words), H.np_i32_dev(perm), k, n)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), O.repack_int4(words, perm))


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
def test_dequantize_int4(dt):
    k, n, gs = 256, 96, 64
    rng = np.random.default_rng(3)
    codes = rng.integers(0, 16, (k, n), dtype=np.uint8)
    s = O.round_to(rng.uniform(0.002, 0.02, (k // gs, n)).astype(np.float32), dt)
    z = O.round_to(rng.integers(6, 10, (k // gs, n)).astype(np.float32), dt)
    st, _ = H.to_dev(s, dt)
    zt, _ = H.to_dev(z, dt)
    out = torch.empty(k, n, device="cuda", dtype=H.torch_dtype(dt))
    ks.quant.dequantize_int4(out, H.np_i32_dev(O.pack_k8_int32(codes)), st, zt, k, n, gs)
    torch.cuda.synchronize()
    exp = O.round_to(O.dequant_int4(O.pack_k8_int32(codes), s, z, gs), dt)
    assert np.array_equal(H.from_dev_f32(out), exp)


def _special_rows(cols):
    """Rows with +-Inf, the largest finite floats, subnormals, exact rounding
    ties and zeros (NaN is left out: the reference's `a > b ? a : b` amax
    keeps or drops a NaN depending on its lane, so its result is not defined;
    this build ignores NaN in amax, as the oracle does)."""
    rng = np.random.default_rng(5)
    x = rng.standard_normal((6, cols)).astype(np.float32)
    x[0, 130] = np.inf
    x[1, 3] = -np.inf
    x[2, 0:4] = [3.0e38, -3.0e38, 1e-40, -1e-40]
    x[3, :] = rng.uniform(-1, 1, cols).astype(np.float32) * np.float32(1e-39)
    x[4, :8] = [448.0, -448.0, 464.0, 480.0, 0.5 * 2 ** -9, 1.5 * 2 ** -9, 57344.0, 61440.0]
    x[5, :] = 0.0
    return x


@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("fmt", [O.E4M3, O.E5M2])
@pytest.mark.parametrize("gs", [128, 64])
def test_quantize_fp8_group_special_values(dt, fmt, gs):
    cols = 512
    t, xv = H.to_dev(_special_rows(cols), dt)
    got_q, got_s = _group(t, 6, cols, gs, fmt, dt)
    eq, es = O.quant_group(xv, gs, fmt)
    assert np.array_equal(got_s.view(np.uint32), es.view(np.uint32))
    assert np.array_equal(got_q, eq)


@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("fmt", [O.E4M3, O.E5M2])
@pytest.mark.parametrize("mode", [QuantMode.PER_TOKEN, QuantMode.PER_TENSOR])
def test_quantize_fp8_rowwise_special_values(dt, fmt, mode):
    cols = 512
    x = _special_rows(cols)
    if mode == QuantMode.PER_TENSOR:
        x = x[2:]  # one infinity would make every code of the tensor NaN or 0
    rows = x.shape[0]
    t, xv = H.to_dev(x, dt)
    fdt, tdt = FP8[fmt]
    out = torch.empty(rows, cols, device=t.device, dtype=tdt)
    sc = torch.empty(rows if mode == QuantMode.PER_TOKEN else 1, device=t.device, dtype=torch.float32)
    ks.quant.quantize_fp8(out, sc, t, rows, cols, fp8_dtype=fdt, mode=mode)
    torch.cuda.synchronize()
    eq, es = (O.quant_row(xv, fmt) if mode == QuantMode.PER_TOKEN else O.quant_tensor(xv, fmt))
    assert np.array_equal(sc.cpu().numpy().view(np.uint32), np.asarray(es, np.float32).view(np.uint32))
    assert np.array_equal(H.u8(out), eq)


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_quantize_int8_special_values(dt):
    cols = 512
    x = _special_rows(cols)[2:]  # finite rows (int8 of an infinite scale is undefined)
    t, xv = H.to_dev(x, dt)
    out = torch.empty(4, cols, device=t.device, dtype=torch.int8)
    sc = torch.empty(4, device=t.device, dtype=torch.float32)
    ks.quant.quantize_int8(out, sc, t, 4, cols)
    torch.cuda.synchronize()
    eq, es = O.quant_row(xv, O.INT8)
    assert np.array_equal(sc.cpu().numpy().view(np.uint32), es.view(np.uint32))
    assert np.array_equal(H.u8(out), eq)
