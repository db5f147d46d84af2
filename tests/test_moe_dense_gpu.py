"""GPU parity: dense grouped GEMM ks_moe_grouped_gemm (moe_grouped_gemm.cu:136-198)
against the oracle, through the C ABI.

* Integer-valued operands make every fp32 partial sum exact in any order, so
  the HIP result must equal the scalar oracle (the reference kernel's order)
  bit for bit after the same output rounding, for all five dtypes, on the MFMA
  tile path (1-, 2- and 4-block pass heights) and on the any-shape path.
* Rows outside every expert's range keep what the caller put there.
* bf16 / f16 N(0,1) operands at the BASELINE config 5 shapes (64 experts, top-8
  of 256 tokens; gate_up K=2048 N=1536, down K=768 N=2048) are within max rel
  err 1e-2 of one fp32 matmul per expert; f32 within 1e-5.
"""
import numpy as np
import pytest
import torch

import kernel_set as ks
import oracle as O
from kernel_set.enums import DType
from tests import helpers as H

pytestmark = pytest.mark.gpu

DTYPES = ["bf16", "f16", "f32", "e4m3", "e5m2"]
FMT = {"e4m3": O.E4M3, "e5m2": O.E5M2}
TORCH8 = {"e4m3": torch.float8_e4m3fn, "e5m2": torch.float8_e5m2}


def to_dev(x, dt):
    """fp32 numpy -> device tensor of dtype dt, plus the fp32 values it holds."""
    if dt in FMT:
        codes = O.fp8_encode(x, FMT[dt])
        return H.np_u8_dev(codes).view(TORCH8[dt]), O.fp8_decode(codes, FMT[dt]).astype(np.float32)
    return H.to_dev(x, dt)


def round_out(x, dt):
    """Oracle fp32 -> the bits the kernel stores, as comparable numpy arrays."""
    if dt in FMT:
        return O.fp8_encode(x, FMT[dt])
    if dt == "bf16":
        return O.f32_to_bf16_bits(x)
    if dt == "f16":
        return np.ascontiguousarray(x, np.float32).astype(np.float16).view(np.uint16)
    return np.ascontiguousarray(x, np.float32).view(np.uint32)


def bits(t, dt):
    if dt in FMT:
        return H.u8(t)
    if dt == "f32":
        return t.detach().cpu().numpy().view(np.uint32)
    return t.detach().cpu().view(torch.int16).numpy().view(np.uint16)


def run(a_t, b_t, offs, n, k, c_init=None):
    rows = a_t.shape[0]
    E = len(offs) - 1
    c = torch.empty(rows, n, device=a_t.device, dtype=a_t.dtype) if c_init is None else c_init
    ks.moe.grouped_gemm(c, a_t, b_t, H.np_i32_dev(offs), E, rows, n, k)
    torch.cuda.synchronize()
    return c


def sentinel(rows, n, dt):
    """A device C prefilled with a recognisable value (-7)."""
    t, _ = to_dev(np.full((rows, n), -7.0, np.float32), dt)
    return t


def offsets(counts, head=0):
    return np.concatenate([[head], head + np.cumsum(counts)]).astype(np.int32)


@pytest.mark.parametrize("dt", DTYPES)
@pytest.mark.parametrize("counts", [[5, 0, 16, 3, 11, 9],          # avg <= 16: 16-row passes
                                    [30, 0, 31, 17, 64, 2],        # avg <= 32: 32-row passes
                                    [70, 0, 129, 33, 1, 100]])     # 64-row passes, multi-pass
def test_integer_case_bit_exact(dt, counts):
    rng = np.random.default_rng(sum(counts))
    E, K, N = len(counts), 512, 384
    head, tail = 3, 5  # unrouted rows before the first and after the last expert
    offs = offsets(counts, head)
    rows = int(offs[-1]) + tail
    a = rng.integers(-3, 4, (rows, K)).astype(np.float32)
    b = rng.integers(-3, 4, (E, K, N)).astype(np.float32)
    print(f"dense grouped gemm {dt} counts={counts}", flush=True)
    a_t, a_v = to_dev(a, dt)
    b_t, b_v = to_dev(b, dt)
    c = run(a_t, b_t, offs, N, K, sentinel(rows, N, dt))
    init = np.full((rows, N), -7.0, np.float32)
    ref = O.grouped_gemm_scalar(a_v, b_v.reshape(E, K, N), offs, init)
    np.testing.assert_array_equal(bits(c, dt), round_out(ref, dt))


@pytest.mark.parametrize("dt", ["bf16", "e4m3", "f32"])
@pytest.mark.parametrize("K,N", [(100, 30),    # any-shape kernel (K and N off the tile grid)
                                 (256, 136),   # tile kernel, last column tile 8 wide
                                 (128, 20)])   # any-shape (bf16/f32: N*es not a 16 B multiple)
def test_odd_shapes_bit_exact(dt, K, N):
    rng = np.random.default_rng(K * N)
    counts = [7, 0, 21, 2]
    offs = offsets(counts, 1)
    rows = int(offs[-1]) + 2
    E = len(counts)
    a = rng.integers(-3, 4, (rows, K)).astype(np.float32)
    b = rng.integers(-3, 4, (E, K, N)).astype(np.float32)
    print(f"dense grouped gemm {dt} K={K} N={N}", flush=True)
    a_t, a_v = to_dev(a, dt)
    b_t, b_v = to_dev(b, dt)
    c = run(a_t, b_t, offs, N, K, sentinel(rows, N, dt))
    ref = O.grouped_gemm_scalar(a_v, b_v.reshape(E, K, N), offs, np.full((rows, N), -7.0, np.float32))
    np.testing.assert_array_equal(bits(c, dt), round_out(ref, dt))


def config5_rows(seed):
    """Rows grouped by expert from top-8 of router logits ~N(0,1), 256 tokens,
    64 experts (BASELINE config 5 routing), padded to 16 per expert."""
    rng = np.random.default_rng(seed)
    ids = O.moe_topk_ids(rng.standard_normal((256, 64)).astype(np.float32), 8)
    src, offs = O.moe_group_rows(ids, 64, 16)
    return src, offs


@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("K,N", [(2048, 1536), (768, 2048)])
def test_config5_shapes_within_tolerance(dt, K, N):
    src, offs = config5_rows(K)
    rows, E = len(src), 64
    rng = np.random.default_rng(N)
    a = rng.standard_normal((rows, K), dtype=np.float32)
    a[src < 0] = 0.0
    b = (rng.standard_normal((E, K, N), dtype=np.float32) * 0.02).astype(np.float32)
    print(f"dense grouped gemm config5 {dt} K={K} N={N}", flush=True)
    a_t, a_v = to_dev(a, dt)
    b_t, b_v = to_dev(b, dt)
    got = H.from_dev_f32(run(a_t, b_t, offs, N, K))
    ref = O.grouped_gemm_ref(a_v, b_v.reshape(E, K, N), offs)
    assert O.rel_err(got, ref) <= 1e-2


def test_f32_random_tight():
    rng = np.random.default_rng(5)
    counts = [40, 3, 0, 77]
    offs = offsets(counts)
    rows, E, K, N = int(offs[-1]), len(counts), 256, 256
    a = rng.standard_normal((rows, K), dtype=np.float32)
    b = rng.standard_normal((E, K, N), dtype=np.float32)
    got = H.from_dev_f32(run(*[to_dev(x, "f32")[0] for x in (a, b)], offs, N, K))
    assert O.rel_err(got, O.grouped_gemm_ref(a, b, offs)) <= 1e-5


def test_dispatch_moe_dense_form():
    """ks.dispatch.moe without scales takes the reference's dense grouped form
    (_registry.py:1040-1046) and returns C of a's dtype."""
    rng = np.random.default_rng(9)
    counts = [20, 0, 44]
    offs = offsets(counts)
    rows, E, K, N = int(offs[-1]), len(counts), 256, 128
    a_t, a_v = to_dev(rng.integers(-3, 4, (rows, K)).astype(np.float32), "bf16")
    b_t, b_v = to_dev(rng.integers(-3, 4, (E, K, N)).astype(np.float32), "bf16")
    c = ks.dispatch.moe(a_t, b_t, H.np_i32_dev(offs), num_experts=E, n=N, k=K)
    torch.cuda.synchronize()
    assert c.dtype == torch.bfloat16 and tuple(c.shape) == (rows, N)
    ref = O.grouped_gemm_scalar(a_v, b_v.reshape(E, K, N), offs)
    np.testing.assert_array_equal(bits(c, "bf16"), round_out(ref, "bf16"))


def test_no_rows_and_bad_dtype():
    a_t, _ = to_dev(np.ones((4, 64), np.float32), "bf16")
    b_t, _ = to_dev(np.ones((2, 64, 32), np.float32), "bf16")
    c = sentinel(4, 32, "bf16")
    offs = H.np_i32_dev(np.zeros(3, np.int32))
    ks.moe.grouped_gemm(c, a_t, b_t, offs, 2, 0, 32, 64)  # total_rows 0: nothing written
    torch.cuda.synchronize()
    assert np.all(H.from_dev_f32(c) == -7.0)
    with pytest.raises(ks.KernelSetError):
        ks.moe.grouped_gemm(c, a_t, b_t, offs, 2, 4, 32, 64, dtype=DType.I8)
