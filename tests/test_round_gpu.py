"""GPU: the 16-bit output rounding shared by every kernel (elem<Out>::from_f32).

bf16 is pinned to the integer definition of round-to-nearest-even (NaN: top
16 bits with the quiet bit set), f16 to numpy's IEEE conversion (NaN: any
NaN), over whole 2^24-pattern ranges of fp32 bit patterns that cover
subnormals, exact ties, the largest finite values, infinities and NaNs of
both signs. Called through the test hook ks_testing_round_bits.
"""
import numpy as np
import pytest
import torch

import kernel_set as ks
from kernel_set import _lib
from kernel_set.enums import DType

pytestmark = pytest.mark.gpu

STARTS = [0x00000000, 0x3F000000, 0x477F0000, 0x7F000000, 0x80000000, 0xC7000000, 0xFF000000]
N = 1 << 24


def run(start, n, dtype):
    out = torch.empty(n, device="cuda", dtype=torch.int16)
    ks.check(_lib.lib.ks_testing_round_bits(out.data_ptr(), start, n, int(dtype),
                                            torch.cuda.current_stream().cuda_stream),
             "ks_testing_round_bits")
    torch.cuda.synchronize()
    return out.cpu().numpy().view(np.uint16)


def bf16_ref(u):
    u = u.astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    rne = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return np.where(nan, (u >> 16) | 0x40, rne).astype(np.uint16)


@pytest.mark.parametrize("start", STARTS)
def test_bf16_rounding(start):
    u = (np.arange(N, dtype=np.uint64) + start).astype(np.uint32)
    got = run(start, N, DType.BF16)
    np.testing.assert_array_equal(got, bf16_ref(u))


@pytest.mark.parametrize("start", STARTS)
def test_f16_rounding(start):
    u = (np.arange(N, dtype=np.uint64) + start).astype(np.uint32)
    got = run(start, N, DType.F16)
    with np.errstate(over="ignore", invalid="ignore"):
        ref = u.view(np.float32).astype(np.float16)
    nan = np.isnan(ref)
    np.testing.assert_array_equal(got[~nan], ref[~nan].view(np.uint16))
    g = got[nan]
    assert np.all(((g & 0x7C00) == 0x7C00) & ((g & 0x03FF) != 0))


def test_round_bits_rejects_bad_range():
    out = torch.empty(4, device="cuda", dtype=torch.int16)
    st = _lib.lib.ks_testing_round_bits(out.data_ptr(), 0xFFFFFFFF, 4, int(DType.BF16),
                                        torch.cuda.current_stream().cuda_stream)
    assert st != 0
