"""GPU parity of ks_gemm_w4a16_noalloc, the entry point that never allocates.

It runs the kernels of ks_gemm_w4a16 with the split-K partial planes in a fixed
per-device 16 MiB array, so its output must equal ks_gemm_w4a16's bit for bit
(and, through that, the oracle within the W4A16 tolerance). Two calls run in a
row, the second with a smaller input, because every call on a device shares
the array and keeps the previous call's contents. A shape whose planes exceed
the array must be refused before any kernel runs.
"""
import numpy as np
import pytest
import torch

import kernel_set as ks
import oracle as O
from kernel_set._lib import KS_ERROR_INVALID_ARGUMENT, KernelSetError
from tests import helpers as H

pytestmark = pytest.mark.gpu
TOL = 1e-2


def _inputs(m, k, n, gs, seed):
    a, codes, s, z = H.w4a16_inputs(m, k, n, gs, "int69", seed)
    b = O.pack_k2_uint8(codes)
    at, av = H.to_dev(a, "bf16")
    st, sv = H.to_dev(s, "bf16")
    zt, zv = H.to_dev(z, "bf16")
    return (at, H.np_u8_dev(b), st, zt), (av, b, sv, zv)


def _bits(t):
    return t.view(torch.int16).cpu().numpy()


# (m, k, n, gs) pairs: the second call of each pair is smaller. Paths: decode
# MFMA (M <= 8, 16 K splits), LDS-ring tile with K split (8 < M <= 64),
# dequantize-to-LDS tile with K split (M > 64 on a small grid), dot2 decode
# (group size 16).
PAIRS = [
    ((1, 4096, 4096, 128), (1, 2048, 1024, 128)),
    ((8, 4096, 14336, 128), (3, 4096, 4096, 128)),
    ((64, 4096, 14336, 128), (16, 2048, 4096, 128)),
    ((128, 4096, 1024, 128), (96, 2048, 512, 64)),
    ((4, 2048, 1040, 16), (2, 1024, 528, 16)),
]


@pytest.mark.parametrize("first,second", PAIRS)
def test_noalloc_matches_allocating_entry(first, second):
    for idx, (m, k, n, gs) in enumerate((first, second)):
        print(f"noalloc case m={m} k={k} n={n} gs={gs}", flush=True)
        (at, bt, st, zt), (av, b, sv, zv) = _inputs(m, k, n, gs, seed=31 * idx + m)
        c_ref = torch.full((m, n), float("nan"), device="cuda", dtype=torch.bfloat16)
        c_new = torch.full((m, n), float("nan"), device="cuda", dtype=torch.bfloat16)
        ks.gemm.gemm_w4a16(c_ref, at, bt, st, zt, m, n, k, gs)
        ks.gemm.gemm_w4a16_noalloc(c_new, at, bt, st, zt, m, n, k, gs)
        torch.cuda.synchronize()
        assert np.array_equal(_bits(c_new), _bits(c_ref)), (m, k, n, gs)
        ref = O.w4a16_ref(av, b, sv, zv, gs, "bf16")
        assert O.rel_err(H.from_dev_f32(c_new), ref) <= TOL


def test_noalloc_with_bias_repeated():
    m, k, n, gs = 2, 4096, 4096, 128
    (at, bt, st, zt), _ = _inputs(m, k, n, gs, seed=5)
    bias = torch.randn(n, device="cuda").to(torch.bfloat16)
    c_ref = torch.empty(m, n, device="cuda", dtype=torch.bfloat16)
    ks.gemm.gemm_w4a16(c_ref, at, bt, st, zt, m, n, k, gs, bias=bias)
    for _ in range(3):
        c_new = torch.empty(m, n, device="cuda", dtype=torch.bfloat16)
        ks.gemm.gemm_w4a16_noalloc(c_new, at, bt, st, zt, m, n, k, gs, bias=bias)
        torch.cuda.synchronize()
        assert np.array_equal(_bits(c_new), _bits(c_ref))


def test_noalloc_refuses_oversized_scratch():
    # M = 1, K = 4096: 16 K splits x 8 plane rows x N fp32 = 512 * N bytes,
    # 32 MiB at N = 65536 -- beyond the 16 MiB array. Refused before any launch.
    m, k, n, gs = 1, 4096, 65536, 128
    a = torch.randn(m, k, device="cuda").to(torch.bfloat16)
    b = torch.zeros(k // 2, n, device="cuda", dtype=torch.uint8)
    s = torch.ones(k // gs, n, device="cuda", dtype=torch.bfloat16)
    c = torch.full((m, n), 7.0, device="cuda", dtype=torch.bfloat16)
    with pytest.raises(KernelSetError) as ei:
        ks.gemm.gemm_w4a16_noalloc(c, a, b, s, None, m, n, k, gs)
    assert ei.value.status == KS_ERROR_INVALID_ARGUMENT
    assert "no-allocation" in str(ei.value)
    torch.cuda.synchronize()
    assert bool((c == 7.0).all())
    # the allocating entry point still serves the shape
    ks.gemm.gemm_w4a16(c, a, b, s, None, m, n, k, gs)
    torch.cuda.synchronize()
    assert bool((c.float() == 0.0).all())
