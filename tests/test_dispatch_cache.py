"""ks.dispatch.fp8_gemm keeps one [K, N] copy per [N, K] weight tensor (CPU
check of the cache logic; the GEMM itself is covered by the GPU tests)."""
import gc

import torch

from kernel_set import dispatch as d


def test_transposed_weight_is_made_once_and_revalidated():
    w = torch.arange(6 * 4, dtype=torch.uint8).view(6, 4)  # [N, K]
    kn1 = d._weight_kn(w)
    assert torch.equal(kn1, w.t()) and kn1.is_contiguous()
    assert d._weight_kn(w) is kn1                 # reused while unmodified
    w.add_(1)                                     # in-place edit bumps the version
    kn2 = d._weight_kn(w)
    assert kn2 is not kn1 and torch.equal(kn2, w.t())
    other = w.clone()
    assert d._weight_kn(other) is not kn2         # keyed per tensor
    n_before = len(d._KN_CACHE)
    del other
    gc.collect()
    assert len(d._KN_CACHE) == n_before - 1       # dropped with its weight
