"""HIP-graph replay of every main kernel path (the way bench.py and serving
loops run them): each call is warmed up eagerly on a dedicated stream (library
scratch for that stream is allocated then), captured into a graph, and the
graph is replayed several times. Between replays the output is cleared and
unrelated eager calls of other shapes run on the default stream (which has its
own scratch). Every replay must reproduce the eager result bit for bit.
No path here records a memset into the graph.
"""
import zlib

import pytest
import torch

import kernel_set as ks
from kernel_set.enums import QuantMode

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _fp8(shape, g, scale=50.0):
    return (torch.randn(*shape, device=DEV, generator=g) * scale).to(torch.float8_e4m3fn)


def _w4(m, n, k, g, gs=128):
    a = torch.randn(m, k, device=DEV, generator=g).to(torch.bfloat16)
    b = torch.randint(0, 256, (k // 2, n), device=DEV, dtype=torch.uint8, generator=g)
    s = (torch.rand(k // gs, n, device=DEV, generator=g) * 0.018 + 0.002).to(torch.bfloat16)
    z = torch.randint(6, 10, (k // gs, n), device=DEV, generator=g).to(torch.bfloat16)
    c = torch.empty(m, n, device=DEV, dtype=torch.bfloat16)
    return lambda: ks.gemm.gemm_w4a16(c, a, b, s, z, m, n, k, group_size=gs), c


def _fp8_block(m, n, k, g):
    a = _fp8((m, k), g)
    b = _fp8((k, n), g)
    a_s = torch.rand(m, k // 128, device=DEV, generator=g) * 0.01 + 0.001
    b_s = torch.rand(k // 128, n // 128, device=DEV, generator=g) * 0.01 + 0.001
    out = torch.empty(m, n, device=DEV, dtype=torch.bfloat16)
    return lambda: ks.gemm.gemm_fp8_blockwise(out, a, b, a_s, b_s, m, n, k), out


def _fused(m, n, k, g):
    x = torch.randn(m, k, device=DEV, generator=g).to(torch.bfloat16)
    b = _fp8((k, n), g)
    b_s = torch.rand(k // 128, n // 128, device=DEV, generator=g) * 0.01 + 0.001
    out = torch.empty(m, n, device=DEV, dtype=torch.bfloat16)
    return lambda: ks.gemm.gemm_fp8_blockwise_fused_quant(out, x, b, b_s, m, n, k), out


def _fp8_plain(m, n, k, g):
    a = _fp8((m, k), g)
    b = _fp8((k, n), g)
    a_s = torch.rand(m, device=DEV, generator=g) * 0.01 + 0.001
    b_s = torch.rand(n, device=DEV, generator=g) * 0.01 + 0.001
    out = torch.empty(m, n, device=DEV, dtype=torch.bfloat16)
    return lambda: ks.gemm.gemm_fp8(out, a, b, a_s, b_s, m, n, k), out


def _w8a8(m, n, k, g):
    a = torch.randint(-127, 128, (m, k), device=DEV, dtype=torch.int8, generator=g)
    b = torch.randint(-127, 128, (k, n), device=DEV, dtype=torch.int8, generator=g)
    a_s = torch.rand(m, device=DEV, generator=g) * 0.02 + 0.01
    b_s = torch.rand(n, device=DEV, generator=g) * 0.02 + 0.01
    c = torch.empty(m, n, device=DEV, dtype=torch.bfloat16)
    return lambda: ks.gemm.gemm_w8a8(c, a, b, a_s, b_s, m, n, k, a_mode=QuantMode.PER_TOKEN,
                                     b_mode=QuantMode.PER_CHANNEL), c


def _w8a8_fused(m, n, k, g, a_mode=QuantMode.PER_TOKEN):
    x = torch.randn(m, k, device=DEV, generator=g).to(torch.bfloat16)
    b = torch.randint(-127, 128, (k, n), device=DEV, dtype=torch.int8, generator=g)
    b_s = torch.rand(n, device=DEV, generator=g) * 0.02 + 0.01
    c = torch.empty(m, n, device=DEV, dtype=torch.bfloat16)
    return lambda: ks.gemm.gemm_w8a8_fused_quant(c, x, b, b_s, m, n, k, a_mode=a_mode), c


def _quant_group(m, k, g):
    x = torch.randn(m, k, device=DEV, generator=g).to(torch.bfloat16)
    q = torch.empty(m, k, device=DEV, dtype=torch.float8_e4m3fn)
    s = torch.empty(m, k // 128, device=DEV, dtype=torch.float32)

    def fn():
        ks.quant.quantize_fp8_group(q, s, x, m, k)
    return fn, (q, s)


def _moe_offsets(counts):
    import numpy as np
    return torch.tensor(np.concatenate([[0], np.cumsum(counts)]).astype("int32"), device=DEV)


def _moe_dense(dtype, g, counts=(5, 0, 40, 17, 64, 3, 0, 30), k=512, n=384):
    rows = sum(counts)
    E = len(counts)
    a = torch.randn(rows, k, device=DEV, generator=g).to(dtype)
    b = (torch.randn(E, k, n, device=DEV, generator=g) * 0.05).to(dtype)
    offs = _moe_offsets(counts)
    c = torch.empty(rows, n, device=DEV, dtype=dtype)  # every row is routed
    return lambda: ks.moe.grouped_gemm(c, a, b, offs, E, rows, n, k), c


def _moe_w4(g, counts=(5, 0, 40, 17, 64, 3, 0, 30), k=512, n=384, gs=128):
    rows = sum(counts)
    E = len(counts)
    a = torch.randn(rows, k, device=DEV, generator=g).to(torch.bfloat16)
    b = torch.randint(0, 256, (E, k // 2, n), device=DEV, dtype=torch.uint8, generator=g)
    s = (torch.rand(E, k // gs, n, device=DEV, generator=g) * 0.018 + 0.002).to(torch.bfloat16)
    offs = _moe_offsets(counts)
    c = torch.empty(rows, n, device=DEV, dtype=torch.bfloat16)
    return lambda: ks.moe.grouped_gemm_w4a16(c, a, b, s, None, offs, E, rows, n, k, gs), c


CASES = {
    "moe_dense_bf16": lambda g: _moe_dense(torch.bfloat16, g),
    "moe_dense_fp8": lambda g: _moe_dense(torch.float8_e4m3fn, g),
    "moe_dense_f32": lambda g: _moe_dense(torch.float32, g),
    "moe_w4a16_ring": lambda g: _moe_w4(g),
    "w4a16_decode_M1": lambda g: _w4(1, 4096, 4096, g),
    "w4a16_decode_M8": lambda g: _w4(8, 4096, 4096, g),
    "w4a16_ring_M16": lambda g: _w4(16, 4096, 4096, g),
    "w4a16_dq_M256": lambda g: _w4(256, 2048, 1024, g),
    "fp8_block_skinny_M1": lambda g: _fp8_block(1, 7168, 2048, g),
    "fp8_block_splitk_M64": lambda g: _fp8_block(64, 2048, 4096, g),
    "fp8_block_fast_M512": lambda g: _fp8_block(512, 7168, 1024, g),
    "fp8_fused_M4": lambda g: _fused(4, 2048, 2048, g),
    "fp8_fused_staged_M40": lambda g: _fused(40, 2048, 2048, g),
    "fp8_plain_skinny_M3": lambda g: _fp8_plain(3, 4096, 2048, g),
    "w8a8_skinny_M2": lambda g: _w8a8(2, 4096, 4096, g),
    "w8a8_splitk_M128": lambda g: _w8a8(128, 1024, 4096, g),
    "w8a8_fused_M3": lambda g: _w8a8_fused(3, 2048, 4096, g),
    "w8a8_fused_tensor_M2": lambda g: _w8a8_fused(2, 2048, 2048, g, QuantMode.PER_TENSOR),
    "w8a8_fused_staged_M24": lambda g: _w8a8_fused(24, 2048, 2048, g),
    "quant_group_2048x7168": lambda g: _quant_group(2048, 7168, g),
}


def _snapshot(out):
    outs = out if isinstance(out, tuple) else (out,)
    return [o.clone() for o in outs], outs


@pytest.mark.parametrize("name", sorted(CASES))
def test_graph_replay_matches_eager(name):
    g = torch.Generator(device=DEV).manual_seed(zlib.crc32(name.encode()) & 0xFFFF)
    fn, out = CASES[name](g)
    other_fn, _ = _fp8_block(2, 4096, 1024, g)  # unrelated eager work (own scratch)
    other_fn2, _ = _w4(16, 2048, 2048, g)
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        fn()  # warm-up: scratch for `side` is allocated outside the capture
    torch.cuda.synchronize()
    ref, outs = _snapshot(out)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        fn()
    torch.cuda.synchronize()
    for rep in range(3):
        for o in outs:
            o.view(torch.uint8).fill_(0xA5)  # poison the outputs (eager fill kernel)
        other_fn()
        other_fn2()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for o, r in zip(outs, ref):
            assert torch.equal(o.view(torch.uint8), r.view(torch.uint8)), f"replay {rep} differs"


def test_scratch_growth_keeps_captured_graph_valid():
    """A graph captured at a small shape keeps working after an eager call on
    the same stream grows that stream's scratch: outgrown buffers are retired,
    never freed, so the graph's split-K nodes still address live memory."""
    g = torch.Generator(device=DEV).manual_seed(77)
    small_fn, small_out = _w4(1, 4096, 4096, g)   # 16-split decode plane
    big_fn, big_out = _w4(64, 4096, 14336, g)     # much larger ring-tile plane
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        small_fn()
    torch.cuda.synchronize()
    ref = small_out.clone()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        small_fn()
    torch.cuda.synchronize()
    with torch.cuda.stream(side):
        big_fn()  # grows side's scratch; the small plane is retired
    torch.cuda.synchronize()
    big_ref = big_out.clone()
    for rep in range(3):
        small_out.view(torch.uint8).fill_(0xA5)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(small_out, ref), f"replay {rep} after growth differs"
        with torch.cuda.stream(side):
            big_fn()
        torch.cuda.synchronize()
        assert torch.equal(big_out, big_ref)


def test_scratch_growth_refused_during_capture():
    """A call that would have to grow scratch while its stream is being
    captured returns KS_ERROR_INVALID_ARGUMENT (no sync, no allocation), and
    the capture itself stays usable."""
    from kernel_set._lib import KS_ERROR_INVALID_ARGUMENT, KernelSetError
    g = torch.Generator(device=DEV).manual_seed(78)
    fn, _ = _w4(1, 4096, 4096, g)
    fresh = torch.cuda.Stream()  # no scratch yet for this stream
    graph = torch.cuda.CUDAGraph()
    err = None
    with torch.cuda.stream(fresh):
        graph.capture_begin()
        try:
            fn()
        except KernelSetError as e:
            err = e
        finally:
            graph.capture_end()
    torch.cuda.synchronize()
    assert err is not None and err.status == KS_ERROR_INVALID_ARGUMENT
    assert "being captured" in str(err)
    with torch.cuda.stream(fresh):
        fn()  # eager: allocates normally
    torch.cuda.synchronize()
