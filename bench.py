"""Benchmark: kernel-set quantized-inference path on one MI355X.

Headline (``value``): W4A16 GEMV achieved HBM GB/s at M=1, K=N=4096, g=128
(BASELINE config 1 shape, the north_star's >=70%-of-HBM target), weights cold:
``--rotate`` distinct weight sets (default 64 x 8.9 MB = 571 MB, over twice the
256 MB MALL) are cycled so every call streams its weights from HBM. A step is
one ks_gemm_w4a16 call.

Secondary lines (key ``secondary``) cover every BASELINE config: the fp8
blockwise GEMM and its 1x128 activation quantizer (config 3, the second half of
the metric; plus the same GEMM at decode M = 1 and M = 64 with cold weights), the W4A16 sweep (config 2), W8A8 (config 4) and the MoE grouped
W4A16 GEMM (config 5).

Timing: exactly --steps calls are captured into one HIP graph (so host launch
overhead is not measured) and replayed once after untimed warm-up replays that
cycle every rotated buffer set; HIP events recorded on the replay stream
bracket exactly the timed calls. Time per call = elapsed / steps. The
MFMA-bound secondary lines time max(32, min(steps, 64)) calls.

cpu_baseline: the reference bench's torch CPU path (benchmarks/bench.py
:1274-1285 W4A16, :1434-1502 fp8 blockwise: dequantize, then fp32 matmul) on
the host cores with torch's thread count stated, each half timed separately
(median of >= 3 after a warm-up); W4A16 at the headline shape and fp8
blockwise at the config 3 shape.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--only headline]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "kernel-set_amd"))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0      # MI355X HBM3E
PEAK_TFLOPS = {"fp8": 5000.0, "bf16": 2500.0, "int8": 5000.0}  # dense MFMA
METRIC = "W4A16 GEMV HBM GB/s (% peak) @M=1; fp8-block GEMM TFLOP/s (% peak) @M=2048"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


class Timer:
    """Graph-captured replay timing on a dedicated stream."""

    def __init__(self, torch, graph=True):
        self.torch = torch
        self.stream = torch.cuda.Stream()
        self.graph = graph

    def run(self, fn, rotate, steps, warmup):
        """Times exactly `steps` calls. fn(i) issues call i on buffer set i
        (i < rotate). The timed graph holds calls 0..steps-1 on sets i % rotate;
        a warm-up graph replays every set once in order (at least `warmup`
        calls) right before it, so set 0, the first timed one, was last touched
        `rotate` calls earlier (cold in HBM when the sets outgrow the MALL).
        At least 3 ms of warm-up replays are queued ahead of the start event,
        so the timed replay starts on a busy, full-clock GPU with no host gap.
        Returns (ms per call, calls timed)."""
        torch = self.torch
        inner = fn
        fn = lambda i: inner(i % rotate)  # noqa: E731
        with torch.cuda.stream(self.stream):
            for i in range(rotate):  # eager warm-up: allocates library scratch
                fn(i)
        torch.cuda.synchronize()
        if not self.graph:
            return self._run_eager(fn, steps, warmup)
        g_warm = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g_warm, stream=self.stream):
            for i in range(rotate):
                fn(i)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=self.stream):
            for i in range(steps):
                fn(i)
        with torch.cuda.stream(self.stream):
            g.replay()  # first replay of a graph carries one-time setup
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record()
            g_warm.replay()
            e1.record()
        torch.cuda.synchronize()
        warm_ms = max(e0.elapsed_time(e1), 1e-3)
        # Keep >= 3 ms of warm-up work queued ahead of the start event (and at
        # least `warmup` calls), so the GPU is busy at full clock while the
        # host enqueues the timed replay: no idle gap, no clock ramp inside it.
        reps = max(-(-warmup // rotate), int(3.0 / warm_ms) + 1)
        with torch.cuda.stream(self.stream):
            for _ in range(reps):
                g_warm.replay()
            start = torch.cuda.Event(enable_timing=True)
            end = torch.cuda.Event(enable_timing=True)
            start.record()
            g.replay()
            end.record()
        torch.cuda.synchronize()
        ms = start.elapsed_time(end) / steps
        del g, g_warm
        return ms, steps

    def _run_eager(self, fn, steps, warmup):
        """Plain launches, each call bracketed by its own event pair on the
        launch stream (profiler-friendly: no graph). Returns the mean
        event-measured duration of one call."""
        torch = self.torch
        with torch.cuda.stream(self.stream):
            for i in range(warmup):
                fn(i)
            torch.cuda.synchronize()
            ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                  for _ in range(steps)]
            # A bounded spin kernel holds the stream while the host enqueues
            # every call, so the event pairs time GPU execution, not host gaps.
            torch.cuda._sleep(self._sleep_cycles(steps * 300e-6))
            for i, (a, b) in enumerate(ev):
                a.record()
                fn(i)
                b.record()
        torch.cuda.synchronize()
        return sum(a.elapsed_time(b) for a, b in ev) / steps, steps

    def _sleep_cycles(self, seconds):
        torch = self.torch
        if not hasattr(self, "_cyc_per_s"):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            with torch.cuda.stream(self.stream):
                a.record()
                torch.cuda._sleep(1 << 20)
                b.record()
            torch.cuda.synchronize()
            self._cyc_per_s = (1 << 20) / max(a.elapsed_time(b) * 1e-3, 1e-6)
        return int(min(seconds, 1.0) * self._cyc_per_s)


PROFILES = os.path.join(ROOT, "profiles")
HEADLINE_KEY = "w4a16_gemv_M1_K4096_N4096 (headline)"


def measured_traffic():
    """HBM bytes per call of each bench line, from the committed rocprofv3 PMC
    summaries in profiles/ (FETCH_SIZE + WRITE_SIZE per dispatch, scaled by a
    copy calibration): lines `traffic_bytes_per_call[<line key>]: <bytes>`."""
    out = {}
    try:
        names = sorted(os.listdir(PROFILES))
    except OSError:
        return out
    for fn in names:
        if not fn.endswith(".md"):
            continue
        with open(os.path.join(PROFILES, fn)) as f:
            for ln in f:
                if ln.startswith("traffic_bytes_per_call[") and "]:" in ln:
                    key, val = ln[len("traffic_bytes_per_call["):].split("]:", 1)
                    out[key] = int(float(val.strip()))
    return out


def rot_copies(t, n):
    return [t] + [t.clone() for _ in range(n - 1)]


# ---------------------------------------------------------------------------
# workloads: each returns (fn, per_graph, bytes/call, flops/call, extra)
# ---------------------------------------------------------------------------
def wl_w4a16(torch, ks, H, m, k, n, gs, zero_mode, rotate, seed=0):
    import oracle as O
    a, codes, s, z = H.w4a16_inputs(m, k, n, gs, zero_mode, seed)
    at, _ = H.to_dev(a, "bf16")
    bs = rot_copies(H.np_u8_dev(O.pack_k2_uint8(codes)), rotate)
    ss = rot_copies(H.to_dev(s, "bf16")[0], rotate)
    zs = rot_copies(H.to_dev(z, "bf16")[0], rotate)
    c = torch.empty(m, n, device="cuda", dtype=torch.bfloat16)

    def fn(i):
        ks.gemm.gemm_w4a16(c, at, bs[i], ss[i], zs[i], m, n, k, gs)

    nbytes = (k // 2) * n + 2 * (k // gs) * n * 2 + m * k * 2 + m * n * 2
    return fn, rotate, nbytes, 2.0 * m * n * k


def wl_quant_group(torch, ks, H, rotate):
    rows, cols = 2048, 7168
    rng = np.random.default_rng(33)
    x = rng.standard_normal((rows, cols)).astype(np.float32)
    xs = rot_copies(H.to_dev(x, "bf16")[0], rotate)
    out = torch.empty(rows, cols, device="cuda", dtype=torch.float8_e4m3fn)
    sc = torch.empty(rows, cols // 128, device="cuda", dtype=torch.float32)

    def fn(i):
        ks.quant.quantize_fp8_group(out, sc, xs[i], rows, cols, group_size=128)

    nbytes = rows * cols * 2 + rows * cols + rows * (cols // 128) * 4
    return fn, rotate, nbytes, 0.0


def config3_activations(torch, ks, seed=2048, m=2048, k=7168):
    """BASELINE config 3 activations: bf16 [M, K] ~N(0,1) with 0.1% of the
    entries x50, quantized by ks_quantize_fp8_group (1x128 e4m3fn)."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    x = torch.randn(m, k, device="cuda", generator=g)
    idx = torch.randperm(m * k, device="cuda", generator=g)[: (m * k) // 1000]
    x.view(-1)[idx] *= 50.0
    x = x.to(torch.bfloat16)
    a8, a_s = ks.dispatch.per_token_group_quant(x, group_size=128)
    return x, a8, a_s


def block_quant_weight(torch, k, n, seed, bk=128, bn=128):
    """BASELINE config 3 weights: fp32 [K, N] ~N(0, 0.02), e4m3fn with one fp32
    scale per (bk x bn) block, scale = max(amax / 448, 1e-12) (the reference
    bench's recipe, benchmarks/bench.py:1434-1461)."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    w = torch.randn(k, n, device="cuda", generator=g) * 0.02
    blk = w.view(k // bk, bk, n // bn, bn)
    b_s = (blk.abs().amax(dim=(1, 3)) / 448.0).clamp_min(1e-12)
    b8 = (blk / b_s[:, None, :, None]).view(k, n).to(torch.float8_e4m3fn)
    return b8, b_s.contiguous()


def wl_fp8_gemm(torch, ks, H, rotate=6):
    """Config 3: activations from ks_quantize_fp8_group (warm: one 14.7 MB set),
    block-quantized weights cold: `rotate` distinct 51 MB sets (308 MB at 6,
    over the 256 MB MALL), so every call streams B from HBM."""
    m, n, k = 2048, 7168, 7168
    _, a8, a_s = config3_activations(torch, ks)
    ws = [block_quant_weight(torch, k, n, 100 + r) for r in range(rotate)]
    out = torch.empty(m, n, device="cuda", dtype=torch.bfloat16)

    def fn(i):
        b8, b_s = ws[i]
        ks.gemm.gemm_fp8_blockwise(out, a8, b8, a_s, b_s, m, n, k)

    nbytes = m * k + k * n + m * n * 2 + a_s.numel() * 4 + ws[0][1].numel() * 4
    return fn, rotate, nbytes, 2.0 * m * n * k


def wl_fp8_plain(torch, ks, H, rotate=6):
    """ks_gemm_fp8 at the config 3 shape: the same activations quantized per
    token (ks_quantize_fp8), weights ~N(0, 0.02) quantized per output channel;
    weights cold as in wl_fp8_gemm."""
    m, n, k = 2048, 7168, 7168
    x, _, _ = config3_activations(torch, ks)
    a8 = torch.empty(m, k, device="cuda", dtype=torch.float8_e4m3fn)
    a_s = torch.empty(m, device="cuda", dtype=torch.float32)
    ks.quant.quantize_fp8(a8, a_s, x, m, k, mode=1)  # KS_QUANT_PER_TOKEN
    ws = []
    for r in range(rotate):
        g = torch.Generator(device="cuda").manual_seed(200 + r)
        w = torch.randn(k, n, device="cuda", generator=g) * 0.02
        b_s = (w.abs().amax(dim=0) / 448.0).clamp_min(1e-12)
        ws.append(((w / b_s).to(torch.float8_e4m3fn), b_s.contiguous()))
        del w
    out = torch.empty(m, n, device="cuda", dtype=torch.bfloat16)

    def fn(i):
        b8, b_s = ws[i]
        ks.gemm.gemm_fp8(out, a8, b8, a_s, b_s, m, n, k)

    nbytes = m * k + k * n + m * n * 2 + (m + n) * 4
    return fn, rotate, nbytes, 2.0 * m * n * k


def wl_fp8_skinny(torch, ks, H, m, rotate=6):
    """fp8 blockwise GEMM at decode / small-batch M (N = K = 7168, the config 3
    width): `rotate` distinct 51 MB weight sets (over the 256 MB MALL at 6) so
    every call streams B from HBM."""
    import oracle as O
    n = k = 7168
    rng = np.random.default_rng(m)
    a8 = torch.from_numpy(O.fp8_encode(rng.standard_normal((m, k)).astype(np.float32))).cuda()
    a_s = torch.from_numpy(rng.uniform(0.001, 0.01, (m, k // 128)).astype(np.float32)).cuda()
    g = torch.Generator(device="cuda").manual_seed(m)
    bs = [torch.randint(0, 256, (k, n), device="cuda", dtype=torch.uint8, generator=g)
          .bitwise_and_(0x77).view(torch.float8_e4m3fn) for _ in range(rotate)]  # finite codes
    bsc = [torch.rand(k // 128, n // 128, device="cuda", generator=g) * 0.01 + 0.001
           for _ in range(rotate)]
    a8 = a8.view(torch.float8_e4m3fn)
    out = torch.empty(m, n, device="cuda", dtype=torch.bfloat16)

    def fn(i):
        ks.gemm.gemm_fp8_blockwise(out, a8, bs[i], a_s, bsc[i], m, n, k)

    nbytes = m * k + k * n + m * n * 2 + a_s.numel() * 4 + bsc[0].numel() * 4
    return fn, rotate, nbytes, 2.0 * m * n * k


def wl_w8a8(torch, ks, H):
    m = n = k = 4096
    rng = np.random.default_rng(8)
    a = torch.from_numpy(rng.integers(-127, 128, (m, k)).astype(np.int8)).cuda()
    b = torch.from_numpy(rng.integers(-127, 128, (k, n)).astype(np.int8)).cuda()
    a_s = torch.rand(m, device="cuda") * 0.02 + 0.01
    b_s = torch.rand(n, device="cuda") * 0.02 + 0.01
    out = torch.empty(m, n, device="cuda", dtype=torch.bfloat16)

    def fn(i):
        ks.gemm.gemm_w8a8(out, a, b, a_s, b_s, m, n, k)

    return fn, 8, m * k + k * n + m * n * 2, 2.0 * m * n * k


def wl_moe(torch, ks, H, K, N, rotate):
    import oracle as O
    E, T, top_k, gs = 64, 256, 8, 128
    rng = np.random.default_rng(K)
    ids = O.moe_topk_ids(rng.standard_normal((T, E)).astype(np.float32), top_k)
    row_src, offs = O.moe_group_rows(ids, E, 16)
    a = np.zeros((len(row_src), K), np.float32)
    live = row_src >= 0
    a[live] = rng.standard_normal((int(live.sum()), K)).astype(np.float32)
    at, _ = H.to_dev(a, "bf16")
    b = np.stack([O.pack_k2_uint8(rng.integers(0, 16, (K, N), dtype=np.uint8)) for _ in range(E)])
    bs = rot_copies(H.np_u8_dev(b), rotate)
    s = rng.uniform(0.002, 0.02, (E, K // gs, N)).astype(np.float32)
    ss = rot_copies(H.to_dev(s, "bf16")[0], rotate)
    zs = rot_copies(H.to_dev(np.full_like(s, 8.0), "bf16")[0], rotate)
    offt = H.np_i32_dev(offs)
    c = torch.empty(len(row_src), N, device="cuda", dtype=torch.bfloat16)
    rows = int(live.sum())

    def fn(i):
        ks.moe.grouped_gemm_w4a16(c, at, bs[i], ss[i], zs[i], offt, E, len(row_src), N, K, gs)

    nbytes = E * (K // 2) * N + 2 * E * (K // gs) * N * 2 + rows * K * 2 + rows * N * 2
    return fn, rotate, nbytes, 2.0 * rows * N * K


def wl_moe_dense(torch, ks, H, K, N, rotate):
    """Dense grouped GEMM (ks_moe_grouped_gemm) at the config 5 routing and
    shapes with bf16 weights ~N(0, 0.02) (the reference's dense form)."""
    import oracle as O
    E, T, top_k = 64, 256, 8
    rng = np.random.default_rng(K + 1)
    ids = O.moe_topk_ids(rng.standard_normal((T, E)).astype(np.float32), top_k)
    row_src, offs = O.moe_group_rows(ids, E, 16)
    a = np.zeros((len(row_src), K), np.float32)
    live = row_src >= 0
    a[live] = rng.standard_normal((int(live.sum()), K)).astype(np.float32)
    at, _ = H.to_dev(a, "bf16")
    g = torch.Generator(device="cuda")
    g.manual_seed(K)
    bs = [(torch.randn(E, K, N, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
          for _ in range(rotate)]
    offt = H.np_i32_dev(offs)
    c = torch.empty(len(row_src), N, device="cuda", dtype=torch.bfloat16)
    rows = int(live.sum())

    def fn(i):
        ks.moe.grouped_gemm(c, at, bs[i], offt, E, len(row_src), N, K)

    nbytes = E * K * N * 2 + rows * K * 2 + rows * N * 2
    return fn, rotate, nbytes, 2.0 * rows * N * K


def _median_time(fn, budget_s, min_reps=3):
    fn()  # warm-up
    times = []
    t0 = time.perf_counter()
    while len(times) < min_reps or time.perf_counter() - t0 < budget_s:
        t1 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t1)
    return float(np.median(times)), len(times)


def cpu_baseline(torch, H, budget_s=10.0):
    """The reference bench's torch CPU path (benchmarks/bench.py:1274-1285 for
    W4A16, :1434-1502 for fp8 blockwise), timed on the host cores:
    (i) dequantize the weights, (ii) fp32 matmul. Each piece is a median of
    >= 3 timed repetitions after one warm-up, within `budget_s` seconds each."""
    threads = int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count() or 1)
    torch.set_num_threads(threads)
    # ---- W4A16, config 1 (M=1, K=N=4096, g=128, zeros 8) ----
    m, k, n, gs = 1, 4096, 4096, 128
    a, codes, s, z = H.w4a16_inputs(m, k, n, gs, "fixed8", 0)
    import oracle as O
    packed = torch.from_numpy(O.pack_k2_uint8(codes))
    at = torch.from_numpy(a).to(torch.bfloat16)
    st = torch.from_numpy(s).to(torch.bfloat16)
    zt = torch.from_numpy(z).to(torch.bfloat16)
    kk = torch.arange(k)
    grp = kk // gs
    odd = (kk & 1).view(k, 1).bool()
    holder = {}

    def dequant():
        byte = packed[kk >> 1]
        q = torch.where(odd, (byte >> 4) & 0xF, byte & 0xF).float()
        holder["w"] = ((q - zt.float()[grp]) * st.float()[grp]).to(torch.bfloat16)

    def matmul():
        holder["c"] = (at.float() @ holder["w"].float()).to(torch.bfloat16)

    t_dq, r_dq = _median_time(dequant, budget_s / 4)
    t_mm, r_mm = _median_time(matmul, budget_s / 4)
    nbytes = (k // 2) * n + 2 * (k // gs) * n * 2 + m * k * 2 + m * n * 2
    out = {
        "value": round(nbytes / (t_dq + t_mm) / 1e9, 4), "unit": "GB/s",
        "cores": torch.get_num_threads(), "kind": "port",
        "os_cpu_count": os.cpu_count(),
        "sample": (f"torch CPU ({torch.get_num_threads()} threads) W4A16 M={m} K={k} N={n} g={gs}: "
                   f"(i) K-packed int4 dequant -> bf16 [K,N] median {t_dq * 1e3:.3f} ms of {r_dq}, "
                   f"(ii) fp32 matmul median {t_mm * 1e3:.3f} ms of {r_mm}; value = algorithmic "
                   "bytes / (i + ii)"),
        "w4a16_dequant_ms": round(t_dq * 1e3, 4), "w4a16_matmul_ms": round(t_mm * 1e3, 4),
    }
    # ---- fp8 blockwise, config 3 shape (M=2048, N=K=7168, 1x128 / 128x128) ----
    m, n, k = 2048, 7168, 7168
    gen = torch.Generator().manual_seed(3)
    a8 = (torch.randn(m, k, generator=gen) * 100).clamp(-448, 448).to(torch.float8_e4m3fn)
    b8 = (torch.randn(k, n, generator=gen) * 100).clamp(-448, 448).to(torch.float8_e4m3fn)
    a_s = torch.rand(m, k // 128, generator=gen) * 0.01 + 1e-4
    b_s = torch.rand(k // 128, n // 128, generator=gen) * 1e-4 + 1e-5

    def dequant8():
        holder["ad"] = (a8.float().view(m, k // 128, 128) * a_s[:, :, None]).view(m, k)
        holder["bd"] = (b8.float().view(k // 128, 128, n // 128, 128)
                        * b_s[:, None, :, None]).view(k, n)

    def matmul8():
        holder["o8"] = (holder["ad"] @ holder["bd"]).to(torch.bfloat16)

    t_dq8, r_dq8 = _median_time(dequant8, budget_s / 4)
    t_mm8, r_mm8 = _median_time(matmul8, budget_s / 4)
    fl = 2.0 * m * n * k
    out["fp8_blockwise"] = {
        "value": round(fl / (t_dq8 + t_mm8) / 1e12, 4), "unit": "TFLOP/s",
        "cores": torch.get_num_threads(), "kind": "port",
        "sample": (f"torch CPU fp8 blockwise M={m} N={n} K={k}: (i) float(fp8) * scale for A and B "
                   f"median {t_dq8 * 1e3:.1f} ms of {r_dq8}, (ii) fp32 matmul median "
                   f"{t_mm8 * 1e3:.1f} ms of {r_mm8}"),
        "dequant_ms": round(t_dq8 * 1e3, 2), "matmul_ms": round(t_mm8 * 1e3, 2),
    }
    return out


def line(name, ms, calls, nbytes, flops, bound, peak_key=None, note=None):
    d = {"us_per_call": round(ms * 1e3, 3), "calls": calls, "bytes": nbytes,
         "GB/s": round(nbytes / (ms * 1e-3) / 1e9, 2)}
    if note:
        d["inputs"] = note
    if flops:
        d["TFLOP/s"] = round(flops / (ms * 1e-3) / 1e12, 2)
    if bound == "hbm":
        d["roofline_frac"] = round(d["GB/s"] / HBM_PEAK_GBS, 4)
    else:
        d["roofline_frac"] = round(d["TFLOP/s"] / PEAK_TFLOPS[peak_key], 4)
    d["bound"] = bound if bound == "hbm" else f"mfma-{peak_key}"
    log(f"{name}: {d}")
    return d


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1024)
    ap.add_argument("--warmup", type=int, default=128)
    ap.add_argument("--rotate", type=int, default=64)
    ap.add_argument("--only", default="all",
                    help="all | headline | comma list of gemm8, quant, w4a16, moe")
    ap.add_argument("--cpu-budget", type=float, default=10.0)
    ap.add_argument("--no-graph", action="store_true",
                    help="plain launches with per-call events (for rocprofv3 runs)")
    ap.add_argument("--calib-copy-mib", type=int, default=0,
                    help="only run --steps device copies of this many MiB (PMC byte calibration)")
    args = ap.parse_args()

    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU only: kernel-set is a "
                                   "single-device kernel library and every GPU box here "
                                   "has one GPU; run with --gpus 1"}))
        sys.exit(2)

    import torch
    if args.calib_copy_mib:
        nb = args.calib_copy_mib << 20
        src = torch.empty(nb, dtype=torch.uint8, device="cuda").fill_(7)
        dst = torch.empty_like(src)
        for _ in range(args.steps):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calib_copy_bytes": nb, "copies": args.steps}), flush=True)
        return
    import kernel_set as ks
    from tests import helpers as H

    dev_name = torch.cuda.get_device_name(0)
    props = torch.cuda.get_device_properties(0)
    log(f"device: {dev_name} {getattr(props, 'gcnArchName', '')} CUs={props.multi_processor_count}")
    T = Timer(torch, graph=not args.no_graph)

    # ---- headline: W4A16 GEMV, config 1 shape, cold weights ----------------
    m, k, n, gs = 1, 4096, 4096, 128
    fn, per, nbytes, flops = wl_w4a16(torch, ks, H, m, k, n, gs, "fixed8", args.rotate)
    ms, calls = T.run(fn, per, args.steps, args.warmup)
    gbs = nbytes / (ms * 1e-3) / 1e9
    log(f"w4a16 gemv M=1 K=N=4096 (cold): {ms * 1e3:.3f} us/call, {gbs:.1f} GB/s")
    wfn, wper, _, _ = wl_w4a16(torch, ks, H, m, k, n, gs, "fixed8", 1)
    ms_warm, _ = T.run(wfn, wper, args.steps, args.warmup)

    result = {
        "metric": METRIC,
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": calls,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16 x int4 (fp32 accumulate)",
        "data": "synthetic (BASELINE config 1 distributions, seeded)",
        "config": {"workload": "w4a16_gemv", "M": m, "K": k, "N": n, "group_size": gs,
                   "zeros": "fixed 8.0", "weights": f"cold: {args.rotate} rotated copies",
                   "timing": ("per-call events, plain launches" if args.no_graph else
                              "HIP-graph replay, events on the replay stream"),
                   "device": dev_name},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic().get(HEADLINE_KEY),
                     "kernel": "ks_gemm_w4a16 call = ks::w4dec::dec_kernel + ks::w4a16::dec_reduce_kernel",
                     "bytes_per_launch": nbytes},
        "warm_cache": {"us_per_call": round(ms_warm * 1e3, 3),
                       "GB/s": round(nbytes / (ms_warm * 1e-3) / 1e9, 2)},
    }

    only = set(args.only.split(","))
    if "all" in only:
        only = {"gemm8", "quant", "w4a16", "moe"}
    if only - {"headline"}:
        sec = {}
        steps = max(64, args.steps // 8)
        n_mfma = max(32, min(args.steps, 64))  # timed calls per MFMA-bound line
        if "gemm8" in only:
            fn, per, nb, fl = wl_fp8_gemm(torch, ks, H)
            ms2, c2 = T.run(fn, per, n_mfma, 12)
            sec["fp8_blockwise_gemm_M2048_N7168_K7168"] = line(
                "fp8 gemm", ms2, c2, nb, fl, "mfma", "fp8",
                note="config 3: A = ks_quantize_fp8_group(bf16 N(0,1), 0.1% x50), warm; "
                     "W ~N(0,0.02) 128x128 block-quantized, cold (6 rotated 51 MB sets)")
            fn, per, nb, fl = wl_fp8_plain(torch, ks, H)
            ms2, c2 = T.run(fn, per, n_mfma, 12)
            sec["fp8_per_token_gemm_M2048_N7168_K7168"] = line(
                "fp8 gemm per-token", ms2, c2, nb, fl, "mfma", "fp8",
                note="config 3 activations per-token quantized (warm); W per-channel, cold")
            for mm in (1, 64):  # decode / small batch: HBM-bound (B = 51 MB)
                fn, per, nb, fl = wl_fp8_skinny(torch, ks, H, mm)
                ms2, c2 = T.run(fn, per, max(64, steps // 4), 12)
                sec[f"fp8_blockwise_gemm_M{mm}_N7168_K7168_cold"] = line(
                    f"fp8 gemm M={mm}", ms2, c2, nb, fl, "hbm")
        if "quant" in only:
            fn, per, nb, fl = wl_quant_group(torch, ks, H, 16)
            ms2, c2 = T.run(fn, per, steps, 32)
            sec["quant_fp8_group_2048x7168_cold"] = line("quant group", ms2, c2, nb, fl, "hbm")
        for mm in ((1, 16, 64, 256) if "w4a16" in only else ()):
            fn, per, nb, fl = wl_w4a16(torch, ks, H, mm, 4096, 14336, 128, "int69", 16, seed=mm)
            ms2, c2 = T.run(fn, per, steps, 32)
            t_roof = max(nb / (HBM_PEAK_GBS * 1e9), fl / (PEAK_TFLOPS["bf16"] * 1e12))
            d = line(f"w4a16 M={mm}", ms2, c2, nb, fl, "hbm")
            d["roofline_frac"] = round(t_roof / (ms2 * 1e-3), 4)
            d["bound"] = "hbm" if nb / (HBM_PEAK_GBS * 1e9) >= fl / (PEAK_TFLOPS["bf16"] * 1e12) else "mfma-bf16"
            sec[f"w4a16_M{mm}_K4096_N14336_cold"] = d
        if "gemm8" in only:
            fn, per, nb, fl = wl_w8a8(torch, ks, H)
            ms2, c2 = T.run(fn, per, n_mfma, 8)
            sec["w8a8_M4096_N4096_K4096"] = line("w8a8", ms2, c2, nb, fl, "mfma", "int8")
        for K_, N_, nm in (((2048, 1536, "gate_up"), (768, 2048, "down")) if "moe" in only else ()):
            fn, per, nb, fl = wl_moe(torch, ks, H, K_, N_, 4)
            ms2, c2 = T.run(fn, per, steps, 16)
            sec[f"moe_w4a16_{nm}_E64_top8_T256_cold"] = line(f"moe {nm}", ms2, c2, nb, fl, "hbm")
        for K_, N_, nm in (((2048, 1536, "gate_up"), (768, 2048, "down")) if "moe" in only else ()):
            fn, per, nb, fl = wl_moe_dense(torch, ks, H, K_, N_, 2)
            ms2, c2 = T.run(fn, per, steps, 16)
            sec[f"moe_dense_bf16_{nm}_E64_top8_T256_cold"] = line(f"moe dense {nm}", ms2, c2, nb, fl, "hbm")
        traffic = measured_traffic()
        for key, d in sec.items():
            d["traffic"] = traffic.get(key)
        result["secondary"] = sec
        fp8 = sec.get("fp8_blockwise_gemm_M2048_N7168_K7168")
        if fp8:
            result["fp8_gemm_tflops"] = fp8["TFLOP/s"]
            result["fp8_gemm_frac_of_peak"] = fp8["roofline_frac"]

    result["cpu_baseline"] = cpu_baseline(torch, H, args.cpu_budget)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
