"""Benchmark of the MI355X conv/norm hot path.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME] [--no-cpu]

Prints ONE JSON line. A step is one pass of the workload over synthetic
seeded inputs already resident in HBM; the timed region is K steps between two
HIP events on the library's stream (synchronised on both sides). Also
reported: the dominant kernel's roofline (algorithmic work / its average
duration, timed the same way) and the CPU oracle timed on the host cores.
One GPU only: --gpus above 1 exits with a message.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "ms per 512² UNet denoise step; conv MFMA util %; GroupNorm HBM GB/s"
PEAK_F32_MFMA_TFLOPS = 157.3
PEAK_HBM_GBPS = 8000.0


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def time_region(ctx, fn, steps):
    """Average ms of fn() over `steps` calls between two events on the stream."""
    ctx.synchronize()
    e0, e1 = ctx.event(), ctx.event()
    e0.record()
    for _ in range(steps):
        fn()
    e1.record()
    ms = e0.elapsed_ms(e1)
    ctx.synchronize()
    return ms / steps


def cpu_threads():
    return int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count() or 1)


def bench_conv_gn(args):
    """conv3x3 64x64x320 -> 320 + GroupNorm(32, eps 1e-5) + SiLU, f32."""
    from moebius_cpu_amd import engine as E
    from moebius_cpu_amd import workloads as W

    ctx = E.Context(0)
    wl = W.conv3x3_gn_silu()
    x = E.Tensor.from_numpy(ctx, wl.x)
    conv = E.Conv3x3.same(ctx, 320, 320, E.Param(ctx, wl.w), wl.b)
    gn = E.GroupNorm(ctx, wl.groups, wl.eps, wl.gamma, wl.beta)
    y, z = E.Tensor(ctx, *wl.x.shape[:3], 320), E.Tensor(ctx, *wl.x.shape[:3], 320)

    def step():
        conv.forward(x, y)
        gn.forward(y, None, True, z)

    for _ in range(args.warmup):
        step()
    ms = time_region(ctx, step, args.steps)
    conv_ms = time_region(ctx, lambda: conv.forward(x, y), args.steps)
    gn_ms = time_region(ctx, lambda: gn.forward(y, None, True, z), args.steps)
    elems = y.pixels() * 320
    conv_tflops = wl.flops / (conv_ms * 1e-3) / 1e12
    gn_gbps = 8.0 * elems / (gn_ms * 1e-3) / 1e9

    out = {
        "metric": METRIC, "value": round(ms, 5), "unit": "ms", "higher_is_better": False,
        "ms_per_step": round(ms, 5), "dtype": "f32",
        "config": {"workload": "conv3x3 64x64x320->320 + GroupNorm(32)+SiLU (f32, batch 1)",
                   "input": [1, 64, 64, 320], "weight": [320, 3, 3, 320], "groups": 32, "eps": 1e-5},
        "roofline": {"bound": "mfma", "kernel": "gemm_f32_kernel (implicit-GEMM conv3x3)",
                     "achieved": round(conv_tflops, 3), "peak": PEAK_F32_MFMA_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(conv_tflops / PEAK_F32_MFMA_TFLOPS, 4), "traffic": None,
                     "work_per_launch": f"{wl.flops / 1e9:.3f} GFLOP", "avg_launch_ms": round(conv_ms, 5)},
        "components": {"conv_ms": round(conv_ms, 5), "conv_mfma_util": round(conv_tflops / PEAK_F32_MFMA_TFLOPS, 4),
                       "groupnorm_silu_ms": round(gn_ms, 5), "groupnorm_gbps_8B_per_elem": round(gn_gbps, 1)},
    }
    if not args.no_cpu:
        import oracle

        oracle.set_threads(cpu_threads())
        oracle.group_norm(oracle.conv3x3(wl.x, wl.w, wl.b), 32, wl.eps, wl.gamma, wl.beta, silu=True)
        times = []
        t_end = time.perf_counter() + 15.0
        while len(times) < 5 or (time.perf_counter() < t_end and len(times) < 50):
            t0 = time.perf_counter()
            oracle.group_norm(oracle.conv3x3(wl.x, wl.w, wl.b), 32, wl.eps, wl.gamma, wl.beta, silu=True)
            times.append(time.perf_counter() - t0)
        out["cpu_baseline"] = {"value": round(float(np.median(times)) * 1e3, 3), "unit": "ms",
                               "cores": oracle.threads(), "kind": "port",
                               "sample": f"full workload, median of {len(times)} runs after one warm-up "
                                         "(C++ restatement of the CPU engine: Winograd F(2x2,3x3) + GN)"}
    ctx.close()
    return out


WORKLOADS = {"conv3x3_gn_silu": bench_conv_gn}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="conv3x3_gn_silu", choices=sorted(WORKLOADS))
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (got --gpus {args.gpus}); the multi-GPU design is described in "
              "DESIGN.md and no multi-GPU figure is produced.", file=sys.stderr)
        sys.exit(2)
    res = WORKLOADS[args.workload](args)
    line = {"metric": res.pop("metric"), "value": res.pop("value"), "unit": res.pop("unit"), "n_gpus": 1,
            "steps": args.steps, "warmup": args.warmup, "ms_per_step": res.pop("ms_per_step"),
            "higher_is_better": res.pop("higher_is_better"), "scaling": "weak", "vs_baseline": None,
            "dtype": res.pop("dtype"), "data": "synthetic (seeded splitmix64/Box-Muller; random-init weights)",
            **res}
    print(json.dumps(line))


if __name__ == "__main__":
    main()
