"""CPU baseline runner (test infrastructure): times the oracle on a benchmark
workload in a process of its own, which never touches the GPU, and prints one
JSON line. bench.py's cpu_baseline leg runs it as

    python -X faulthandler -m oracle.baseline --workload unet_step --threads N
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

import oracle  # noqa: E402


def _time(fn, budget_s, min_runs, max_runs):
    fn()  # warm-up
    times = []
    end = time.perf_counter() + budget_s
    while len(times) < min_runs or (time.perf_counter() < end and len(times) < max_runs):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return float(np.median(times)) * 1e3, len(times)


def unet_step(cfg: bool, budget_s: float):
    from moebius_cpu_amd import unet_params as U

    params = U.random_unet(seed=4000)
    inp = U.unet_input(seed=5000)
    net = oracle.UNet(params)
    ms, runs = _time(lambda: net.forward(inp.x, inp.timestep, cfg=cfg), budget_s, 1, 3)
    return ms, runs, ("the same denoise step (same seeded weights and inputs), median of "
                      f"{runs} runs after one warm-up")


def conv3x3_gn_silu(budget_s: float):
    from moebius_cpu_amd import workloads as W

    wl = W.conv3x3_gn_silu()

    def run():
        y = oracle.conv3x3(wl.x, wl.w, wl.b)
        oracle.group_norm(y, wl.groups, wl.eps, wl.gamma, wl.beta, silu=True)

    ms, runs = _time(run, budget_s, 5, 50)
    return ms, runs, f"full workload, median of {runs} runs after one warm-up"


def vae_decode(budget_s: float):
    from moebius_cpu_amd import synthetic as S
    from moebius_cpu_amd import vae_params as V

    vae = oracle.Vae(V.random_vae())
    lat = S.normal(24, (1, 64, 64, 4))
    ms, runs = _time(lambda: vae.decode(lat), budget_s, 1, 3)
    return ms, runs, f"the same decode ([1,64,64,4] -> [1,512,512,3]), median of {runs} runs after one warm-up"


def vae_encode(budget_s: float):
    from moebius_cpu_amd import synthetic as S
    from moebius_cpu_amd import vae_params as V

    vae = oracle.Vae(V.random_vae())
    images = V.vae_images(seed=25, b=2, h=512, w=512)
    noise = S.normal(26, (2, 64, 64, 4))
    ms, runs = _time(lambda: vae.encode(images, noise), budget_s, 1, 3)
    return ms, runs, f"the same encode (2 x [512,512,3]), median of {runs} runs after one warm-up"


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--workload", default="unet_step",
                    choices=["unet_step", "conv3x3_gn_silu", "vae_decode", "vae_encode"])
    ap.add_argument("--threads", type=int, default=0)
    ap.add_argument("--cond-only", action="store_true")
    ap.add_argument("--budget-s", type=float, default=20.0)
    args = ap.parse_args()
    if args.threads > 0:
        oracle.set_threads(args.threads)
    if args.workload == "unet_step":
        ms, runs, sample = unet_step(not args.cond_only, args.budget_s)
    elif args.workload == "vae_decode":
        ms, runs, sample = vae_decode(args.budget_s)
    elif args.workload == "vae_encode":
        ms, runs, sample = vae_encode(args.budget_s)
    else:
        ms, runs, sample = conv3x3_gn_silu(args.budget_s)
    print(json.dumps({"value": round(ms, 3), "unit": "ms", "cores": oracle.threads(), "runs": runs,
                      "sample": sample}))


if __name__ == "__main__":
    main()
