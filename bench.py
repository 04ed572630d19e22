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
PEAK_F16_MFMA_TFLOPS = 2500.0
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


def cpu_baseline(workload, extra=(), note=""):
    """Times the CPU oracle on the same workload in a child process that never
    touches the GPU (oracle/baseline.py); a failure there is reported, not fatal."""
    import subprocess

    cmd = [sys.executable, "-X", "faulthandler", "-m", "oracle.baseline", "--workload", workload,
           "--threads", str(cpu_threads()), *extra]
    log("CPU baseline: " + " ".join(cmd[1:]))
    try:
        r = subprocess.run(cmd, cwd=ROOT, capture_output=True, text=True, timeout=600)
    except subprocess.TimeoutExpired:
        return {"value": None, "unit": "ms", "cores": cpu_threads(), "kind": "port", "error": "timed out"}
    if r.returncode != 0:
        log(r.stderr[-2000:])
        return {"value": None, "unit": "ms", "cores": cpu_threads(), "kind": "port",
                "error": f"baseline process exited with {r.returncode}"}
    res = json.loads(r.stdout.strip().splitlines()[-1])
    return {"value": res["value"], "unit": "ms", "cores": res["cores"], "kind": "port",
            "sample": res["sample"] + note}


def bench_conv_gn(args):
    """conv3x3 64x64x320 -> 320 + GroupNorm(32, eps 1e-5) + SiLU, f32. The conv
    runs as Winograd F(2x2,3x3) (the CPU engine's algorithm for stride-1 convs);
    the implicit-GEMM conv is timed beside it."""
    from moebius_cpu_amd import engine as E
    from moebius_cpu_amd import workloads as W

    ctx = E.Context(0)
    wl = W.conv3x3_gn_silu()
    x = E.Tensor.from_numpy(ctx, wl.x)
    conv = E.Conv3x3.same(ctx, 320, 320, E.Param(ctx, wl.w), wl.b, winograd=True)
    conv_g = E.Conv3x3.same(ctx, 320, 320, E.Param(ctx, wl.w), wl.b)
    gn = E.GroupNorm(ctx, wl.groups, wl.eps, wl.gamma, wl.beta)
    y, z = E.Tensor(ctx, *wl.x.shape[:3], 320), E.Tensor(ctx, *wl.x.shape[:3], 320)

    def step():
        conv.forward(x, y)
        gn.forward(y, None, True, z)

    for _ in range(args.warmup):
        step()
    ms = time_region(ctx, step, args.steps)
    conv_ms = time_region(ctx, lambda: conv.forward(x, y), args.steps)
    conv_g.forward(x, y)
    gemm_ms = time_region(ctx, lambda: conv_g.forward(x, y), args.steps)
    gn_ms = time_region(ctx, lambda: gn.forward(y, None, True, z), args.steps)
    elems = y.pixels() * 320
    wino_flops = 16 * 2.0 * (64 // 2) * (64 // 2) * 320 * 320  # 16 plane GEMMs over 32x32 tiles
    conv_tflops = wino_flops / (conv_ms * 1e-3) / 1e12
    gemm_tflops = wl.flops / (gemm_ms * 1e-3) / 1e12
    gn_gbps = 8.0 * elems / (gn_ms * 1e-3) / 1e9

    out = {
        "metric": METRIC, "value": round(ms, 5), "unit": "ms", "higher_is_better": False,
        "ms_per_step": round(ms, 5), "dtype": "f32",
        "config": {"workload": "conv3x3 64x64x320->320 (Winograd F(2x2,3x3)) + GroupNorm(32)+SiLU (f32, batch 1)",
                   "input": [1, 64, 64, 320], "weight": [320, 3, 3, 320], "groups": 32, "eps": 1e-5},
        "roofline": {"bound": "mfma", "kernel": "Winograd conv3x3 (input transform, 16 batched gemm_f32_kernel "
                                                "plane GEMMs, output transform)",
                     "achieved": round(conv_tflops, 3), "peak": PEAK_F32_MFMA_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(conv_tflops / PEAK_F32_MFMA_TFLOPS, 4), "traffic": None,
                     "work_per_launch": f"{wino_flops / 1e9:.3f} GFLOP of plane GEMMs per conv (direct conv: "
                                        f"{wl.flops / 1e9:.3f} GFLOP, {wl.flops / (conv_ms * 1e-3) / 1e12:.1f} "
                                        "TFLOP/s equivalent)", "avg_launch_ms": round(conv_ms, 5)},
        "components": {"conv_winograd_ms": round(conv_ms, 5), "conv_implicit_gemm_ms": round(gemm_ms, 5),
                       "conv_implicit_gemm_mfma_util": round(gemm_tflops / PEAK_F32_MFMA_TFLOPS, 4),
                       "groupnorm_silu_ms": round(gn_ms, 5), "groupnorm_gbps_8B_per_elem": round(gn_gbps, 1)},
    }
    ctx.close()
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline("conv3x3_gn_silu", note=" (C++ restatement of the CPU engine: "
                                           "Winograd F(2x2,3x3) conv + GroupNorm, OpenMP)")
    return out


def _components(ctx, steps):
    """Standalone per-kernel figures of the metric: the 3x3 conv's f32 MFMA
    utilisation (64x64x320 -> 320, implicit GEMM), the same conv as Winograd
    F(2x2,3x3), and GroupNorm+SiLU HBM GB/s at the VAE's 512x512x128 map
    (8 B/element: one read, one write)."""
    from moebius_cpu_amd import engine as E
    from moebius_cpu_amd import synthetic as S
    from moebius_cpu_amd import workloads as W

    wl = W.conv3x3_gn_silu()
    x = E.Tensor.from_numpy(ctx, wl.x)
    conv = E.Conv3x3.same(ctx, 320, 320, E.Param(ctx, wl.w), wl.b)
    y = E.Tensor(ctx, 1, 64, 64, 320)
    conv.forward(x, y)
    conv_ms = time_region(ctx, lambda: conv.forward(x, y), steps)
    wconv = E.Conv3x3.same(ctx, 320, 320, E.Param(ctx, wl.w), wl.b, winograd=True)
    wconv.forward(x, y)
    wino_ms = time_region(ctx, lambda: wconv.forward(x, y), steps)
    xg = E.Tensor.from_numpy(ctx, S.normal(77, (1, 512, 512, 128)))
    gn = E.GroupNorm(ctx, 32, 1e-6, S.normal(78, (128,), 0.1, 1.0), S.normal(79, (128,), 0.1))
    z = E.Tensor(ctx, 1, 512, 512, 128)
    gn.forward(xg, None, True, z)
    gn_ms = time_region(ctx, lambda: gn.forward(xg, None, True, z), steps)
    conv_tf = wl.flops / (conv_ms * 1e-3) / 1e12
    gn_gbps = 8.0 * 512 * 512 * 128 / (gn_ms * 1e-3) / 1e9
    return {"conv3x3_64x64x320_ms": round(conv_ms, 5),
            "conv3x3_mfma_util": round(conv_tf / PEAK_F32_MFMA_TFLOPS, 4),
            "conv3x3_64x64x320_winograd_ms": round(wino_ms, 5),
            "conv3x3_winograd_direct_equivalent_tflops": round(wl.flops / (wino_ms * 1e-3) / 1e12, 1),
            "groupnorm_silu_512x512x128_ms": round(gn_ms, 5),
            "groupnorm_silu_gbps_8B_per_elem": round(gn_gbps, 1),
            "groupnorm_hbm_frac": round(gn_gbps / PEAK_HBM_GBPS, 4)}


# HBM bytes per launch of the dominant kernel (below), from rocprofv3 --pmc FETCH_SIZE and
# WRITE_SIZE over this script's own default run (two UNet steps plus the standalone
# timing loop), each scaled by the counter's reading for a plain 256 MiB device copy
# (FETCH_SIZE reads half the copied bytes, WRITE_SIZE all of them), averaged over the
# standalone loop's 51 launches: 13.28 MiB fetched + 10.00 MiB written per launch.
DOMINANT_TRAFFIC_BYTES = int((13.28 + 10.00) * 1048576)


def _dominant_gemm(ctx, steps, fast=False):
    """The step's most frequent GEMM, timed on its own with events: the 1x1 conv of
    a [2,64,64,320] map to 320 channels with bias (gemm_f32_kernel, 32x64 tiles on
    v_mfma_f32_16x16x4f32, 1280 workgroups), i.e. M = 8192, N = 320, K = 320."""
    from moebius_cpu_amd import engine as E
    from moebius_cpu_amd import synthetic as S

    x = E.Tensor.from_numpy(ctx, S.normal(81, (2, 64, 64, 320)))
    conv = E.Conv1x1(ctx, 320, 320, E.Param(ctx, S.normal(82, (320, 320), 0.05), f16=fast), S.normal(83, (320,), 0.02))
    y = E.Tensor(ctx)
    conv.forward(x, y)
    us = time_region(ctx, lambda: conv.forward(x, y), steps) * 1e3
    flops = 2.0 * 8192 * 320 * 320
    tf = flops / (us * 1e-6) / 1e12
    if fast:
        # f16 products at 16x the f32 rate leave this shape bound by its operand
        # traffic: x read and y written in f32, the weight read in f16.
        nbytes = 8192 * 320 * 4 * 2 + 320 * 320 * 2 + 320 * 4
        gbps = nbytes / (us * 1e-6) / 1e9
        return {"bound": "hbm", "kernel": "gemm_h16_kernel (f16 MFMA, f32 accumulate; 1x1 conv [2,64,64,320] -> "
                                          "320, M=8192 N=320 K=320: the step's most frequent GEMM)",
                "achieved": round(gbps, 1), "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                "frac": round(gbps / PEAK_HBM_GBPS, 4), "traffic": None,
                "work_per_launch": f"algorithmic bytes {nbytes}; {flops / 1e9:.3f} GFLOP "
                                   f"({tf:.1f} TFLOP/s = {tf / PEAK_F16_MFMA_TFLOPS:.3f} of f16 MFMA peak)",
                "avg_launch_us": round(us, 2)}
    return {"bound": "mfma", "kernel": "gemm_f32_kernel<32,64,dense> (1x1 conv [2,64,64,320] -> 320, "
                                       "M=8192 N=320 K=320: the step's most frequent GEMM)",
            "achieved": round(tf, 2), "peak": PEAK_F32_MFMA_TFLOPS, "unit": "TFLOP/s",
            "frac": round(tf / PEAK_F32_MFMA_TFLOPS, 4), "traffic": DOMINANT_TRAFFIC_BYTES,
            "work_per_launch": f"{flops / 1e9:.3f} GFLOP; algorithmic bytes {(8192 * 320 * 2 + 320 * 320) * 4}",
            "avg_launch_us": round(us, 2)}


def bench_unet(args):
    """One full 512^2 denoise step: 64x64x9 latent stack, CFG batch 2, f32 Exact."""
    from moebius_cpu_amd import engine as E
    from moebius_cpu_amd import unet_params as U
    from moebius_cpu_amd.unet import UNet

    cfg = not args.cond_only
    b = 2 if cfg else 1
    log("generating random-init weights")
    params = U.random_unet(seed=4000)
    inp = U.unet_input(seed=5000)
    ctx = E.Context(0)
    if args.fast:
        ctx.set_precision(True)
    net = UNet(ctx, params, f16_gemm=args.f16_weights or args.fast)
    x = E.DeviceArray.from_numpy(ctx, inp.x)
    eps = E.DeviceArray(ctx, (b, 64, 64, 4))
    step = lambda: net.forward(x, inp.timestep, cfg, eps)  # noqa: E731
    log("warm-up")
    for _ in range(max(args.warmup, 1)):
        step()
    ctx.synchronize()
    log("timed steps")
    ms = time_region(ctx, step, args.steps)
    flops = U.step_flops(b, winograd=True)  # the upsample convs run as Winograd F(2x2,3x3)
    direct = U.step_flops(b)["total"]
    achieved = flops["total"] / (ms * 1e-3) / 1e12
    wbytes, pbytes = net.memory()
    peak = PEAK_F16_MFMA_TFLOPS if args.fast else PEAK_F32_MFMA_TFLOPS
    if args.fast:
        arith = "FAST: f16-stored GEMM weights, GEMM operands rounded to f16 on f16 MFMA with f32 accumulate"
    else:
        arith = f"{'f16-stored GEMM weights, ' if args.f16_weights else ''}f32 arithmetic"
    out = {
        "metric": METRIC, "value": round(ms, 4), "unit": "ms", "higher_is_better": False,
        "ms_per_step": round(ms, 4), "dtype": "f16 (f32 accumulate)" if args.fast else "f32",
        "config": {"workload": "Moebius UNet denoise step, 512x512 image (64x64x9 latent stack), "
                               f"{'CFG batch 2' if cfg else 'cond-only batch 1'}, {arith}",
                   "latent": [1, 64, 64, 9], "batch": b, "timestep": inp.timestep,
                   "params_M": round(U.param_count() / 1e6, 1), "weight_bytes": wbytes, "pool_bytes": pbytes},
        "step_roofline": {"bound": "mfma", "kernel": "whole step (all kernels, one stream)",
                          "achieved": round(achieved, 2), "peak": peak, "unit": "TFLOP/s",
                          "frac": round(achieved / peak, 4),
                          "work": f"{flops['total'] / 1e9:.1f} GFLOP per step (matrix-core work as executed: "
                                  f"the upsample convs as Winograd GEMMs; {direct / 1e9:.1f} GFLOP with direct convs)",
                          "direct_equivalent_tflops": round(direct / (ms * 1e-3) / 1e12, 2)},
    }
    log("dominant kernel and component kernels")
    out["roofline"] = _dominant_gemm(ctx, 50, fast=args.fast)
    ctx.set_precision(False)
    out["components"] = _components(ctx, 20)
    del net, x, eps
    ctx.close()
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline("unet_step", () if cfg else ("--cond-only",),
                                           note=" (C++ restatement of the CPU engine's UNet, OpenMP)")
    return out


def _vae_run(args, which):
    """VAE decode ([1,64,64,4] latent -> [1,512,512,3]) or encode (2 x 512x512 images), f32."""
    from moebius_cpu_amd import engine as E
    from moebius_cpu_amd import synthetic as S
    from moebius_cpu_amd import vae_params as V
    from moebius_cpu_amd.vae import Vae

    log("generating random-init VAE weights")
    params = V.random_vae()
    ctx = E.Context(0)
    vae = Vae(ctx, params, f16_gemm=args.f16_weights)
    if which == "decode":
        lat = E.DeviceArray.from_numpy(ctx, S.normal(24, (1, 64, 64, 4)))
        out = E.DeviceArray(ctx, (1, 512, 512, 3))
        step = lambda: vae.decode(lat, out)  # noqa: E731
        flops, direct = V.decode_flops(64, 64, winograd=True), V.decode_flops(64, 64)
        wl = "Moebius VAE decode, [1,64,64,4] latent -> [1,512,512,3] image"
    else:
        img = E.DeviceArray.from_numpy(ctx, V.vae_images(seed=25, b=2, h=512, w=512))
        noise = E.DeviceArray.from_numpy(ctx, S.normal(26, (2, 64, 64, 4)))
        z = E.DeviceArray(ctx, (2, 64, 64, 4))
        step = lambda: vae.encode(img, noise, z)  # noqa: E731
        flops, direct = V.encode_flops(2, 512, 512, winograd=True), V.encode_flops(2, 512, 512)
        wl = "Moebius VAE encode, 2 x [512,512,3] images (image + masked image) -> [2,64,64,4]"
    for _ in range(max(args.warmup, 1)):
        step()
    ctx.synchronize()
    ms = time_region(ctx, step, args.steps)
    achieved = flops / (ms * 1e-3) / 1e12
    wbytes, pbytes = vae.memory()
    res = {
        "metric": METRIC, "value": round(ms, 4), "unit": "ms", "higher_is_better": False,
        "ms_per_step": round(ms, 4), "dtype": "f32",
        "config": {"workload": wl + (", f16-stored weights" if args.f16_weights else "") + ", f32 arithmetic",
                   "params_M": round(V.param_count() / 1e6, 1), "weight_bytes": wbytes, "pool_bytes": pbytes},
        "roofline": {"bound": "mfma", "kernel": "whole pass (all kernels, one stream)",
                     "achieved": round(achieved, 2), "peak": PEAK_F32_MFMA_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / PEAK_F32_MFMA_TFLOPS, 4), "traffic": None,
                     "work_per_launch": f"{flops / 1e9:.1f} GFLOP per pass (stride-1 3x3 convs as Winograd GEMMs; "
                                        f"{direct / 1e9:.1f} GFLOP with direct convs)", "avg_launch_ms": round(ms, 4),
                     "direct_equivalent_tflops": round(direct / (ms * 1e-3) / 1e12, 2)},
    }
    vae.close()
    ctx.close()
    if not args.no_cpu:
        res["cpu_baseline"] = cpu_baseline(f"vae_{which}", note=" (C++ restatement of the CPU engine's VAE, OpenMP)")
    return res


WORKLOADS = {"unet_step": bench_unet, "conv3x3_gn_silu": bench_conv_gn,
             "vae_decode": lambda a: _vae_run(a, "decode"), "vae_encode": lambda a: _vae_run(a, "encode")}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="unet_step", choices=sorted(WORKLOADS))
    ap.add_argument("--cond-only", action="store_true", help="UNet: batch 1 (no CFG)")
    ap.add_argument("--f16-weights", action="store_true", help="UNet / VAE: f16-stored GEMM weights")
    ap.add_argument("--fast", action="store_true",
                    help="UNet: FAST precision (f16-stored weights, f16 MFMA with f32 accumulate)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--calibration-copy", action="store_true",
                    help="end with one 256 MiB device-to-device copy (the known-size reference that "
                         "scales rocprofv3 FETCH_SIZE / WRITE_SIZE readings)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (got --gpus {args.gpus}); the multi-GPU design is described in "
              "DESIGN.md and no multi-GPU figure is produced.", file=sys.stderr)
        sys.exit(2)
    res = WORKLOADS[args.workload](args)
    if args.calibration_copy:
        from moebius_cpu_amd import engine as E

        ctx = E.Context(0)
        n = 64 << 20  # floats: 256 MiB
        src, dst = E.DeviceArray(ctx, (n,)), E.DeviceArray(ctx, (n,))
        E.check(E.lib().mh_memcpy_d2d(ctx.h, dst.ptr, src.ptr, 4 * n))
        ctx.synchronize()
        del src, dst
        ctx.close()
    line = {"metric": res.pop("metric"), "value": res.pop("value"), "unit": res.pop("unit"), "n_gpus": 1,
            "steps": args.steps, "warmup": args.warmup, "ms_per_step": res.pop("ms_per_step"),
            "higher_is_better": res.pop("higher_is_better"), "scaling": "weak", "vs_baseline": None,
            "dtype": res.pop("dtype"), "data": "synthetic (seeded splitmix64/Box-Muller; random-init weights)",
            **res}
    print(json.dumps(line))


if __name__ == "__main__":
    main()
