"""Benchmark of the MI355X conv/norm hot path.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME] [--no-cpu] [--no-configs]

Prints ONE JSON line. A step is one pass of the workload over synthetic
seeded inputs already resident in HBM; the timed region is K steps between two
HIP events on the library's stream (synchronised on both sides). The headline
is one 512x512 UNet denoise step (CFG batch 2, f32). Also reported: the
dominant kernel's roofline (algorithmic work / its average duration, timed the
same way), and, under "configs", every benchmark configuration:

  cfg1  3x3 conv 64x64x320 -> 320 + GroupNorm(32)+SiLU
  cfg2  kernel sweep at (64,320) (32,640) (16,1280) (8,1280): 1x1 C->C (f32 and
        f16-stored weights), depthwise 3x3, GroupNorm(32)+SiLU, bias + residual;
        plus GroupNorm+add+SiLU at 2x64x64x320
  cfg3  ResNet block 32x32, 320 -> 640 with a time embedding
  cfg4  the UNet step in EXACT (batch 2 and 1) and FAST (f16 MFMA; batch 2 and 1)
  cfg5  VAE encode [1,512,512,3] and decode [1,64,64,4] -> [1,512,512,3]

and "inpaint": one whole inpainting call through the moebius_inpaint C API
(Exact and Fast presets, 1024x768 RGB image, 400x300 mask: an 800 px window
resampled to 512 and back), wall time per call with its stage split,

each with its time, its rate and roofline fraction, and the CPU oracle on the
same inputs, timed in the same run (a child process on the host cores).
One GPU only: --gpus above 1 exits with a message.
"""
from __future__ import annotations

import argparse
import json
import os
import sys

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
    """Average ms of fn() over `steps` back-to-back calls between two events on the stream."""
    ctx.synchronize()
    e0, e1 = ctx.event(), ctx.event()
    e0.record()
    for _ in range(steps):
        fn()
    e1.record()
    ms = e0.elapsed_ms(e1)
    ctx.synchronize()
    return ms / steps


def warm_time(ctx, fn, steps, warmup=1):
    for _ in range(max(warmup, 1)):
        fn()
    return time_region(ctx, fn, steps)


def cpu_threads():
    return int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count() or 1)


def r(v, nd=5):
    return None if v is None else round(float(v), nd)


def mfma_entry(ms, flops, peak=PEAK_F32_MFMA_TFLOPS):
    tf = flops / (ms * 1e-3) / 1e12
    return {"ms": r(ms), "tflops": r(tf, 2), "bound": "mfma", "peak_tflops": peak, "frac": r(tf / peak, 4),
            "gflop": r(flops / 1e9, 4)}


def hbm_entry(ms, nbytes):
    gbps = nbytes / (ms * 1e-3) / 1e9
    return {"ms": r(ms), "gbps": r(gbps, 1), "bound": "hbm", "peak_gbps": PEAK_HBM_GBPS,
            "frac": r(gbps / PEAK_HBM_GBPS, 4), "bytes": int(nbytes)}


def cpu_run(workload, extra=(), timeout=900):
    """Runs the CPU oracle on a workload in a child process that never touches the
    GPU (oracle/baseline.py); returns its JSON, or an error record."""
    import subprocess

    cmd = [sys.executable, "-X", "faulthandler", "-m", "oracle.baseline", "--workload", workload,
           "--threads", str(cpu_threads()), *extra]
    log("CPU baseline: " + " ".join(cmd[1:]))
    try:
        p = subprocess.run(cmd, cwd=ROOT, capture_output=True, text=True, timeout=timeout)
    except subprocess.TimeoutExpired:
        return {"error": "timed out"}
    if p.returncode != 0:
        log(p.stderr[-2000:])
        return {"error": f"baseline process exited with {p.returncode}"}
    return json.loads(p.stdout.strip().splitlines()[-1])


def cpu_record(ms, cores, sample, model=None):
    rec = {"value": r(ms, 3), "unit": "ms", "cores": cores, "kind": "port", "sample": sample}
    if model:
        rec["cpu_model"] = model
    return rec


# ---------------------------------------------------------------- cfg1

def cfg1_conv_gn(ctx, steps):
    """conv3x3 64x64x320 -> 320 + GroupNorm(32, eps 1e-5) + SiLU, f32. The conv runs
    as Winograd F(2x2,3x3) (the CPU engine's algorithm for stride-1 convs); the
    implicit-GEMM conv is timed beside it for the f32-MFMA utilisation."""
    from moebius_cpu_amd import engine as E
    from moebius_cpu_amd import workloads as W

    wl = W.conv3x3_gn_silu()
    x = E.Tensor.from_numpy(ctx, wl.x)
    w = E.Param(ctx, wl.w)
    conv_w = E.Conv3x3.same(ctx, 320, 320, w, wl.b, winograd=True)
    conv_g = E.Conv3x3.same(ctx, 320, 320, w, wl.b)
    gn = E.GroupNorm(ctx, wl.groups, wl.eps, wl.gamma, wl.beta)
    y, z = E.Tensor(ctx), E.Tensor(ctx)

    def step():
        conv_w.forward(x, y)
        gn.forward(y, None, True, z)

    total = warm_time(ctx, step, steps)
    wino = warm_time(ctx, lambda: conv_w.forward(x, y), steps)
    gemm = warm_time(ctx, lambda: conv_g.forward(x, y), steps)
    gn_ms = warm_time(ctx, lambda: gn.forward(y, None, True, z), steps)
    elems = 64 * 64 * 320
    wino_flops = 16 * 2.0 * 32 * 32 * 320 * 320  # 16 plane GEMMs over 32x32 tiles
    out = {"workload": "conv3x3 [1,64,64,320] -> 320 (stride 1, pad 1) + GroupNorm(32, eps 1e-5) + SiLU, f32",
           "ms": r(total),
           "conv_winograd": {**mfma_entry(wino, wino_flops),
                             "direct_equivalent_tflops": r(wl.flops / (wino * 1e-3) / 1e12, 2)},
           "conv_implicit_gemm": mfma_entry(gemm, wl.flops),
           "groupnorm_silu": {**hbm_entry(gn_ms, 8.0 * elems), "convention": "8 B/elem (read + write)"}}
    return out


# ---------------------------------------------------------------- cfg2

def cfg2_sweep(ctx, steps):
    """The kernel sweep at the four (S, C) points, plus GroupNorm+add+SiLU at 2x64x64x320."""
    from moebius_cpu_amd import engine as E
    from moebius_cpu_amd import synthetic as S
    from moebius_cpu_amd import workloads as W

    D = lambda a: E.DeviceArray.from_numpy(ctx, np.ascontiguousarray(a, np.float32))  # noqa: E731
    points = []
    for s, c in W.SWEEP:
        p = W.sweep_point(s, c)
        x = E.Tensor.from_numpy(ctx, p.x)
        res = E.Tensor.from_numpy(ctx, p.residual)
        out = E.Tensor(ctx)
        conv32 = E.Conv1x1(ctx, c, c, E.Param(ctx, p.w1), p.b1)
        conv16 = E.Conv1x1(ctx, c, c, E.Param(ctx, p.w1, f16=True), p.b1)
        dw_w, dw_b, bias = D(p.dw_w), D(p.dw_b), D(p.bias)
        gn = E.GroupNorm(ctx, 32, 1e-5, p.gamma, p.beta)
        flops = 2.0 * s * s * c * c
        elems = s * s * c
        e = {"S": s, "C": c}
        e["conv1x1_f32"] = mfma_entry(warm_time(ctx, lambda: conv32.forward(x, out), steps), flops)
        e["conv1x1_f16w"] = {**mfma_entry(warm_time(ctx, lambda: conv16.forward(x, out), steps), flops),
                             "note": "f16-stored weight widened to f32 in the tile loader; f32 MFMA"}
        e["depthwise"] = hbm_entry(warm_time(ctx, lambda: E.depthwise3x3(x, dw_w, dw_b, "none", out), steps),
                                   8.0 * elems + 40.0 * c)
        e["groupnorm_silu"] = hbm_entry(warm_time(ctx, lambda: gn.forward(x, None, True, out), steps), 8.0 * elems)
        e["bias_residual"] = hbm_entry(warm_time(ctx, lambda: E.bias_residual_add(x, bias, res, out), steps),
                                       12.0 * elems)
        points.append(e)
    # src/engine GroupNorm+add+SiLU at 2x64x64x320 (the CPU engine's kernel benchmark)
    xg = E.Tensor.from_numpy(ctx, S.normal(2501, (2, 64, 64, 320)))
    add = D(S.normal(2502, (2, 320), 0.5))
    gn = E.GroupNorm(ctx, 32, 1e-5, S.normal(2503, (320,), 0.1, 1.0), S.normal(2504, (320,), 0.1))
    out = E.Tensor(ctx)
    gna = hbm_entry(warm_time(ctx, lambda: gn.forward(xg, add, True, out), steps), 8.0 * 2 * 64 * 64 * 320)
    return {"workload": "kernel sweep, f32 activations; depthwise, GroupNorm and bias+residual have no "
                        "f16-stored operand (the converter keeps them f32), so only the 1x1 has an f16w variant",
            "points": points, "groupnorm_add_silu_2x64x64x320": gna}


# ---------------------------------------------------------------- cfg3

def cfg3_resnet(ctx, steps):
    from moebius_cpu_amd import workloads as W

    wl = W.resnet_block()
    blk = W.ResnetBlockGpu(ctx, wl)
    ms = warm_time(ctx, blk.forward, steps)
    # executed matrix work: the two 3x3 convs as 16 Winograd plane GEMMs over 16x16 tiles
    p = 32 * 32
    exe = 8.0 * p * (320 * 640 + 640 * 640) + 2.0 * p * 320 * 640 + 2.0 * 1280 * 640
    return {"workload": "ResNet block [1,32,32,320] -> 640 with time embedding [1280] (Linear 1280->640 on "
                        "SiLU(temb)), GN(32, eps 1e-5)+SiLU before each 3x3 conv (applied inside the Winograd "
                        "input transform), 1x1 skip, residual add; f32",
            **mfma_entry(ms, exe), "direct_gflop": r(wl.flops / 1e9, 3),
            "direct_equivalent_tflops": r(wl.flops / (ms * 1e-3) / 1e12, 2)}


# ---------------------------------------------------------------- cfg4

# HBM bytes per launch of the dominant kernel come from the committed rocprofv3 --pmc summary
# (FETCH_SIZE and WRITE_SIZE passes over this script's own run, each scaled by the counter's
# reading for a plain device copy), which names the GEMM configuration it measured on a line
#   traffic_config: <config> | traffic_bytes_per_launch: <bytes>
# The figure is used only while the live configuration of that GEMM is the same one.
TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "unet_step_traffic_pmc.md")


def _profiled_traffic(config):
    """(bytes, note) from the committed PMC summary for this GEMM configuration."""
    import re

    try:
        with open(TRAFFIC_PROFILE, encoding="utf-8") as f:
            text = f.read()
    except OSError:
        return None, "no committed PMC summary"
    m = re.search(r"^traffic_config: (.+?) \| traffic_bytes_per_launch: (\d+)\s*$", text, re.M)
    if not m:
        return None, "the PMC summary names no traffic line"
    if m.group(1).strip() != config:
        return None, f"the PMC summary measured '{m.group(1).strip()}', not the live '{config}'"
    return int(m.group(2)), "from " + os.path.relpath(TRAFFIC_PROFILE, ROOT)


def _gemm_config(ctx, fn):
    """The kernel configuration key (mh_context_gemm_times) of the GEMM fn launches."""
    ctx.set_tuning("gemm_time", 1)
    try:
        fn()
        recs = ctx.gemm_times()
    finally:
        ctx.set_tuning("gemm_time", None)
    return recs[0]["config"] if recs else None


def _in_step_gemms(ctx, step, steps, peak, config=None, overhead_us=0.0):
    """Every GEMM launch of `steps` denoise steps timed with events around it, grouped
    by kernel configuration: the configuration with the most step time (and the
    standalone dominant kernel's configuration, when given) with their in-step
    launch time and rate, and the GEMMs' total per step. overhead_us: what the
    events add to one launch (the standalone GEMM's evented minus plain launch
    time), taken off each launch for the `_net` figures."""
    ctx.set_tuning("gemm_time", 1)
    try:
        for _ in range(steps):
            step()
        recs = ctx.gemm_times()
    finally:
        ctx.set_tuning("gemm_time", None)

    def entry(rec):
        us = rec["us"] / rec["launches"]
        tf = rec["flops"] / (rec["us"] * 1e-6) / 1e12
        net = max(us - overhead_us, 1e-3)
        tf_net = rec["flops"] / rec["launches"] / (net * 1e-6) / 1e12
        return {"config": rec["config"], "launches_per_step": rec["launches"] / steps,
                "us_per_step": r(rec["us"] / steps, 1), "avg_launch_us": r(us, 2), "achieved": r(tf, 2),
                "unit": "TFLOP/s", "frac": r(tf / peak, 4), "avg_launch_us_net": r(net, 2),
                "achieved_net": r(tf_net, 2), "frac_net": r(tf_net / peak, 4)}

    recs.sort(key=lambda e: -e["us"])
    out = {"method": "HIP events recorded before and after every GEMM launch (split-K reduce included) over "
                     f"{steps} steps run after the timed ones; each launch's time includes its event overhead",
           "event_overhead_us_per_launch": r(overhead_us, 2),
           "gemm_us_per_step": r(sum(e["us"] for e in recs) / steps, 1),
           "gemm_launches_per_step": sum(e["launches"] for e in recs) / steps,
           "most_time": entry(recs[0]) if recs else None}
    same = [e for e in recs if e["config"] == config]
    if same:
        out["dominant_config_in_step"] = entry(same[0])
    return out


def _dominant_gemm(ctx, steps, fast=False):
    """The step's most frequent GEMM, timed on its own with events: the 1x1 conv of
    a [2,64,64,320] map to 320 channels with bias, M = 8192, N = 320, K = 320.
    Timed after `steps` warm-up launches (about 4 ms at 200): a freshly created
    operand set timed after a single launch reads 10-15% slow while clocks and
    caches settle, which no launch inside a denoise step sees."""
    from moebius_cpu_amd import engine as E
    from moebius_cpu_amd import synthetic as S

    x = E.Tensor.from_numpy(ctx, S.normal(81, (2, 64, 64, 320)))
    conv = E.Conv1x1(ctx, 320, 320, E.Param(ctx, S.normal(82, (320, 320), 0.05), f16=fast), S.normal(83, (320,), 0.02))
    y = E.Tensor(ctx)
    us = warm_time(ctx, lambda: conv.forward(x, y), steps, warmup=steps) * 1e3
    config = _gemm_config(ctx, lambda: conv.forward(x, y))
    # the same launches with an event before and after each (the in-step census's method)
    ctx.set_tuning("gemm_time", 1)
    try:
        for _ in range(steps):
            conv.forward(x, y)
        rec = ctx.gemm_times()[0]
    finally:
        ctx.set_tuning("gemm_time", None)
    event_us = rec["us"] / rec["launches"]
    flops = 2.0 * 8192 * 320 * 320
    tf = flops / (us * 1e-6) / 1e12
    if fast:
        nbytes = 8192 * 320 * 4 * 2 + 320 * 320 * 2 + 320 * 4
        gbps = nbytes / (us * 1e-6) / 1e9
        return {"bound": "hbm", "kernel": "gemm_h16_kernel (f16 MFMA, f32 accumulate; 1x1 conv [2,64,64,320] -> "
                                          "320, M=8192 N=320 K=320: the step's most frequent GEMM)",
                "achieved": round(gbps, 1), "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                "frac": round(gbps / PEAK_HBM_GBPS, 4), "traffic": None,
                "work_per_launch": f"algorithmic bytes {nbytes}; {flops / 1e9:.3f} GFLOP "
                                   f"({tf:.1f} TFLOP/s = {tf / PEAK_F16_MFMA_TFLOPS:.3f} of f16 MFMA peak)",
                "avg_launch_us": round(us, 2), "config": config, "evented_launch_us": round(event_us, 2)}
    traffic, note = _profiled_traffic(config)
    return {"bound": "mfma", "kernel": f"gemm_f32_kernel, {config} (1x1 conv [2,64,64,320] -> 320, "
                                       "M=8192 N=320 K=320: the step's most frequent GEMM), timed standalone",
            "achieved": round(tf, 2), "peak": PEAK_F32_MFMA_TFLOPS, "unit": "TFLOP/s",
            "frac": round(tf / PEAK_F32_MFMA_TFLOPS, 4), "traffic": traffic, "traffic_source": note,
            "work_per_launch": f"{flops / 1e9:.3f} GFLOP; algorithmic bytes {(8192 * 320 * 2 + 320 * 320) * 4}",
            "avg_launch_us": round(us, 2), "config": config, "evented_launch_us": round(event_us, 2)}


def _components(ctx, steps):
    """Per-kernel figures of the metric: the 3x3 conv's f32 MFMA utilisation
    (64x64x320 -> 320, implicit GEMM), the same conv as Winograd F(2x2,3x3), and
    GroupNorm+SiLU HBM GB/s at the VAE's 512x512x128 map (8 B/element)."""
    from moebius_cpu_amd import engine as E
    from moebius_cpu_amd import synthetic as S
    from moebius_cpu_amd import workloads as W

    wl = W.conv3x3_gn_silu()
    x = E.Tensor.from_numpy(ctx, wl.x)
    y = E.Tensor(ctx, 1, 64, 64, 320)
    conv = E.Conv3x3.same(ctx, 320, 320, E.Param(ctx, wl.w), wl.b)
    conv_ms = warm_time(ctx, lambda: conv.forward(x, y), steps)
    wconv = E.Conv3x3.same(ctx, 320, 320, E.Param(ctx, wl.w), wl.b, winograd=True)
    wino_ms = warm_time(ctx, lambda: wconv.forward(x, y), steps)
    xg = E.Tensor.from_numpy(ctx, S.normal(77, (1, 512, 512, 128)))
    gn = E.GroupNorm(ctx, 32, 1e-6, S.normal(78, (128,), 0.1, 1.0), S.normal(79, (128,), 0.1))
    z = E.Tensor(ctx, 1, 512, 512, 128)
    gn_ms = warm_time(ctx, lambda: gn.forward(xg, None, True, z), steps)
    conv_tf = wl.flops / (conv_ms * 1e-3) / 1e12
    gn_gbps = 8.0 * 512 * 512 * 128 / (gn_ms * 1e-3) / 1e9
    return {"conv3x3_64x64x320_ms": round(conv_ms, 5),
            "conv3x3_mfma_util": round(conv_tf / PEAK_F32_MFMA_TFLOPS, 4),
            "conv3x3_64x64x320_winograd_ms": round(wino_ms, 5),
            "conv3x3_winograd_direct_equivalent_tflops": round(wl.flops / (wino_ms * 1e-3) / 1e12, 1),
            "groupnorm_silu_512x512x128_ms": round(gn_ms, 5),
            "groupnorm_silu_gbps_8B_per_elem": round(gn_gbps, 1),
            "groupnorm_hbm_frac": round(gn_gbps / PEAK_HBM_GBPS, 4)}


def _unet_step_entry(ctx, net, inp, cfg, steps, warmup, fast):
    from moebius_cpu_amd import engine as E
    from moebius_cpu_amd import unet_params as U

    b = 2 if cfg else 1
    x = E.DeviceArray.from_numpy(ctx, inp.x)
    eps = E.DeviceArray(ctx, (b, 64, 64, 4))
    step = lambda: net.forward(x, inp.timestep, cfg, eps)  # noqa: E731
    ms = warm_time(ctx, step, steps, warmup)
    flops = U.step_flops(b, winograd=True, cfg_shared=cfg)["total"]
    direct = U.step_flops(b)["total"]
    peak = PEAK_F16_MFMA_TFLOPS if fast else PEAK_F32_MFMA_TFLOPS
    tf = flops / (ms * 1e-3) / 1e12
    return ms, {"ms": r(ms, 4), "batch": b, "tflops_executed": r(tf, 2), "peak_tflops": peak, "frac": r(tf / peak, 4),
                "gflop_executed": r(flops / 1e9, 1), "gflop_direct": r(direct / 1e9, 1),
                "direct_equivalent_tflops": r(direct / (ms * 1e-3) / 1e12, 2)}


def bench_unet(args):
    """One full 512^2 denoise step: 64x64x9 latent stack, CFG batch 2, f32 Exact (the
    headline); with configs, also batch 1 and the FAST precision at batch 2 and 1."""
    from moebius_cpu_amd import engine as E
    from moebius_cpu_amd import unet_params as U
    from moebius_cpu_amd.unet import UNet

    cfg = not args.cond_only
    log("generating random-init weights")
    params = U.random_unet(seed=4000)
    inp = U.unet_input(seed=5000)
    ctx = E.Context(0)
    if args.fast:
        ctx.set_precision(True)
    net = UNet(ctx, params, f16_gemm=args.f16_weights or args.fast)
    log("warm-up and timed steps")
    ms, head = _unet_step_entry(ctx, net, inp, cfg, args.steps, args.warmup, args.fast)
    b = head["batch"]
    wbytes, pbytes = net.memory()
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
                          "achieved": head["tflops_executed"], "peak": head["peak_tflops"], "unit": "TFLOP/s",
                          "frac": head["frac"],
                          "work": f"{head['gflop_executed']} GFLOP per step (matrix-core work as executed: the "
                                  f"upsample convs as Winograd GEMMs; {head['gflop_direct']} GFLOP with direct convs)",
                          "direct_equivalent_tflops": head["direct_equivalent_tflops"]},
    }
    log("dominant kernel and component kernels")
    out["roofline"] = _dominant_gemm(ctx, 200, fast=args.fast)
    log("GEMM launches inside the step")
    xin = E.DeviceArray.from_numpy(ctx, inp.x)
    eps = E.DeviceArray(ctx, (b, 64, 64, 4))
    rl = out["roofline"]
    rl["in_step"] = _in_step_gemms(ctx, lambda: net.forward(xin, inp.timestep, cfg, eps), 3, head["peak_tflops"],
                                   rl.get("config"), max(0.0, rl["evented_launch_us"] - rl["avg_launch_us"]))
    ctx.set_precision(False)
    out["components"] = _components(ctx, 20)
    unet_entries = None
    if args.configs and not args.fast and not args.f16_weights and cfg:
        log("cfg4: EXACT batch 1, FAST batch 2 and 1")
        unet_entries = {"exact_b2": head}
        _, unet_entries["exact_b1"] = _unet_step_entry(ctx, net, inp, False, args.steps, args.warmup, False)
        del net
        ctx.set_precision(True)
        fnet = UNet(ctx, params, f16_gemm=True)
        _, unet_entries["fast_b2"] = _unet_step_entry(ctx, fnet, inp, True, args.steps, args.warmup, True)
        _, unet_entries["fast_b1"] = _unet_step_entry(ctx, fnet, inp, False, args.steps, args.warmup, True)
        fnet.close()
        del fnet
        ctx.set_precision(False)
    else:
        del net
    return out, ctx, unet_entries


# ---------------------------------------------------------------- cfg5

def cfg5_vae(ctx, steps, f16_weights=False, which=("decode", "encode_b1", "encode_b2")):
    """VAE encode of one [1,512,512,3] image in U[-1,1] (and the pipeline's batch of
    2) and decode of a [1,64,64,4] latent, f32 end to end."""
    from moebius_cpu_amd import engine as E
    from moebius_cpu_amd import synthetic as S
    from moebius_cpu_amd import vae_params as V
    from moebius_cpu_amd.vae import Vae

    log("cfg5: generating random-init VAE weights")
    vae = Vae(ctx, V.random_vae(), f16_gemm=f16_weights)
    lat = E.DeviceArray.from_numpy(ctx, S.normal(24, (1, 64, 64, 4)))
    img = E.DeviceArray(ctx, (1, 512, 512, 3))
    res = {"workload": "Moebius VAE (SDXL AutoencoderKL f8d4), Kaiming weights, GroupNorm gamma 1 + N(0,0.05), "
                       "beta N(0,0.05), f32" + (", f16-stored weights" if f16_weights else "")}
    if "decode" in which:
        dec_ms = warm_time(ctx, lambda: vae.decode(lat, img), steps)
        res["decode"] = {**mfma_entry(dec_ms, V.decode_flops(64, 64, winograd=True)),
                         "direct_gflop": r(V.decode_flops(64, 64) / 1e9, 1),
                         "direct_equivalent_tflops": r(V.decode_flops(64, 64) / (dec_ms * 1e-3) / 1e12, 2)}
    for b in (1, 2):
        if f"encode_b{b}" not in which:
            continue
        im = E.DeviceArray.from_numpy(ctx, V.vae_images(seed=25, b=b, h=512, w=512))
        nz = E.DeviceArray.from_numpy(ctx, S.normal(26, (b, 64, 64, 4)))
        z = E.DeviceArray(ctx, (b, 64, 64, 4))
        ms = warm_time(ctx, lambda: vae.encode(im, nz, z), steps)
        res[f"encode_b{b}"] = {**mfma_entry(ms, V.encode_flops(b, 512, 512, winograd=True)),
                               "direct_gflop": r(V.encode_flops(b, 512, 512) / 1e9, 1),
                               "direct_equivalent_tflops": r(V.encode_flops(b, 512, 512) / (ms * 1e-3) / 1e12, 2)}
    vae.close()
    return res


# ---------------------------------------------------------------- whole inpaint

def inpaint_bench(reps=3):
    """Wall time of whole moebius_inpaint calls (host in, host out, synchronous),
    after one warm-up call per preset, with the stage split the progress
    callback sees. Models: random-init UNet (f16-stored GEMM weights, the
    converter's default; f32 arithmetic) and VAE, loaded from safetensors files."""
    import ctypes
    import tempfile
    import time

    from moebius_cpu_amd import _lib
    from moebius_cpu_amd import unet_params as U
    from moebius_cpu_amd import vae_params as V
    from moebius_cpu_amd.weights_io import write_weights

    log("inpaint: writing the model files")
    tmp = tempfile.mkdtemp(prefix="moebius-bench-")
    gemm = sorted(s.name for s in U.unet_specs() if s.gemm)
    write_weights(os.path.join(tmp, "unet.safetensors"), U.random_unet(seed=4000), gemm, f16=True)
    write_weights(os.path.join(tmp, "vae.safetensors"), V.random_vae(), metadata={"scaling_factor": "0.13025"})
    L = _lib.lib()
    eng = ctypes.c_void_p()
    _lib.check(L.moebius_engine_create(tmp.encode(), 0, ctypes.byref(eng)))
    for f in os.listdir(tmp):
        os.remove(os.path.join(tmp, f))
    os.rmdir(tmp)
    h, w = 768, 1024
    yy, xx = np.mgrid[0:h, 0:w]
    img0 = np.stack([xx * 255 // (w - 1), yy * 255 // (h - 1), (xx + yy) % 256], -1).astype(np.uint8)
    mask = np.zeros((h, w), np.uint8)
    mask[234:534, 312:712] = 255
    marks = []

    def cb(_u, stage, done, total):
        marks.append((stage, done, total, time.perf_counter()))
        return 0
    fn = _lib.PROGRESS_FN(cb)
    res = {"workload": "moebius_inpaint, 1024x768 RGB, 400x300 mask (800 px window <-> 512), random-init models "
                       "from safetensors (UNet GEMM weights f16-stored, f32 arithmetic), feather paste; wall "
                       "time per call, host buffers in and out"}
    for name, preset in (("exact", 0), ("fast", 1)):
        p = _lib.MoebiusParams(preset=preset, steps=0, guidance=0.0, seed=1, paste=0, mask_dilate=0)
        runs = []
        for i in range(reps + 1):
            img = img0.copy()
            marks.clear()
            t0 = time.perf_counter()
            _lib.check(L.moebius_inpaint(eng, img.ctypes.data, w, h, w * 3, 3, mask.ctypes.data, w,
                                         ctypes.byref(p), fn, None, None))
            t1 = time.perf_counter()
            if i == 0:
                continue  # first call: the pools are allocated
            at = {(s, d): t for s, d, _, t in marks}
            n = marks[-3][2]  # denoise steps
            runs.append({"total": (t1 - t0) * 1e3, "prepare": (at[(0, 0)] - t0) * 1e3,
                         "encode": (at[(0, 1)] - at[(0, 0)]) * 1e3, "denoise": (at[(1, n)] - at[(0, 1)]) * 1e3,
                         "decode": (at[(2, 1)] - at[(2, 0)]) * 1e3, "finish": (t1 - at[(2, 1)]) * 1e3,
                         "steps": n})
        med = {k: float(np.median([r_[k] for r_ in runs])) for k in runs[0]}
        res[name] = {"ms": r(med["total"], 2), "denoise_steps": int(med["steps"]),
                     "stages_ms": {k: r(med[k], 2) for k in ("prepare", "encode", "denoise", "decode", "finish")},
                     "ms_per_denoise_step": r(med["denoise"] / med["steps"], 3), "runs": reps}
    L.moebius_engine_destroy(eng)
    res["reference_published"] = {"fast_s": [10.7, 11.9], "hardware": "i7-13620H, 10 threads",
                                  "source": "src/preset.rs:2-4 (per 512-px inpaint, from cool)"}
    return res


# ---------------------------------------------------------------- assembly

def attach_cpu(configs, cpu):
    """Puts the CPU oracle's time next to each GPU entry (same inputs, same run)."""
    if "error" in cpu:
        configs["cpu_error"] = cpu["error"]
        return
    cores, c, model = cpu["cores"], cpu["configs"], cpu.get("cpu_model")
    note = lambda s: {"cores": cores, "cpu_model": model, "kind": "port", "sample": s}  # noqa: E731
    if "cfg1" in configs and "cfg1" in c:
        configs["cfg1"]["cpu"] = {"ms": c["cfg1"]["total_ms"], "conv_ms": c["cfg1"]["conv_ms"],
                                  "groupnorm_silu_ms": c["cfg1"]["gn_silu_ms"],
                                  **note("conv3x3 (Winograd) + GroupNorm+SiLU, median after one warm-up")}
    if "cfg2" in configs and "sweep" in c:
        for e in configs["cfg2"]["points"]:
            k = f"{e['S']}x{e['C']}"
            for name in ("conv1x1_f32", "conv1x1_f16w", "depthwise", "groupnorm_silu", "bias_residual"):
                e[name]["cpu_ms"] = c["sweep"][k][name]
        configs["cfg2"]["groupnorm_add_silu_2x64x64x320"]["cpu_ms"] = c["gn_add_silu_2x64x64x320"]
        configs["cfg2"]["cpu"] = note("each kernel alone, median of >= 5 runs after one warm-up; the f16w 1x1 "
                                      "on the f16-rounded weights")
    if "cfg3" in configs and "resnet_block" in c:
        configs["cfg3"]["cpu"] = {"ms": c["resnet_block"], **note("the same block, median after one warm-up")}
    if "cfg4" in configs and "unet_b2" in c:
        u = configs["cfg4"]
        for key, ck in (("exact_b2", "unet_b2"), ("exact_b1", "unet_b1"), ("fast_b2", "unet_b2"),
                        ("fast_b1", "unet_b1")):
            u[key]["cpu_ms"] = c[ck]
        u["cpu"] = note("the same step, median after one warm-up; the CPU engine's Fast preset keeps f32 "
                        "arithmetic (f16-stored weights widened), so FAST is compared with the same CPU step")
    if "cfg5" in configs and "vae_decode" in c:
        v = configs["cfg5"]
        v["decode"]["cpu_ms"] = c["vae_decode"]
        v["encode_b1"]["cpu_ms"] = c["vae_encode_b1"]
        v["encode_b2"]["cpu_ms"] = c.get("vae_encode_b2")
        v["cpu"] = note("the same passes, median after one warm-up")
    if "inpaint" in configs and "unet_b2" in c and "vae_decode" in c:
        ip = configs["inpaint"]
        # The oracle is not run end to end (about 25 s per Exact call on 16 cores): its estimate is the
        # sum of the parts it ran in this same run. Exact: encode batch 2 + 19 CFG steps + decode; Fast:
        # encode batch 1 (the ROI encode of the image window is left out) + 3 CFG + 6 cond-only + decode.
        ip["exact"]["cpu_ms_estimate"] = r(c["vae_encode_b2"] + ip["exact"]["denoise_steps"] * c["unet_b2"]
                                           + c["vae_decode"], 1)
        nf = ip["fast"]["denoise_steps"]
        ip["fast"]["cpu_ms_estimate"] = r(c["vae_encode_b1"] + 3 * c["unet_b2"] + (nf - 3) * c["unet_b1"]
                                          + c["vae_decode"], 1)
        ip["cpu"] = note("estimate: the sum of the oracle's measured encode, steps and decode in this run")


def run_all(args):
    out, ctx, unet_entries = bench_unet(args)
    cpu_sets = []
    if args.configs and unet_entries is not None:
        configs = {}
        log("cfg1: conv3x3 + GroupNorm+SiLU 64x64x320")
        configs["cfg1"] = cfg1_conv_gn(ctx, args.steps)
        log("cfg2: kernel sweep")
        configs["cfg2"] = cfg2_sweep(ctx, args.steps)
        log("cfg3: ResNet block 32x32")
        configs["cfg3"] = cfg3_resnet(ctx, args.steps)
        configs["cfg4"] = {"workload": "UNet denoise step, 512x512 (64x64x9 latent stack); EXACT = f32 MFMA; "
                                       "FAST = f16-stored weights on f16 MFMA with f32 accumulate",
                           **unet_entries}
        configs["cfg5"] = cfg5_vae(ctx, max(3, args.steps // 4))
        configs["inpaint"] = inpaint_bench()
        out["configs"] = configs
        cpu_sets = ["configs"]
    ctx.close()
    if not args.no_cpu:
        if cpu_sets:
            cpu = cpu_run("configs")
            attach_cpu(out["configs"], cpu)
            if "error" not in cpu:
                key = "unet_b2" if not args.cond_only else "unet_b1"
                out["cpu_baseline"] = cpu_record(cpu["configs"][key], cpu["cores"],
                                                 "the same denoise step (same seeded weights and inputs), median "
                                                 "after one warm-up (C++ restatement of the CPU engine's UNet, "
                                                 "OpenMP)", cpu.get("cpu_model"))
        else:
            cpu = cpu_run("unet_step", () if not args.cond_only else ("--cond-only",))
            if "error" not in cpu:
                out["cpu_baseline"] = cpu_record(cpu["value"], cpu["cores"], cpu["sample"] +
                                                 " (C++ restatement of the CPU engine's UNet, OpenMP)",
                                                 cpu.get("cpu_model"))
    return out


def single(args):
    """One configuration alone (profiling runs): the headline-style line for it."""
    from moebius_cpu_amd import engine as E

    ctx = E.Context(0)
    w = args.workload
    if w == "conv3x3_gn_silu":
        res = cfg1_conv_gn(ctx, args.steps)
        ms = res["ms"]
    elif w == "sweep":
        res = cfg2_sweep(ctx, args.steps)
        ms = sum(e[k]["ms"] for e in res["points"] for k in ("conv1x1_f32", "depthwise", "groupnorm_silu",
                                                               "bias_residual"))
    elif w == "resnet_block":
        res = cfg3_resnet(ctx, args.steps)
        ms = res["ms"]
    elif w == "vae_decode":
        res = cfg5_vae(ctx, args.steps, args.f16_weights, which=("decode",))
        ms = res["decode"]["ms"]
    elif w == "vae_encode":
        res = cfg5_vae(ctx, args.steps, args.f16_weights, which=("encode_b1",))
        ms = res["encode_b1"]["ms"]
    elif w == "inpaint":
        res = inpaint_bench(max(1, args.steps))
        ms = res["exact"]["ms"]
    else:
        raise SystemExit(f"unknown workload {w}")
    ctx.close()
    return {"metric": METRIC, "value": ms, "unit": "ms", "higher_is_better": False, "ms_per_step": ms,
            "dtype": "f32", "config": {"workload": w}, "result": res}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="unet_step",
                    choices=["unet_step", "conv3x3_gn_silu", "sweep", "resnet_block", "vae_decode", "vae_encode",
                             "inpaint"])
    ap.add_argument("--cond-only", action="store_true", help="UNet: batch 1 (no CFG)")
    ap.add_argument("--f16-weights", action="store_true", help="UNet / VAE: f16-stored GEMM weights")
    ap.add_argument("--fast", action="store_true",
                    help="UNet: FAST precision (f16-stored weights, f16 MFMA with f32 accumulate)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-configs", dest="configs", action="store_false",
                    help="UNet: the headline only, without the per-configuration block")
    ap.add_argument("--calibration-copy", action="store_true",
                    help="end with one 256 MiB device-to-device copy (the known-size reference that "
                         "scales rocprofv3 FETCH_SIZE / WRITE_SIZE readings)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (got --gpus {args.gpus}); the multi-GPU design is described in "
              "DESIGN.md and no multi-GPU figure is produced.", file=sys.stderr)
        sys.exit(2)
    res = run_all(args) if args.workload == "unet_step" else single(args)
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
