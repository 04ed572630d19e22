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


def cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo), "unknown" where it is not readable."""
    try:
        with open("/proc/cpuinfo", encoding="utf-8", errors="replace") as f:
            for line in f:
                if line.lower().startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


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
    images = V.vae_images(seed=25, b=1, h=512, w=512)
    noise = S.normal(26, (1, 64, 64, 4))
    ms, runs = _time(lambda: vae.encode(images, noise), budget_s, 1, 3)
    return ms, runs, f"the same encode ([1,512,512,3]), median of {runs} runs after one warm-up"


def configs():
    """Every benchmark configuration on the oracle, on the inputs bench.py puts on the
    device: per-config medians (ms) after one warm-up, bounded to a few runs each
    (about half a minute of CPU work in all)."""
    from moebius_cpu_amd import synthetic as S
    from moebius_cpu_amd import unet_params as U
    from moebius_cpu_amd import vae_params as V
    from moebius_cpu_amd import workloads as W

    out = {}
    wl = W.conv3x3_gn_silu()
    y = oracle.conv3x3(wl.x, wl.w, wl.b)
    conv_ms, _ = _time(lambda: oracle.conv3x3(wl.x, wl.w, wl.b), 5.0, 5, 20)
    gn_ms, _ = _time(lambda: oracle.group_norm(y, wl.groups, wl.eps, wl.gamma, wl.beta, silu=True), 2.0, 5, 50)
    out["cfg1"] = {"conv_ms": round(conv_ms, 3), "gn_silu_ms": round(gn_ms, 3), "total_ms": round(conv_ms + gn_ms, 3)}

    sweep = {}
    for s, c in W.SWEEP:
        p = W.sweep_point(s, c)
        w16 = p.w1.astype(np.float16).astype(np.float32)
        res2d = p.residual.reshape(-1, c)
        x2d = p.x.reshape(-1, c)

        def bias_res():
            pre, _ = oracle.init_output(s * s, c, p.bias, res2d)
            oracle.add(pre, x2d)

        e = {}
        for name, fn in (("conv1x1_f32", lambda: oracle.conv1x1(p.x, p.w1, p.b1)),
                         ("conv1x1_f16w", lambda: oracle.conv1x1(p.x, w16, p.b1)),
                         ("depthwise", lambda: oracle.depthwise3x3(p.x, p.dw_w, p.dw_b, "none")),
                         ("groupnorm_silu", lambda: oracle.group_norm(p.x, 32, 1e-5, p.gamma, p.beta, silu=True)),
                         ("bias_residual", bias_res)):
            ms, _ = _time(fn, 1.0, 5, 200)
            e[name] = round(ms, 4)
        sweep[f"{s}x{c}"] = e
    out["sweep"] = sweep
    xg = S.normal(2501, (2, 64, 64, 320))
    add = S.normal(2502, (2, 320), 0.5)
    g, b = S.normal(2503, (320,), 0.1, 1.0), S.normal(2504, (320,), 0.1)
    ms, _ = _time(lambda: oracle.group_norm(xg, 32, 1e-5, g, b, add=add, silu=True), 1.0, 5, 200)
    out["gn_add_silu_2x64x64x320"] = round(ms, 4)

    rb = W.resnet_block()

    def resnet():
        sc, sh = oracle.group_norm_affine(rb.x, 32, rb.eps, rb.gn1_g, rb.gn1_b)
        h = oracle.conv3x3(rb.x, rb.w1, rb.b1, prologue=(sc, sh, True))
        tp = oracle.conv1x1(oracle.silu(rb.temb).reshape(1, 1, 1, -1), rb.lin_w, rb.lin_b).reshape(-1)
        sc2, sh2 = oracle.group_norm_affine(h, 32, rb.eps, rb.gn2_g, rb.gn2_b, add=tp)
        o = oracle.conv3x3(h, rb.w2, rb.b2, prologue=(sc2, sh2, True))
        return oracle.conv1x1(rb.x, rb.ws, rb.bs, residual=o)

    ms, _ = _time(resnet, 3.0, 5, 20)
    out["resnet_block"] = round(ms, 3)

    net = oracle.UNet(U.random_unet(seed=4000))
    inp = U.unet_input(seed=5000)
    for key, cfg in (("unet_b2", True), ("unet_b1", False)):
        ms, _ = _time(lambda: net.forward(inp.x, inp.timestep, cfg=cfg), 0.0, 2, 2)
        out[key] = round(ms, 3)
    del net

    vae = oracle.Vae(V.random_vae())
    lat = S.normal(24, (1, 64, 64, 4))
    ms, _ = _time(lambda: vae.decode(lat), 0.0, 1, 1)
    out["vae_decode"] = round(ms, 3)
    for bb in (1, 2):
        images = V.vae_images(seed=25, b=bb, h=512, w=512)
        noise = S.normal(26, (bb, 64, 64, 4))
        ms, _ = _time(lambda: vae.encode(images, noise), 0.0, 1, 1)
        out[f"vae_encode_b{bb}"] = round(ms, 3)
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--workload", default="unet_step",
                    choices=["unet_step", "conv3x3_gn_silu", "vae_decode", "vae_encode", "configs"])
    ap.add_argument("--threads", type=int, default=0)
    ap.add_argument("--cond-only", action="store_true")
    ap.add_argument("--budget-s", type=float, default=20.0)
    args = ap.parse_args()
    if args.threads > 0:
        oracle.set_threads(args.threads)
    if args.workload == "configs":
        print(json.dumps({"cores": oracle.threads(), "cpu_model": cpu_model(), "configs": configs()}))
        return
    if args.workload == "unet_step":
        ms, runs, sample = unet_step(not args.cond_only, args.budget_s)
    elif args.workload == "vae_decode":
        ms, runs, sample = vae_decode(args.budget_s)
    elif args.workload == "vae_encode":
        ms, runs, sample = vae_encode(args.budget_s)
    else:
        ms, runs, sample = conv3x3_gn_silu(args.budget_s)
    print(json.dumps({"value": round(ms, 3), "unit": "ms", "cores": oracle.threads(), "cpu_model": cpu_model(),
                      "runs": runs, "sample": sample}))


if __name__ == "__main__":
    main()
