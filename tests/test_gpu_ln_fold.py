"""LayerNorm folded into the 1x1 conv that reads it (mh_conv1x1_layer_norm, the
transformers' LayerNorm 1 -> q | k | v and LayerNorm 3 -> MixFFN inverted path,
src/unet/transformer.rs:100-126): against the oracle's layer_norm then conv1x1
(src/engine/norm.rs:151-173, conv.rs:38-55) and SiLU, in EXACT (f32 bar, and
on rows with a mean far from zero, where the fold's x . W' - mean . rowsum
cancels) and FAST precision (the f16 bar), f32 and f16-stored weights, ragged
row counts, and every tiling the planner can be forced to."""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from moebius_cpu_amd import engine as E
from tests.util import max_abs_rel

pytestmark = pytest.mark.gpu

F32_TOL = 1e-4
F32_TIGHT = 2e-5
F16_TOL = 2e-2


@pytest.fixture(scope="module")
def ctx():
    c = E.Context(0)
    yield c
    c.synchronize()
    c.close()


def run(ctx, x, gamma, beta, w, b, silu, f16=False, eps=1e-5):
    rows, ci = x.shape
    co = w.shape[0]
    param = E.Param(ctx, w, f16=f16)
    dev = {k: E.DeviceArray.from_numpy(ctx, v) for k, v in dict(x=x, g=gamma, be=beta, b=b).items()}
    out = E.DeviceArray(ctx, (rows, co))
    E.check(E.lib().mh_conv1x1_layer_norm(ctx.h, dev["x"].ptr, rows, ci, dev["g"].ptr, dev["be"].ptr, eps, param.ptr,
                                          param.dtype, co, dev["b"].ptr, 1 if silu else 0, out.ptr))
    return out.numpy()


def want(x, gamma, beta, w, b, silu, eps=1e-5):
    t = oracle.layer_norm(x, gamma, beta, eps)
    y = oracle.conv1x1(t.reshape(1, 1, *t.shape), w, b).reshape(x.shape[0], w.shape[0])
    return oracle.silu(y) if silu else y


def inputs(rows, ci, co, seed, offset=0.0):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((rows, ci)) * 1.5 + offset).astype(np.float32)
    gamma = (1 + 0.1 * rng.standard_normal(ci)).astype(np.float32)
    beta = (0.1 * rng.standard_normal(ci)).astype(np.float32)
    w = (rng.standard_normal((co, ci)) / np.sqrt(ci)).astype(np.float32)
    b = (0.05 * rng.standard_normal(co)).astype(np.float32)
    return x, gamma, beta, w, b


# the UNet's q | k | v (c -> c + c/4) and inverted (c -> 5c) shapes at 2x16x16,
# 2x8x8 and 1x4x4 latents, and a ragged one
SHAPES = [(512, 320, 400), (512, 320, 1600), (128, 640, 800), (128, 640, 3200), (16, 1280, 1600), (198, 200, 72)]


@pytest.mark.parametrize("rows,ci,co", SHAPES)
@pytest.mark.parametrize("silu", [False, True])
@pytest.mark.parametrize("f16", [False, True])
def test_exact_matches_layer_norm_then_conv1x1(ctx, rows, ci, co, silu, f16):
    x, g, be, w, b = inputs(rows, ci, co, rows + ci + co)
    if f16:
        w = w.astype(np.float16).astype(np.float32)
    print(f"ln fold exact {rows}x{ci}->{co} silu={silu} f16={f16}", flush=True)
    got = run(ctx, x, g, be, w, b, silu, f16)
    assert max_abs_rel(got, want(x, g, be, w, b, silu)) <= F32_TIGHT


@pytest.mark.parametrize("offset", [8.0, -30.0])
def test_exact_rows_far_from_zero_mean(ctx, offset):
    x, g, be, w, b = inputs(512, 320, 400, 91, offset)
    got = run(ctx, x, g, be, w, b, False)
    assert max_abs_rel(got, want(x, g, be, w, b, False)) <= F32_TOL


@pytest.mark.parametrize("rows,ci,co", SHAPES[:4])
@pytest.mark.parametrize("silu", [False, True])
def test_fast_matches_within_the_f16_bar(ctx, rows, ci, co, silu):
    x, g, be, w, b = inputs(rows, ci, co, 7 + rows + co)
    print(f"ln fold fast {rows}x{ci}->{co} silu={silu}", flush=True)
    ctx.set_precision(True)
    try:
        got = run(ctx, x, g, be, w, b, silu, f16=True)
    finally:
        ctx.set_precision(False)
    assert max_abs_rel(got, want(x, g, be, w.astype(np.float16).astype(np.float32), b, silu)) <= F16_TOL


@pytest.mark.parametrize("plan", ["32,32,1", "32,64,1", "64,64,1", "128,128,1", "64,64,3", "64,80,1,4,1,1,1",
                                  "64,80,1,4,1,1", "32,80,1,2,1,2,1", "160,64,1,2,2,1,1,16"])
def test_every_tiling(ctx, plan, tune):
    """A forced K split is ignored (the fold needs each workgroup to see whole rows)."""
    x, g, be, w, b = inputs(198, 320, 160, 5)
    tune("gemm_plan", plan)
    print(f"ln fold plan {plan}", flush=True)
    got = run(ctx, x, g, be, w, b, True)
    assert max_abs_rel(got, want(x, g, be, w, b, True)) <= F32_TIGHT
