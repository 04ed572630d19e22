"""LayerNorm folded into the 1x1 conv that reads it (mh_conv1x1_layer_norm, the
transformers' LayerNorm 1 -> q | k | v and LayerNorm 3 -> MixFFN inverted path,
src/unet/transformer.rs:100-126): against the oracle's layer_norm then conv1x1
(src/engine/norm.rs:151-173, conv.rs:38-55) and SiLU, in EXACT (f32 bar, and
on rows with a mean far from zero, where the fold's x . W' - mean . rowsum
cancels) and FAST precision (the f16 bar), f32 and f16-stored weights, ragged
row counts, and every tiling the planner can be forced to. Then the default
path of the transformers: the row statistics from partial sums the producer of
h writes (proj_in's epilogue, mh_conv1x1_row_partials; the cross-lambda
kernel, mh_cross_lambda_row_sums), folded by mh_conv1x1_layer_norm_stats."""
from __future__ import annotations

import ctypes

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


# ---- row statistics from the producer's partials (the transformers' default path)


def producer(ctx, x, w, b, f16=False):
    """mh_conv1x1_row_partials: y = x . W^T + b and its LayerNorm row partials."""
    rows, ci = x.shape
    co = w.shape[0]
    param = E.Param(ctx, w, f16=f16)
    xd, bd = E.DeviceArray.from_numpy(ctx, x), E.DeviceArray.from_numpy(ctx, b)
    out = E.DeviceArray(ctx, (rows, co))
    part = E.DeviceArray(ctx, (rows, -(-co // 32), 2))
    per_row = ctypes.c_uint32()
    E.check(E.lib().mh_conv1x1_row_partials(ctx.h, xd.ptr, rows, ci, param.ptr, param.dtype, co, bd.ptr, out.ptr,
                                            part.ptr, ctypes.byref(per_row)))
    n = per_row.value
    return out.numpy(), part.numpy().reshape(-1)[: rows * n * 2].reshape(rows, n, 2), n


def consumer(ctx, x, parts, gamma, beta, w, b, silu, f16=False, eps=1e-5):
    rows, ci = x.shape
    co = w.shape[0]
    param = E.Param(ctx, w, f16=f16)
    dev = {k: E.DeviceArray.from_numpy(ctx, np.ascontiguousarray(v))
           for k, v in dict(x=x, g=gamma, be=beta, b=b, p=parts).items()}
    out = E.DeviceArray(ctx, (rows, co))
    E.check(E.lib().mh_conv1x1_layer_norm_stats(ctx.h, dev["x"].ptr, rows, ci, dev["g"].ptr, dev["be"].ptr, eps,
                                                param.ptr, param.dtype, co, dev["b"].ptr, 1 if silu else 0,
                                                dev["p"].ptr, parts.shape[1], out.ptr))
    return out.numpy()


@pytest.mark.parametrize("rows,c,co", [(512, 320, 400), (512, 320, 1600), (128, 640, 800), (16, 1280, 1600),
                                       (198, 200, 72)])
@pytest.mark.parametrize("plan", [None, "32,32,1", "64,64,1", "128,128,1", "64,80,1,4,1,1,1", "32,80,1,2,1,2,1",
                                  "160,64,1,2,2,1,1,16"])
def test_row_partials_then_folded_layer_norm(ctx, rows, c, co, plan, tune):
    """proj_in (c -> c) writes h and its row partials; the q | k | v (or inverted)
    GEMM folds LayerNorm(h) with those statistics. The partials sum to h's row
    sums; the result matches the oracle's layer_norm then conv1x1 of that h."""
    rng = np.random.default_rng(rows + c + co)
    x = rng.standard_normal((rows, c)).astype(np.float32)
    wp = (rng.standard_normal((c, c)) / np.sqrt(c)).astype(np.float32)
    bp = (0.1 * rng.standard_normal(c)).astype(np.float32)
    _, g, be, w, b = inputs(rows, c, co, 3 + co)
    if plan:
        tune("gemm_plan", plan)
    print(f"row partials {rows}x{c}->{co} plan {plan}", flush=True)
    h, parts, n = producer(ctx, x, wp, bp)
    if n == 0:
        pytest.skip(f"plan {plan} writes no row partials for this shape")
    hd = h.astype(np.float64)
    assert np.allclose(parts[:, :, 0].astype(np.float64).sum(1), hd.sum(1), rtol=1e-5, atol=1e-3)
    assert np.allclose(parts[:, :, 1].astype(np.float64).sum(1), (hd * hd).sum(1), rtol=1e-5, atol=1e-3)
    tune("gemm_plan", None)
    got = consumer(ctx, h, parts, g, be, w, b, True)
    assert max_abs_rel(got, want(h, g, be, w, b, True)) <= F32_TIGHT


def test_row_partials_fast_precision(ctx):
    rows, c, co = 512, 320, 1600
    rng = np.random.default_rng(77)
    x = rng.standard_normal((rows, c)).astype(np.float32)
    wp = (rng.standard_normal((c, c)) / np.sqrt(c)).astype(np.float32)
    bp = (0.1 * rng.standard_normal(c)).astype(np.float32)
    _, g, be, w, b = inputs(rows, c, co, 78)
    ctx.set_precision(True)
    try:
        h, parts, n = producer(ctx, x, wp, bp, f16=True)
        assert n > 0
        got = consumer(ctx, h, parts, g, be, w, b, True, f16=True)
    finally:
        ctx.set_precision(False)
    assert max_abs_rel(got, want(h, g, be, w.astype(np.float16).astype(np.float32), b, True)) <= F16_TOL


@pytest.mark.parametrize("offset", [8.0, -30.0])
def test_row_partials_rows_far_from_zero_mean(ctx, offset):
    """sum y*y / K - mean^2 cancels when |mean| >> std: the f32 partials must
    still give the f32 bar (the rows here have std 1.5)."""
    rows, c, co = 512, 320, 400
    rng = np.random.default_rng(11)
    h = (rng.standard_normal((rows, c)) * 1.5 + offset).astype(np.float32)
    _, g, be, w, b = inputs(rows, c, co, 12)
    hd = h.astype(np.float64)
    # partials as a producer writes them: f32 sums over 64-column tiles
    t = hd.reshape(rows, c // 64, 64)
    parts = np.stack([t.sum(2), (t * t).sum(2)], -1).astype(np.float32)
    got = consumer(ctx, h, parts, g, be, w, b, False)
    assert max_abs_rel(got, want(h, g, be, w, b, False)) <= F32_TOL


@pytest.mark.parametrize("nb,hw,k", [(2, 4096, 40), (2, 1024, 80), (2, 256, 160), (1, 37, 40)])
def test_cross_lambda_row_sums(ctx, nb, hw, k):
    """The cross-lambda kernel's row sums are those of the rows it writes, and
    writing them changes none of the written bits."""
    rng = np.random.default_rng(k + hw)
    q = rng.standard_normal((nb, hw, 8 * k)).astype(np.float32)
    e = rng.standard_normal((hw, 10, k)).astype(np.float32)
    vb = rng.standard_normal((2, 10, k)).astype(np.float32)
    lam = (rng.standard_normal((2, k, k)) / np.sqrt(k)).astype(np.float32)
    h = rng.standard_normal((nb, hw, 8 * k)).astype(np.float32)
    dv = {n: E.DeviceArray.from_numpy(ctx, v) for n, v in dict(q=q, e=e, vb=vb, lam=lam).items()}
    print(f"cross-lambda row sums {nb}x{hw} k {k}", flush=True)
    h1, h2 = E.DeviceArray.from_numpy(ctx, h), E.DeviceArray.from_numpy(ctx, h)
    sums = E.DeviceArray(ctx, (nb * hw, 2))
    E.check(E.lib().mh_cross_lambda(ctx.h, dv["q"].ptr, dv["e"].ptr, dv["lam"].ptr, dv["vb"].ptr, 0, nb, hw, k,
                                    h1.ptr, h1.ptr))
    E.check(E.lib().mh_cross_lambda_row_sums(ctx.h, dv["q"].ptr, dv["e"].ptr, dv["lam"].ptr, dv["vb"].ptr, 0, nb, hw,
                                             k, h2.ptr, h2.ptr, sums.ptr))
    a, b2, s = h1.numpy(), h2.numpy(), sums.numpy()
    assert np.array_equal(a, b2)
    rows = a.reshape(nb * hw, 8 * k).astype(np.float64)
    assert np.allclose(s[:, 0], rows.sum(1), rtol=1e-5, atol=1e-3)
    assert np.allclose(s[:, 1], (rows * rows).sum(1), rtol=1e-5, atol=1e-3)


@pytest.mark.parametrize("nb,hh,ww,vd", [(2, 64, 64, 40), (2, 32, 32, 80), (2, 16, 16, 160), (1, 7, 5, 8),
                                         (1, 9, 70, 40)])
@pytest.mark.parametrize("variant,slice_", [(None, None), ("t4", None), ("t8", None), ("4", None), ("2", None),
                                            (None, "4"), ("t4", "2"), ("t8", "1"), ("t4", "5"), ("t4q2", None),
                                            ("t8q2", None), ("t4q2", "2")])
def test_tap_filter_row_sums(ctx, nb, hh, ww, vd, variant, slice_, tune):
    """The tap filter's LayerNorm 2 row sums (mh_tap_filter_row_sums) are those
    of the rows it writes (per channel slice where the kernel slices them), and
    writing them changes none of the written bits, in every kernel variant and
    slice width (a width not dividing the row's quads falls back to whole rows)."""
    if variant is not None:
        tune("tap_heads", variant[:2] if variant.endswith("q2") else variant)
        if variant.endswith("q2"):
            tune("tap_jq", 2)
    if slice_ is not None:
        tune("tap_slice", slice_)
    rng = np.random.default_rng(hh * ww + vd)
    npx = nb * hh * ww
    a = rng.standard_normal((npx, 226, 8)).astype(np.float32)
    v = rng.standard_normal((npx, vd)).astype(np.float32)
    yc = rng.standard_normal((npx, 8 * vd)).astype(np.float32)
    h = rng.standard_normal((npx, 8 * vd)).astype(np.float32)
    dv = {n: E.DeviceArray.from_numpy(ctx, x) for n, x in dict(a=a, v=v, yc=yc).items()}
    h1, h2 = E.DeviceArray.from_numpy(ctx, h), E.DeviceArray.from_numpy(ctx, h)
    sums = E.DeviceArray(ctx, (npx * (vd // 4), 2))
    per_row = ctypes.c_uint32()
    print(f"tap filter row sums {nb}x{hh}x{ww} vd {vd} variant {variant} slice {slice_}", flush=True)
    E.check(E.lib().mh_tap_filter(ctx.h, dv["a"].ptr, dv["v"].ptr, dv["yc"].ptr, h1.ptr, h1.ptr, nb, hh, ww, vd))
    E.check(E.lib().mh_tap_filter_row_sums(ctx.h, dv["a"].ptr, dv["v"].ptr, dv["yc"].ptr, h2.ptr, h2.ptr, nb, hh,
                                           ww, vd, sums.ptr, ctypes.byref(per_row)))
    o1, o2 = h1.numpy(), h2.numpy()
    n = per_row.value
    assert n >= 1 and (vd // 4) % n == 0
    s = sums.numpy()[: npx * n].reshape(npx, n, 2)
    assert np.array_equal(o1, o2)
    # slice j of a row: value channels [j * vd / n, (j + 1) * vd / n) of every head
    rows = o1.astype(np.float64).reshape(npx, 8, n, vd // n)
    assert np.allclose(s[:, :, 0], rows.sum((1, 3)), rtol=1e-5, atol=1e-2)
    assert np.allclose(s[:, :, 1], (rows * rows).sum((1, 3)), rtol=1e-5, atol=1e-2)
