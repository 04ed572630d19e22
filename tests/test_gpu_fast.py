"""GPU parity of the FAST precision (f16 matrix cores, f32 accumulate), through
the C ABI.

Two bars per GEMM-shaped kernel:
  - against the f32 oracle on the original operands: max-abs <= 2e-2 * max|ref|
    (the f16 path's tolerance for this hot path);
  - against an f64 product of the f16-rounded operands: max-abs <= 1e-3 *
    max|ref|. The kernel computes exactly that product with f32 sums, so this
    bar catches a missed K chunk, a mis-rounded operand or a wrong lane layout
    that the loose bar could let through.
Then the whole UNet step in FAST mode (f16-stored weights) against the oracle,
block by block, and the VAE, which keeps f32 arithmetic on a FAST context."""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from moebius_cpu_amd import engine as E
from moebius_cpu_amd import synthetic as S
from moebius_cpu_amd import unet_params as U
from moebius_cpu_amd import vae_params as V
from moebius_cpu_amd import workloads as W
from moebius_cpu_amd.unet import UNet
from moebius_cpu_amd.vae import Vae
from tests import ref_f64 as R
from tests.util import max_abs_rel

pytestmark = pytest.mark.gpu

FAST_TOL = 2e-2   # f16 path vs the f32 oracle
ROUND_TOL = 1e-3  # f16 path vs f64 on the f16-rounded operands


@pytest.fixture(scope="module")
def ctx():
    c = E.Context(0)
    c.set_precision(True)
    yield c
    c.synchronize()
    c.close()


def T(ctx, a):
    return E.Tensor.from_numpy(ctx, a)


def h(a):
    """f16 rounding (round to nearest even), back in f64."""
    return np.asarray(a, np.float32).astype(np.float16).astype(np.float64)


def conv1(ctx, x, w, b=None, r=None, f16=False):
    co, ci = w.shape
    out = E.Tensor(ctx)
    E.Conv1x1(ctx, ci, co, E.Param(ctx, w, f16=f16), b).forward(T(ctx, x), out, None if r is None else T(ctx, r))
    return out.numpy()


def conv3(ctx, x, w, b=None, stride=1, pad=(1, 1, 1, 1), up=False, prologue=None, f16=False):
    co, ci = w.shape[0], w.shape[3]
    out = E.Tensor(ctx)
    E.Conv3x3(ctx, ci, co, E.Param(ctx, w, f16=f16), b, stride, pad, up).forward_prologue(T(ctx, x), prologue, out)
    return out.numpy()


@pytest.mark.parametrize("plan", [None, "32,32,1", "32,32,3", "64,64,1", "64,64,2", "128,128,1", "128,128,2"])
@pytest.mark.parametrize("c_out,c_in", [(72, 320), (70, 200), (40, 9)])
@pytest.mark.parametrize("f16", [False, True])
def test_conv1x1_fast_every_tiling(ctx, plan, c_out, c_in, f16, tune):
    if plan:
        tune("gemm_plan", plan)
    rng = np.random.default_rng(c_out * 1000 + c_in)
    x = rng.standard_normal((2, 11, 13, c_in)).astype(np.float32)
    w = (rng.standard_normal((c_out, c_in)) * np.sqrt(2.0 / c_in)).astype(np.float32)
    b = (rng.standard_normal(c_out) * 0.02).astype(np.float32)
    r = rng.standard_normal((2, 11, 13, c_out)).astype(np.float32)
    got = conv1(ctx, x, w, b, r, f16=f16)
    exact = h(x).reshape(-1, c_in) @ h(w).T
    want_r = (r.reshape(-1, c_out).astype(np.float64) + b) + exact
    assert max_abs_rel(got.reshape(-1, c_out), want_r) <= ROUND_TOL
    assert max_abs_rel(got, oracle.conv1x1(x, w, b, r)) <= FAST_TOL


@pytest.mark.parametrize("n,h_,w_,ci,co,stride,pad,up", [
    (2, 9, 11, 64, 48, 1, (1, 1, 1, 1), False),     # Ci % 64 == 0: one tap per K tile
    (1, 16, 12, 320, 96, 2, (1, 1, 1, 1), False),   # stride-2 downsample
    (1, 10, 14, 128, 32, 2, (0, 0, 1, 1), False),   # VAE stride-2 padding
    (2, 6, 5, 160, 64, 1, (1, 1, 1, 1), True),      # nearest-2x upsample, Ci % 64 != 0
    (2, 7, 9, 24, 40, 1, (1, 1, 1, 1), False),      # Ci % 4 == 0 gather
    (1, 8, 8, 13, 22, 1, (1, 1, 1, 1), False),      # scalar gather
])
@pytest.mark.parametrize("f16", [False, True])
def test_conv3x3_fast_variants(ctx, n, h_, w_, ci, co, stride, pad, up, f16):
    rng = np.random.default_rng(ci * 7 + co)
    x = rng.standard_normal((n, h_, w_, ci)).astype(np.float32)
    w = (rng.standard_normal((co, 3, 3, ci)) * np.sqrt(2.0 / (9 * ci))).astype(np.float32)
    b = (rng.standard_normal(co) * 0.02).astype(np.float32)
    got = conv3(ctx, x, w, b, stride, pad, up, f16=f16)
    assert max_abs_rel(got, R.conv3x3(h(x), h(w), b.astype(np.float64), stride, pad, up)) <= ROUND_TOL
    assert max_abs_rel(got, oracle.conv3x3(x, w, b, stride, pad, up)) <= FAST_TOL


@pytest.mark.parametrize("ci,up", [(64, False), (96, True)])
def test_conv3x3_fast_gn_prologue(ctx, ci, up):
    rng = np.random.default_rng(ci)
    x = rng.standard_normal((2, 7, 9, ci)).astype(np.float32) * 3 + 1
    w = (rng.standard_normal((48, 3, 3, ci)) * 0.05).astype(np.float32)
    gamma = (1 + 0.1 * rng.standard_normal(ci)).astype(np.float32)
    beta = (0.1 * rng.standard_normal(ci)).astype(np.float32)
    gn = E.GroupNorm(ctx, 32, 1e-6, gamma, beta)
    aff = gn.affine(T(ctx, x), None, True)
    got = conv3(ctx, x, w, None, up=up, prologue=aff)
    normed = oracle.group_norm(x, 32, 1e-6, gamma, beta, silu=True)  # padding stays 0, not f(0)
    assert max_abs_rel(got, R.conv3x3(h(normed), h(w), 0.0, up=up)) <= ROUND_TOL
    assert max_abs_rel(got, oracle.conv3x3(normed, w, None, upsample2x=up)) <= FAST_TOL


@pytest.mark.parametrize("row_group", [0, 8])
@pytest.mark.parametrize("plan", [None, "32,32,1", "64,64,1", "64,64,2"])
def test_gemm_nt_fast(ctx, row_group, plan, tune):
    if plan:
        tune("gemm_plan", plan)
    rng = np.random.default_rng(9)
    m, n, k = 304, 226, 40
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((n, k)).astype(np.float32)
    ad, bd = E.DeviceArray.from_numpy(ctx, a), E.DeviceArray.from_numpy(ctx, b)
    if row_group:
        g = row_group
        c = E.DeviceArray(ctx, (m // g, n, g))
        E.check(E.lib().mh_gemm_nt(ctx.h, ad.ptr, k, bd.ptr, 0, k, m, n, k, None, None, c.ptr, n * g, g))
        got = c.numpy().transpose(0, 2, 1).reshape(m, n)
    else:
        c = E.DeviceArray(ctx, (m, n))
        E.check(E.lib().mh_gemm_nt(ctx.h, ad.ptr, k, bd.ptr, 0, k, m, n, k, None, None, c.ptr, n, 0))
        got = c.numpy()
    assert max_abs_rel(got, h(a) @ h(b).T) <= ROUND_TOL
    assert max_abs_rel(got, a.astype(np.float64) @ b.astype(np.float64).T) <= FAST_TOL


def test_f16_overflow_saturates_not_inf(ctx):
    """A finite activation beyond f16's range is clamped to +-65504 as it is
    rounded; the f32 sum stays finite."""
    x = np.ones((1, 4, 4, 64), np.float32)
    x[0, 1, 2, 5] = 1e6
    w = np.full((8, 64), 1e-3, np.float32)
    got = conv1(ctx, x, w)
    assert np.all(np.isfinite(got))
    assert np.isclose(got[0, 1, 2, 0], (63 + 65504) * np.float16(1e-3).astype(np.float64), rtol=1e-3)


def test_config_conv3x3_gn_silu_fast(ctx):
    wl = W.conv3x3_gn_silu()
    conv = E.Conv3x3.same(ctx, 320, 320, E.Param(ctx, wl.w, f16=True), wl.b)
    y, z = E.Tensor(ctx), E.Tensor(ctx)
    conv.forward(T(ctx, wl.x), y)
    E.GroupNorm(ctx, wl.groups, wl.eps, wl.gamma, wl.beta).forward(y, None, True, z)
    ref_y = oracle.conv3x3(wl.x, wl.w, wl.b)
    assert max_abs_rel(y.numpy(), ref_y) <= FAST_TOL
    ref_z = oracle.group_norm(ref_y, wl.groups, wl.eps, wl.gamma, wl.beta, silu=True)
    assert max_abs_rel(z.numpy(), ref_z) <= FAST_TOL


@pytest.mark.parametrize("s,c", W.SWEEP)
def test_kernel_sweep_fast_1x1(ctx, s, c):
    p = W.sweep_point(s, c)
    got = conv1(ctx, p.x, p.w1, p.b1, f16=True)
    assert max_abs_rel(got, oracle.conv1x1(p.x, p.w1, p.b1)) <= FAST_TOL


@pytest.fixture(scope="module")
def params():
    return U.random_unet(seed=4000)


def test_unet_step_fast_matches_oracle(ctx, params):
    """FAST mode: f16-stored GEMM weights on f16 matrix cores; every block of
    the step within 2e-2 * max|ref| of the f32 oracle on the same (rounded)
    weights."""
    gemm = {s.name for s in U.unet_specs() if s.gemm}
    rounded = {k: (v.astype(np.float16).astype(np.float32) if k in gemm else v) for k, v in params.items()}
    net = UNet(ctx, params, f16_gemm=True)
    inp = U.unet_input(seed=5006)
    eps_o, tr_o = oracle.UNet(rounded).forward(inp.x, inp.timestep, cfg=True, trace=True)
    eps_g, tr_g = net.forward_traced(inp.x, inp.timestep, cfg=True)
    assert list(tr_g) == list(tr_o)
    worst = 0.0
    for name in tr_o:
        err = max_abs_rel(tr_g[name], tr_o[name])
        worst = max(worst, err)
        assert err <= FAST_TOL, f"{name}: max-abs/max|ref| {err:.3e}"
    print(f"worst block max-abs/max|ref| = {worst:.3e}")
    assert max_abs_rel(eps_g, eps_o) <= FAST_TOL
    # The cond item of a CFG step is the cond-only step up to f16 rounding: the
    # batch-1 GEMMs are tiled (and K-split) differently, and the last-bit f32
    # differences that makes can move a later GEMM input across an f16 rounding
    # boundary. Repeated steps are bitwise equal.
    c = net.forward_host(inp.x, inp.timestep, cfg=False)
    assert max_abs_rel(c[0], eps_g[1]) <= FAST_TOL
    assert np.array_equal(net.forward_host(inp.x, inp.timestep, cfg=True), net.forward_host(inp.x, inp.timestep, cfg=True))


def test_unet_fast_cond_only_matches_oracle(ctx, params):
    """FAST at batch 1 (the cond-only steps of the Fast preset after its CFG steps,
    src/preset.rs:76-82) against the oracle on the f16-rounded weights, per traced
    block, at the FAST bar."""
    gemm = {s.name for s in U.unet_specs() if s.gemm}
    rounded = {k: (v.astype(np.float16).astype(np.float32) if k in gemm else v) for k, v in params.items()}
    net = UNet(ctx, params, f16_gemm=True)
    inp = U.unet_input(seed=5008)
    eps_o, tr_o = oracle.UNet(rounded).forward(inp.x, inp.timestep, cfg=False, trace=True)
    eps_g, tr_g = net.forward_traced(inp.x, inp.timestep, cfg=False)
    assert list(tr_g) == list(tr_o) and eps_g.shape == (1, 64, 64, 4)
    worst = 0.0
    for name in tr_o:
        err = max_abs_rel(tr_g[name], tr_o[name])
        worst = max(worst, err)
        assert err <= FAST_TOL, f"{name}: max-abs/max|ref| {err:.3e}"
    print(f"cond-only: worst block max-abs/max|ref| = {worst:.3e}")
    assert max_abs_rel(eps_g, eps_o) <= FAST_TOL


def test_vae_keeps_f32_on_fast_context(ctx):
    """The VAE computes in f32 whatever the context precision (the SDXL VAE's
    activations overflow f16): the f32 bar holds on a FAST context."""
    params = V.random_vae()
    lat = S.normal(21, (1, 8, 6, 4))
    got = Vae(ctx, params).decode_host(lat)
    assert max_abs_rel(got, oracle.Vae(params).decode(lat)) <= 1e-4


# FAST contexts evaluate the depthwise conv's GLU gate and GroupNorm-prologue
# SiLU with fast_silu (the hardware exp2 and reciprocal, dmath.hpp) instead of
# the reference's exp polynomial and IEEE division: against the oracle (the
# reference's SiLU, src/engine/math.rs:17-36, in depthwise.rs:31-59's tap
# order) within a few f32 ulp of the output's scale; EXACT contexts keep the
# bit-exact SiLU (test_gpu_engine.py).
@pytest.mark.parametrize("n,h,w,c,ep,silu", [(2, 9, 7, 64, "glu_silu", True), (1, 16, 16, 320, "relu", True),
                                             (2, 12, 10, 160, "glu_silu", False), (1, 33, 17, 80, "none", True)])
def test_depthwise_fast_silu(ctx, n, h, w, c, ep, silu):
    rng = np.random.default_rng(h * w + c + 3)
    x = (rng.standard_normal((n, h, w, c)) * 3).astype(np.float32)
    wt = (rng.standard_normal((3, 3, c)) * 0.3).astype(np.float32)
    b = (rng.standard_normal(c) * 0.1).astype(np.float32)
    gamma = (1 + 0.1 * rng.standard_normal(c)).astype(np.float32)
    beta = (0.1 * rng.standard_normal(c)).astype(np.float32)
    sc, sh = oracle.group_norm_affine(x, 2, 1e-5, gamma, beta)
    d = {k: E.DeviceArray.from_numpy(ctx, v) for k, v in dict(x=x, w=wt, b=b, sc=sc, sh=sh).items()}
    co = c // 2 if ep == "glu_silu" else c
    out = E.DeviceArray(ctx, (n, h, w, co))
    E.check(E.lib().mh_depthwise3x3_fused(ctx.h, d["x"].ptr, n, h, w, c, d["w"].ptr, d["b"].ptr, E._lib.EPILOGUE[ep],
                                          d["sc"].ptr, d["sh"].ptr, int(silu), out.ptr))
    a = np.stack([oracle.apply_affine(x[i], sc[i * c:(i + 1) * c], sh[i * c:(i + 1) * c], silu) for i in range(n)])
    want = oracle.depthwise3x3(a, wt, b, ep)
    assert max_abs_rel(out.numpy(), want) <= 4e-6
    # the plain depthwise (no prologue) with the GLU epilogue
    if ep == "glu_silu":
        plain = E.Tensor(ctx)
        E.depthwise3x3(T(ctx, x), wt, b, ep, plain)
        assert max_abs_rel(plain.numpy(), oracle.depthwise3x3(x, wt, b, ep)) <= 4e-6
