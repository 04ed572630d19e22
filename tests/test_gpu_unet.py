"""GPU parity of the UNet path, through the C ABI: the lambda-layer kernels
against the oracle (bit for bit where the kernel restates the CPU operation
order), then one full 512^2 denoise step (64x64 latent, random-init weights)
against the oracle, block by block with the reference's trace names."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

import oracle
from moebius_cpu_amd import engine as E
from moebius_cpu_amd import unet_params as U
from moebius_cpu_amd.unet import UNet
from tests.util import max_abs_rel

pytestmark = pytest.mark.gpu
TOL = 1e-4


@pytest.fixture(scope="module")
def ctx():
    c = E.Context(0)
    yield c
    c.synchronize()
    c.close()


def D(ctx, a):
    return E.DeviceArray.from_numpy(ctx, np.ascontiguousarray(a, dtype=np.float32))


@pytest.mark.parametrize("nb,rows,k", [(2, 4096, 40), (2, 1024, 80), (2, 256, 160), (2, 10, 40)])
def test_softmax_lambda_kernel(ctx, nb, rows, k):
    rng = np.random.default_rng(rows + k)
    keys = (rng.standard_normal((nb, rows, k)) * 2).astype(np.float32)
    v = rng.standard_normal((nb, rows, k)).astype(np.float32)
    out = E.DeviceArray(ctx, (nb, k, k))
    kd, vd_ = D(ctx, keys), D(ctx, v)  # held until the call returns
    E.check(E.lib().mh_softmax_lambda(ctx.h, kd.ptr, vd_.ptr, nb, rows, k, k, out.ptr))
    got = out.numpy()
    for b in range(nb):
        want = oracle.softmax_lambda(keys[b], v[b])
        assert max_abs_rel(got[b].T, want) < 1e-5


# "default": the planner's choice; "t8"/"t4": the LDS-staged row-tile kernel
# with 8 / 4 heads per thread (partial tiles at 9 x 70, 16 x 16 x 160 and
# 20 x 9); "8"/"4"/"2": the per-thread kernel's variants.
@pytest.mark.parametrize("nb,hh,ww,vd", [(2, 16, 12, 40), (1, 7, 5, 8), (2, 16, 16, 160), (1, 20, 9, 80),
                                         (1, 9, 70, 40)])
@pytest.mark.parametrize("heads_per_thread", ["default", "t8", "t4", "8", "4", "2", "t8q2", "t4q2"])
def test_tap_filter_kernel_bit_exact(ctx, nb, hh, ww, vd, heads_per_thread, tune):
    """q2: the tile kernel with two value channel quads per thread."""
    tune("tap_split", 1)  # one thread per output: the reference's tap order
    if heads_per_thread == "default":
        tune("tap_heads", None)
    else:
        tune("tap_heads", heads_per_thread[:2] if heads_per_thread.endswith("q2") else heads_per_thread)
    if heads_per_thread.endswith("q2"):
        tune("tap_jq", 2)
    rng = np.random.default_rng(hh * ww + vd)
    a = rng.standard_normal((nb, hh * ww, 8, 226)).astype(np.float32)
    v = rng.standard_normal((nb, hh * ww, vd)).astype(np.float32)
    o = rng.standard_normal((nb, hh * ww, 8 * vd)).astype(np.float32)
    h = rng.standard_normal((nb, hh * ww, 8 * vd)).astype(np.float32)
    # the device takes A tap-major: [pixel][226][head]
    ad, vdev, yd = D(ctx, a.transpose(0, 1, 3, 2)), D(ctx, v), D(ctx, o)
    out = E.DeviceArray(ctx, o.shape)
    E.check(E.lib().mh_tap_filter(ctx.h, ad.ptr, vdev.ptr, yd.ptr, None, out.ptr, nb, hh, ww, vd))
    got = out.numpy()
    # residual form, in place on the residual: h + u
    hd = D(ctx, h)
    E.check(E.lib().mh_tap_filter(ctx.h, ad.ptr, vdev.ptr, yd.ptr, hd.ptr, hd.ptr, nb, hh, ww, vd))
    got_res = hd.numpy()
    for b in range(nb):
        want = oracle.tap_filter(a[b], v[b], o[b], hh, ww)
        assert np.array_equal(got[b], want)
        assert np.array_equal(got_res[b], h[b] + want)


# The tap rows split over 3 or 5 threads per output (the 32x32 and 16x16
# latents' default): the same sums in partial chains added in row order, so
# within f32 rounding of the reference's order; residual form and LayerNorm 2.
@pytest.mark.parametrize("nb,hh,ww,vd", [(2, 32, 32, 80), (2, 16, 16, 160), (1, 7, 5, 8), (1, 20, 9, 80)])
@pytest.mark.parametrize("split", [3, 5])
@pytest.mark.parametrize("heads_per_thread", ["default", "8", "2"])
def test_tap_filter_row_split(ctx, nb, hh, ww, vd, split, heads_per_thread, tune):
    tune("tap_split", split)
    tune("tap_heads", None if heads_per_thread == "default" else heads_per_thread)
    rng = np.random.default_rng(hh * ww + vd + split)
    a = rng.standard_normal((nb, hh * ww, 8, 226)).astype(np.float32)
    v = rng.standard_normal((nb, hh * ww, vd)).astype(np.float32)
    o = rng.standard_normal((nb, hh * ww, 8 * vd)).astype(np.float32)
    h = rng.standard_normal((nb, hh * ww, 8 * vd)).astype(np.float32)
    g = (1 + 0.1 * rng.standard_normal(8 * vd)).astype(np.float32)
    be = (0.1 * rng.standard_normal(8 * vd)).astype(np.float32)
    ad, vdev, yd = D(ctx, a.transpose(0, 1, 3, 2)), D(ctx, v), D(ctx, o)
    out = E.DeviceArray(ctx, o.shape)
    print(f"tap split {split} heads {heads_per_thread} {nb}x{hh}x{ww}x{vd}", flush=True)
    E.check(E.lib().mh_tap_filter(ctx.h, ad.ptr, vdev.ptr, yd.ptr, None, out.ptr, nb, hh, ww, vd))
    got = out.numpy()
    hd, gd, bd = D(ctx, h), D(ctx, g), D(ctx, be)
    ln = E.DeviceArray(ctx, o.shape)
    E.check(E.lib().mh_tap_filter_ln(ctx.h, ad.ptr, vdev.ptr, yd.ptr, hd.ptr, hd.ptr, nb, hh, ww, vd, gd.ptr, bd.ptr,
                                     1e-5, ln.ptr))
    got_res, got_ln = hd.numpy(), ln.numpy()
    for b in range(nb):
        want = oracle.tap_filter(a[b], v[b], o[b], hh, ww)
        assert max_abs_rel(got[b], want) < 1e-5
        assert max_abs_rel(got_res[b], h[b] + want) < 1e-5
        assert max_abs_rel(got_ln[b], oracle.layer_norm(h[b] + want, g, be, 1e-5)) < 1e-4


# Position coefficients A = Q . W_aug (lambda.rs:131-137) by the matrix-core
# kernel, tap-major, and with lambda_t the content term Yc = Q . lambda_c per
# item (lambda.rs:123): against the f64 products and against the general
# GEMM's outputs of the same products; odd pixel counts leave a half pair.
@pytest.mark.parametrize("nb,hw,k", [(2, 4096, 40), (2, 1024, 80), (2, 256, 160), (1, 7, 40), (3, 1, 80),
                                     (2, 301, 80), (1, 9, 160)])
@pytest.mark.parametrize("content", [False, True])
def test_lambda_position_coeffs_kernel(ctx, nb, hw, k, content):
    rng = np.random.default_rng(nb * hw + k)
    npx = nb * hw
    q = rng.standard_normal((npx, 8, k)).astype(np.float32)
    w = rng.standard_normal((226, k)).astype(np.float32)
    lam_t = rng.standard_normal((nb, k, k)).astype(np.float32)  # [item][j][kk]
    q64 = q.reshape(npx * 8, k).astype(np.float64)
    want = (q64 @ w.astype(np.float64).T).reshape(npx, 8, 226).transpose(0, 2, 1)
    qd, wd, ld = D(ctx, q), D(ctx, w), D(ctx, lam_t)
    out = E.DeviceArray(ctx, (npx, 226, 8))
    yc = E.DeviceArray(ctx, (npx, 8, k)) if content else None
    E.check(E.lib().mh_lambda_position_coeffs(ctx.h, qd.ptr, wd.ptr, ld.ptr if content else None, nb, hw, k, out.ptr,
                                              yc.ptr if content else None))
    got = out.numpy()
    assert max_abs_rel(got, want) < 1e-5
    g = E.DeviceArray(ctx, (npx, 226, 8))
    E.check(E.lib().mh_gemm_nt(ctx.h, qd.ptr, k, wd.ptr, 0, k, npx * 8, 226, k, None, None, g.ptr, 226 * 8, 8))
    assert max_abs_rel(got, g.numpy()) < 1e-5
    if content:
        qi = q.reshape(nb, hw * 8, k).astype(np.float64)
        want_yc = np.stack([qi[b] @ lam_t[b].astype(np.float64).T for b in range(nb)]).reshape(npx, 8, k)
        got_yc = yc.numpy()
        assert max_abs_rel(got_yc, want_yc) < 1e-5
        gy = E.DeviceArray(ctx, (npx, 8, k))
        E.check(E.lib().mh_gemm_nt(ctx.h, qd.ptr, k, ld.ptr, 0, k, hw * 8, k, k, None, None, gy.ptr, k, 0))
        if nb == 1:
            assert max_abs_rel(got_yc, gy.numpy()) < 1e-5


# Every part height of the kernel (80, 48 and 16 rows; the launcher picks one by
# map size) runs each output's MFMA chain unchanged: the same bits as the
# default, for A and Yc, in EXACT and FAST precision.
@pytest.mark.parametrize("nb,hw,k", [(2, 4096, 40), (2, 1024, 80), (2, 256, 160), (1, 7, 40), (2, 301, 80),
                                     (1, 9, 160)])
@pytest.mark.parametrize("fast", [False, True])
def test_lambda_position_coeffs_every_part_height(ctx, nb, hw, k, fast, tune):
    rng = np.random.default_rng(3 * hw + k)
    npx = nb * hw
    q = rng.standard_normal((npx, 8, k)).astype(np.float32)
    w = rng.standard_normal((226, k)).astype(np.float32)
    lam_t = rng.standard_normal((nb, k, k)).astype(np.float32)
    qd, wd, ld = D(ctx, q), D(ctx, w), D(ctx, lam_t)
    runs = []
    ctx.set_precision(fast)
    try:
        for rows in (None, 80, 48, 16):
            tune("taps_rows", rows)
            print(f"position coeffs {nb}x{hw} k {k} fast={fast} rows {rows}", flush=True)
            out, yc = E.DeviceArray(ctx, (npx, 226, 8)), E.DeviceArray(ctx, (npx, 8, k))
            E.check(E.lib().mh_lambda_position_coeffs(ctx.h, qd.ptr, wd.ptr, ld.ptr, nb, hw, k, out.ptr, yc.ptr))
            runs.append((out.numpy(), yc.numpy()))
    finally:
        ctx.set_precision(False)
    for a, y in runs[1:]:
        assert np.array_equal(a, runs[0][0]) and np.array_equal(y, runs[0][1])


# The content term alone (the cross-lambda's Yc = Q . lambda_c[branch], item b
# on branch br0 + b): lambda_t points at the first item's branch.
@pytest.mark.parametrize("br0,nb,hw,k", [(0, 2, 4096, 40), (1, 1, 1024, 80), (0, 2, 256, 160), (0, 2, 37, 40)])
def test_lambda_content_term_alone(ctx, br0, nb, hw, k):
    rng = np.random.default_rng(br0 + hw + k)
    npx = nb * hw
    q = rng.standard_normal((npx, 8, k)).astype(np.float32)
    lam_t = rng.standard_normal((2, k, k)).astype(np.float32)
    qd, ld = D(ctx, q), D(ctx, lam_t)
    yc = E.DeviceArray(ctx, (npx, 8, k))
    first = ctypes.c_void_p(ld.ptr + br0 * k * k * 4)
    E.check(E.lib().mh_lambda_position_coeffs(ctx.h, qd.ptr, None, first, nb, hw, k, None, yc.ptr))
    qi = q.reshape(nb, hw * 8, k).astype(np.float64)
    want = np.stack([qi[b] @ lam_t[br0 + b].astype(np.float64).T for b in range(nb)]).reshape(npx, 8, k)
    assert max_abs_rel(yc.numpy(), want) < 1e-5


def _h16(a):
    return np.clip(a, -65504, 65504).astype(np.float16).astype(np.float64)


# FAST contexts: by default the products of the f32 operands, the EXACT
# kernel's bits; with tuning taps_r16 1 the products of f16-rounded operands (as
# the FAST GEMMs take them), summed in f32: against the f64 sums of the same
# products and against the FAST GEMM's output.
@pytest.mark.parametrize("nb,hw,k", [(2, 4096, 40), (2, 1024, 80), (2, 256, 160), (1, 7, 40)])
def test_lambda_position_coeffs_fast_default_is_exact(ctx, nb, hw, k):
    rng = np.random.default_rng(5 * hw + k)
    npx = nb * hw
    q = rng.standard_normal((npx, 8, k)).astype(np.float32)
    w = rng.standard_normal((226, k)).astype(np.float32)
    lam_t = rng.standard_normal((nb, k, k)).astype(np.float32)
    want = (q.reshape(npx * 8, k).astype(np.float64) @ w.astype(np.float64).T).reshape(npx, 8, 226).transpose(0, 2, 1)
    qd, wd, ld = D(ctx, q), D(ctx, w), D(ctx, lam_t)
    got = {}
    for fast in (False, True):
        out, yc = E.DeviceArray(ctx, (npx, 226, 8)), E.DeviceArray(ctx, (npx, 8, k))
        ctx.set_precision(fast)
        try:
            E.check(E.lib().mh_lambda_position_coeffs(ctx.h, qd.ptr, wd.ptr, ld.ptr, nb, hw, k, out.ptr, yc.ptr))
        finally:
            ctx.set_precision(False)
        got[fast] = (out.numpy(), yc.numpy())
    assert max_abs_rel(got[True][0], want) < 1e-5
    assert np.array_equal(got[True][0], got[False][0]) and np.array_equal(got[True][1], got[False][1])


@pytest.mark.parametrize("nb,hw,k", [(2, 4096, 40), (2, 1024, 80), (2, 256, 160), (1, 7, 40)])
def test_lambda_position_coeffs_fast(ctx, nb, hw, k, tune):
    tune("taps_r16", 1)
    rng = np.random.default_rng(7 * hw + k)
    npx = nb * hw
    q = rng.standard_normal((npx, 8, k)).astype(np.float32)
    w = rng.standard_normal((226, k)).astype(np.float32)
    lam_t = rng.standard_normal((nb, k, k)).astype(np.float32)
    want = (_h16(q.reshape(npx * 8, k)) @ _h16(w).T).reshape(npx, 8, 226).transpose(0, 2, 1)
    qi = _h16(q.reshape(nb, hw * 8, k))
    want_yc = np.stack([qi[b] @ _h16(lam_t[b]).T for b in range(nb)]).reshape(npx, 8, k)
    qd, wd, ld = D(ctx, q), D(ctx, w), D(ctx, lam_t)
    out, yc, g = E.DeviceArray(ctx, (npx, 226, 8)), E.DeviceArray(ctx, (npx, 8, k)), E.DeviceArray(ctx, (npx, 226, 8))
    ctx.set_precision(True)
    try:
        E.check(E.lib().mh_lambda_position_coeffs(ctx.h, qd.ptr, wd.ptr, ld.ptr, nb, hw, k, out.ptr, yc.ptr))
        E.check(E.lib().mh_gemm_nt(ctx.h, qd.ptr, k, wd.ptr, 0, k, npx * 8, 226, k, None, None, g.ptr, 226 * 8, 8))
    finally:
        ctx.set_precision(False)
    assert max_abs_rel(out.numpy(), want) < 1e-5
    assert max_abs_rel(yc.numpy(), want_yc) < 1e-5
    assert max_abs_rel(out.numpy(), g.numpy()) < 1e-5


def test_lambda_position_coeffs_rejects_bad_arguments(ctx):
    q = E.DeviceArray(ctx, (2, 8, 120))
    w = E.DeviceArray(ctx, (226, 120))
    out = E.DeviceArray(ctx, (2, 226, 8))
    assert E.lib().mh_lambda_position_coeffs(ctx.h, q.ptr, w.ptr, None, 1, 2, 120, out.ptr, None) != 0
    # lambda_t without yc
    assert E.lib().mh_lambda_position_coeffs(ctx.h, q.ptr, w.ptr, w.ptr, 1, 2, 40, out.ptr, None) != 0


# The one-pass position path (mh_self_lambda_fused) against the two kernels it
# replaces, mh_lambda_position_coeffs then the tap filter with one thread per
# output (tap_split 1, the tile kernel with 4 heads per thread, whose row sums
# take the same order): the same bits for out and the row sums, with and
# without a residual, EXACT and FAST. Shapes: the UNet's three levels at batch
# 2, a partial last row tile with an odd pixel count (70 = 5 x 12 + 10, 17),
# maps narrower than the window (7 x 5, 1 x 1) and single items.
@pytest.mark.parametrize("nb,hh,ww,k", [(2, 64, 64, 40), (2, 32, 32, 80), (2, 16, 16, 160), (1, 9, 70, 40),
                                        (1, 20, 9, 80), (1, 7, 5, 40), (3, 1, 1, 160), (1, 5, 17, 40)])
@pytest.mark.parametrize("fast", [False, True, "r16"])
def test_self_lambda_fused_bit_exact(ctx, nb, hh, ww, k, fast, tune):
    """r16: a FAST context with tuning taps_r16 1 (f16-rounded products)."""
    tune("tap_split", 1)
    tune("tap_heads", "t4")
    if fast == "r16":
        tune("taps_r16", 1)
    rng = np.random.default_rng(hh * ww + k + nb)
    npx = nb * hh * ww
    q = rng.standard_normal((npx, 8, k)).astype(np.float32)
    w = (rng.standard_normal((226, k)) * 0.3).astype(np.float32)
    lam_t = (rng.standard_normal((nb, k, k)) * 0.3).astype(np.float32)
    v = rng.standard_normal((npx, k)).astype(np.float32)
    h = rng.standard_normal((npx, 8 * k)).astype(np.float32)
    qd, wd, ld, vd_ = D(ctx, q), D(ctx, w), D(ctx, lam_t), D(ctx, v)
    a, yc = E.DeviceArray(ctx, (npx, 226, 8)), E.DeviceArray(ctx, (npx, 8, k))
    ref_h, got_h = D(ctx, h), D(ctx, h)
    ref_o, got_o = E.DeviceArray(ctx, (npx, 8 * k)), E.DeviceArray(ctx, (npx, 8 * k))
    ref_s, got_s = E.DeviceArray(ctx, (npx * k // 4, 2)), E.DeviceArray(ctx, (npx, 2))
    per_row = ctypes.c_uint32()
    print(f"self-lambda fused {nb}x{hh}x{ww} k {k} fast={fast}", flush=True)
    ctx.set_precision(fast)
    try:
        E.check(E.lib().mh_lambda_position_coeffs(ctx.h, qd.ptr, wd.ptr, ld.ptr, nb, hh * ww, k, a.ptr, yc.ptr))
        E.check(E.lib().mh_tap_filter_row_sums(ctx.h, a.ptr, vd_.ptr, yc.ptr, ref_h.ptr, ref_h.ptr, nb, hh, ww, k,
                                               ref_s.ptr, ctypes.byref(per_row)))
        E.check(E.lib().mh_tap_filter(ctx.h, a.ptr, vd_.ptr, yc.ptr, None, ref_o.ptr, nb, hh, ww, k))
        E.check(E.lib().mh_self_lambda_fused(ctx.h, qd.ptr, wd.ptr, ld.ptr, vd_.ptr, got_h.ptr, got_h.ptr, nb, hh, ww,
                                             k, got_s.ptr))
        E.check(E.lib().mh_self_lambda_fused(ctx.h, qd.ptr, wd.ptr, ld.ptr, vd_.ptr, None, got_o.ptr, nb, hh, ww, k,
                                             None))
    finally:
        ctx.set_precision(False)
    assert per_row.value == 1
    assert np.array_equal(got_h.numpy(), ref_h.numpy())
    assert np.array_equal(got_s.numpy(), ref_s.numpy()[:npx])
    assert np.array_equal(got_o.numpy(), ref_o.numpy())


def test_self_lambda_fused_rejects_bad_arguments(ctx):
    q = E.DeviceArray(ctx, (2, 8, 120))
    w = E.DeviceArray(ctx, (226, 120))
    lam = E.DeviceArray(ctx, (1, 120, 120))
    v = E.DeviceArray(ctx, (2, 120))
    out = E.DeviceArray(ctx, (2, 8 * 120))
    assert E.lib().mh_self_lambda_fused(ctx.h, q.ptr, w.ptr, lam.ptr, v.ptr, None, out.ptr, 1, 1, 2, 120, None) != 0
    # out aliasing q
    assert E.lib().mh_self_lambda_fused(ctx.h, q.ptr, w.ptr, lam.ptr, v.ptr, None, q.ptr, 1, 1, 2, 40, None) != 0
    assert E.lib().mh_self_lambda_fused(ctx.h, q.ptr, None, lam.ptr, v.ptr, None, out.ptr, 1, 1, 2, 40, None) != 0


@pytest.mark.parametrize("br0,nb,k", [(0, 2, 40), (1, 1, 80), (0, 2, 160)])
def test_position_term_kernel_bit_exact(ctx, br0, nb, k):
    hw = 37
    rng = np.random.default_rng(k + nb)
    q = rng.standard_normal((nb, hw, 8 * k)).astype(np.float32)
    e = rng.standard_normal((hw, 10, k)).astype(np.float32)
    vb = rng.standard_normal((2, 10, k)).astype(np.float32)
    o = rng.standard_normal((nb, hw, 8 * k)).astype(np.float32)
    h = rng.standard_normal((nb, hw, 8 * k)).astype(np.float32)
    od = D(ctx, o)
    qd, ed, vbd, hd = D(ctx, q), D(ctx, e), D(ctx, vb), D(ctx, h)
    out = E.DeviceArray(ctx, o.shape)
    E.check(E.lib().mh_position_term(ctx.h, qd.ptr, ed.ptr, vbd.ptr, br0, nb, hw, k, od.ptr, None, out.ptr))
    E.check(E.lib().mh_position_term(ctx.h, qd.ptr, ed.ptr, vbd.ptr, br0, nb, hw, k, od.ptr, hd.ptr, hd.ptr))
    got, got_res = out.numpy(), hd.numpy()
    for b in range(nb):
        want = oracle.position_term(q[b], e, vb[br0 + b], o[b])
        assert np.array_equal(got[b], want)
        assert np.array_equal(got_res[b], h[b] + want)


# CrossLambda::forward after to_q (src/unet/lambda.rs:258-271) in one kernel:
# with lambda_c = 0 the Yc part is exactly +0 and the rest must be the
# position term bit for bit; with a real lambda_c, Yc = Q . lambda_c (f64
# reference) within the f32 bar. Sizes select the default heads-per-thread
# variants (4 at 64x64 / k 40 and 32x32 / k 80, 2 at 16x16 / k 160) plus a ragged
# block; MOEBIUS_HIP_CROSS_HEADS forces each variant, 8 included.
# None: the default, the matrix-core kernel for these head widths (its pixel
# blocks never straddle items: 37 and 9 pixels per item leave ragged blocks).
@pytest.mark.parametrize("br0,nb,hw,k", [(0, 2, 4096, 40), (0, 2, 1024, 80), (0, 2, 256, 160), (1, 1, 37, 40),
                                         (0, 2, 37, 80), (0, 2, 9, 160), (0, 2, 13, 40)])
@pytest.mark.parametrize("heads", [None, "2", "4", "8"])
def test_cross_lambda_kernel(ctx, br0, nb, hw, k, heads, tune):
    if heads:
        tune("cross_heads", heads)
    else:
        tune("cross_heads", None)
    rng = np.random.default_rng(k + hw)
    q = rng.standard_normal((nb, hw, 8 * k)).astype(np.float32)
    e = rng.standard_normal((hw, 10, k)).astype(np.float32)
    vb = rng.standard_normal((2, 10, k)).astype(np.float32)
    lam = (rng.standard_normal((2, k, k)) / np.sqrt(k)).astype(np.float32)
    h = rng.standard_normal((nb, hw, 8 * k)).astype(np.float32)
    qd, ed, vbd, hd = D(ctx, q), D(ctx, e), D(ctx, vb), D(ctx, h)
    out = E.DeviceArray(ctx, q.shape)
    zero = D(ctx, np.zeros_like(lam))
    E.check(E.lib().mh_cross_lambda(ctx.h, qd.ptr, ed.ptr, zero.ptr, vbd.ptr, br0, nb, hw, k, None, out.ptr))
    got0 = out.numpy()
    lamd = D(ctx, lam)
    E.check(E.lib().mh_cross_lambda(ctx.h, qd.ptr, ed.ptr, lamd.ptr, vbd.ptr, br0, nb, hw, k, None, out.ptr))
    got = out.numpy()
    E.check(E.lib().mh_cross_lambda(ctx.h, qd.ptr, ed.ptr, lamd.ptr, vbd.ptr, br0, nb, hw, k, hd.ptr, hd.ptr))
    got_res = hd.numpy()
    for b in range(nb):
        zeros = np.zeros((hw, 8 * k), np.float32)
        assert np.array_equal(got0[b], oracle.position_term(q[b], e, vb[br0 + b], zeros))
        yc = (q[b].reshape(hw * 8, k).astype(np.float64) @ lam[br0 + b].astype(np.float64)).reshape(hw, 8 * k)
        want = oracle.position_term(q[b], e, vb[br0 + b], yc.astype(np.float32))
        assert max_abs_rel(got[b], want) < 1e-5
        assert max_abs_rel(got_res[b], h[b] + want) < 1e-5


# Grouped rows (out[m / g][n][m % g], the self-lambda's [pixel][tap][head] A) take
# 16-byte stores of four rows when g % 4 == 0; plain rows, a ragged last tile,
# a K split and the bias epilogue around them.
@pytest.mark.parametrize("row_group", [0, 4, 8])
@pytest.mark.parametrize("plan", [None, "32,32,1", "64,64,1", "64,64,2", "64,80,1,4,1,1,1", "128,80,1,4,1,1,1",
                                  "32,80,1,2,1,2,1", "160,64,1,2,2,1,1", "160,64,1,2,2,1,1,16", "128,128,1,2,2,1,1,16"])
@pytest.mark.parametrize("with_bias", [False, True])
def test_gemm_nt_kernel(ctx, row_group, plan, with_bias, tune):
    if plan:
        tune("gemm_plan", plan)
    rng = np.random.default_rng(9)
    m, n, k = 304, 226, 40
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((n, k)).astype(np.float32)
    bias = rng.standard_normal(n).astype(np.float32)
    want = a.astype(np.float64) @ b.astype(np.float64).T + (bias.astype(np.float64) if with_bias else 0.0)
    ad, bd = D(ctx, a), D(ctx, b)
    biasd = D(ctx, bias) if with_bias else None  # kept alive until the kernel has run
    bp = biasd.ptr if with_bias else None
    if row_group:
        g = row_group
        c = E.DeviceArray(ctx, (m // g, n, g))
        E.check(E.lib().mh_gemm_nt(ctx.h, ad.ptr, k, bd.ptr, 0, k, m, n, k, bp, None, c.ptr, n * g, g))
        got = c.numpy().transpose(0, 2, 1).reshape(m, n)
    else:
        c = E.DeviceArray(ctx, (m, n))
        E.check(E.lib().mh_gemm_nt(ctx.h, ad.ptr, k, bd.ptr, 0, k, m, n, k, bp, None, c.ptr, n, 0))
        got = c.numpy()
    assert max_abs_rel(got, want) < 1e-5


def test_best_fit_matches_reference_policy():
    """src/engine/mod.rs:104-117 and its tests (mod.rs:124-181)."""
    L = E.lib()

    def bf(pairs, want):
        lens = (ctypes.c_uint64 * len(pairs))(*[p[0] for p in pairs])
        caps = (ctypes.c_uint64 * len(pairs))(*[p[1] for p in pairs])
        return L.mh_scratch_best_fit(lens, caps, len(pairs), want)

    assert bf([(100, 100), (1000, 1000), (10, 10)], 1000) == 1
    assert bf([(100, 100), (1000, 1000), (10, 10)], 10) == 2
    assert bf([(100, 100), (1000, 1000), (10, 10)], 100) == 0
    assert bf([(100, 100), (1000, 1000), (10, 10)], 5000) == 1  # largest grows
    assert bf([(10, 200), (50, 60)], 55) == 1                    # least growth within capacity
    assert bf([(64, 64), (64, 64)], 64) == 1                     # later entries win ties
    assert bf([], 1) == -1


@pytest.fixture(scope="module")
def params():
    return U.random_unet(seed=4000)


@pytest.fixture(scope="module")
def onet(params):
    return oracle.UNet(params)


@pytest.fixture(scope="module")
def gnet(ctx, params):
    return UNet(ctx, params)


def _compare_traces(got, want):
    assert list(got) == list(want), "trace names or order differ"
    worst = 0.0
    for name in want:
        err = max_abs_rel(got[name], want[name])
        worst = max(worst, err)
        assert err <= TOL, f"{name}: max-abs/max|ref| {err:.3e}"
    return worst


def test_unet_step_cfg_matches_oracle(ctx, gnet, onet):
    inp = U.unet_input(seed=5000)
    eps_o, tr_o = onet.forward(inp.x, inp.timestep, cfg=True, trace=True)
    eps_g, tr_g = gnet.forward_traced(inp.x, inp.timestep, cfg=True)
    worst = _compare_traces(tr_g, tr_o)
    print(f"worst block max-abs/max|ref| = {worst:.3e}")
    assert max_abs_rel(eps_g, eps_o) <= TOL


def test_unet_step_cond_only_matches_oracle(ctx, gnet, onet):
    inp = U.unet_input(seed=5003)
    eps_o = onet.forward(inp.x, inp.timestep, cfg=False)
    eps_g = gnet.forward_host(inp.x, inp.timestep, cfg=False)
    assert eps_g.shape == (1, 64, 64, 4)
    assert max_abs_rel(eps_g, eps_o) <= TOL


def test_unet_step_is_deterministic_and_batch_consistent(ctx, gnet):
    inp = U.unet_input(seed=5004)
    a = gnet.forward_host(inp.x, inp.timestep, cfg=True)
    b = gnet.forward_host(inp.x, inp.timestep, cfg=True)
    assert np.array_equal(a, b)
    c = gnet.forward_host(inp.x, inp.timestep, cfg=False)
    assert max_abs_rel(c[0], a[1]) <= TOL  # the cond item of a CFG step is the cond-only step


@pytest.mark.parametrize("cfg", [False, True])
@pytest.mark.parametrize("fast", [False, True])
def test_unet_up_path_two_inputs_is_bit_exact(ctx, gnet, fast, cfg, tune):
    """The up path's resnets read [h | skip] from the two tensors (GroupNorm
    statistics, the depthwise staging and the shortcut GEMM each take two base
    pointers) and give the bits of writing the concatenation first, as the
    reference does (src/unet/mod.rs:208-213)."""
    inp = U.unet_input(seed=5011)
    ctx.set_precision(fast)
    try:
        tune("up_concat", "1")
        cat = gnet.forward_host(inp.x, inp.timestep, cfg=cfg)
        tune("up_concat", "0")
        two = gnet.forward_host(inp.x, inp.timestep, cfg=cfg)
    finally:
        ctx.set_precision(False)
    assert np.array_equal(cat, two)


@pytest.mark.parametrize("fast", [False, True])
def test_unet_fused_self_lambda_is_bit_exact(ctx, gnet, fast, tune):
    """The 64x64 level's self-lambda with its position coefficients and content
    term formed inside the tap filter (tap_fused 1, the default) gives the bits of
    writing them first (tap_fused 0): both take one thread per output there."""
    inp = U.unet_input(seed=5013)
    ctx.set_precision(fast)
    try:
        tune("tap_fused", "0")
        apart = gnet.forward_host(inp.x, inp.timestep, cfg=True)
        tune("tap_fused", "1")
        fused = gnet.forward_host(inp.x, inp.timestep, cfg=True)
    finally:
        ctx.set_precision(False)
    assert np.array_equal(apart, fused)


@pytest.mark.parametrize("fast", [False, True])
def test_unet_groupnorm_into_proj_in_is_bit_exact(ctx, gnet, fast, tune):
    """The transformers' GroupNorm applied inside proj_in's operand loads gives the
    bits of the separate apply pass, at every channel count it is used for."""
    inp = U.unet_input(seed=5007)
    ctx.set_precision(fast)
    try:
        tune("gn_in_maxc", "0")
        apart = gnet.forward_host(inp.x, inp.timestep, cfg=True)
        tune("gn_in_maxc", "1280")
        fused = gnet.forward_host(inp.x, inp.timestep, cfg=True)
    finally:
        ctx.set_precision(False)
    assert np.array_equal(apart, fused)


@pytest.fixture(scope="module")
def g16net(ctx, params):
    """The UNet with f16-stored GEMM weights (what FAST's f16 stores apply to)."""
    return UNet(ctx, params, f16_gemm=True)


def _f16a_launches(ctx):
    """Launches of the f16-input GEMM family in the context's GEMM census."""
    return sum(r["launches"] for r in ctx.gemm_times() if r["config"].startswith("f16a "))


def test_unet_fast_f16_operands_are_bit_exact(ctx, g16net, tune):
    """FAST contexts store in f16 what only an f16 GEMM reads: the upsample convs'
    Winograd kernel U (tuning wino_u16) and input transform V (wino_v16), the
    depthwise convs' outputs that only the next 1x1 reads (dw_out16; the resnets'
    DwConv2d and the MixFFN's GLU) and the MixFFN's pointwise output that only
    proj_out reads (with dw_out16). Each is rounded to nearest even with the
    saturation the f16 GEMM applies to f32 operands as it loads them, so every
    combination gives the bits of all of them off. The f16 stores need f16-stored
    GEMM weights; the GEMM census shows the f16-input GEMMs running."""
    inp = U.unet_input(seed=5019)
    ctx.set_precision(True)
    outs, f16a = [], []
    try:
        tune("gemm_time", 1)
        ctx.gemm_times()
        for u16, v16, dw16 in ((0, 0, 0), (1, 0, 0), (1, 1, 0), (0, 0, 1), (1, 1, 1)):
            tune("wino_u16", u16)
            tune("wino_v16", v16)
            tune("dw_out16", dw16)
            outs.append(g16net.forward_host(inp.x, inp.timestep, cfg=True))
            f16a.append(_f16a_launches(ctx))
    finally:
        ctx.set_precision(False)
    for o in outs[1:]:
        assert np.array_equal(o, outs[0])
    # no f16 input with every store off; V in f16 feeds the Winograd plane GEMMs,
    # the depthwise outputs every resnet and MixFFN 1x1 after them
    assert f16a[0] == 0 and f16a[1] == 0
    assert f16a[2] > 0 and f16a[3] > f16a[2] and f16a[4] == f16a[2] + f16a[3]


def test_unet_pool_stops_allocating(ctx, gnet):
    """Once the activation pool covers a step's buffer roles, steps allocate nothing
    (a device allocation or growth mid-step would stall the host)."""
    inp = U.unet_input(seed=5006)
    for _ in range(2):
        gnet.forward_host(inp.x, inp.timestep, cfg=True)
    _, held = gnet.memory()
    for _ in range(2):
        gnet.forward_host(inp.x, inp.timestep, cfg=True)
        assert gnet.memory()[1] == held


def test_unet_f16_stored_weights(ctx, params, onet):
    """f16-stored GEMM weights, f32 arithmetic: EXACT reads the weights' f32
    widening, so the step is bit for bit the f32 model's on the rounded weights,
    and within the f32 bar of the oracle; the f16 copy stays beside it for FAST."""
    p16 = {k: v for k, v in params.items()}
    gemm = {s.name for s in U.unet_specs() if s.gemm}
    rounded = {k: (v.astype(np.float16).astype(np.float32) if k in gemm else v) for k, v in p16.items()}
    net16 = UNet(ctx, params, f16_gemm=True)
    inp = U.unet_input(seed=5005)
    got = net16.forward_host(inp.x, inp.timestep, cfg=False)
    net_r = UNet(ctx, rounded)
    assert np.array_equal(got, net_r.forward_host(inp.x, inp.timestep, cfg=False))
    want = oracle.UNet(rounded).forward(inp.x, inp.timestep, cfg=False)
    assert max_abs_rel(got, want) <= TOL
    w, _ = net16.memory()
    w32, _ = net_r.memory()
    assert w32 < w < 1.5 * w32  # the f16 GEMM weights plus their f32 widening


def test_missing_weight_is_a_weights_error(ctx, params):
    broken = dict(params)
    broken.pop("diff_model.down_blocks.1.attentions.0.proj_in.weight")
    with pytest.raises(E.MoebiusError) as ei:
        UNet(ctx, broken)
    assert ei.value.code == 2 and "proj_in.weight" in ei.value.msg
