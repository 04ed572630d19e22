"""Pins the CPU oracle's engine kernels to the reference's own vectors and to
mathematics. Restates moebius-cpu tests/kernels.rs (fixtures, f64 brute force,
Winograd == im2col, GN prologue == GN then conv) and the in-module tests of
src/engine/{math,gemm,tensor}.rs and src/imaging/blend.rs, then adds closed
forms and a torch fp32 cross-check. CPU only."""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from tests.util import Lcg, assert_close, fixtures, hashed, rel_l2


@pytest.fixture(scope="module")
def fx():
    return fixtures()


# ---- tests/kernels.rs:40-51
def test_conv1x1_bias_and_residual(fx):
    x, w, b, r = fx["c1.x"], fx["c1.w"], fx["c1.b"], fx["c1.r"]
    assert_close(oracle.conv1x1(x, w, b), fx["c1.y"], 1e-5)
    assert_close(oracle.conv1x1(x, w, b, r), fx["c1.yr"], 1e-5)


# ---- tests/kernels.rs:65-84
@pytest.mark.parametrize("name,stride,pad,up", [
    ("c3.same", 1, (1, 1, 1, 1), False),
    ("c3.s2p1", 2, (1, 1, 1, 1), False),
    ("c3.s2vae", 2, (0, 0, 1, 1), False),
    ("c3.up", 1, (1, 1, 1, 1), True),
])
def test_conv3x3_variants(fx, name, stride, pad, up):
    out = oracle.conv3x3(fx["c3.x"], fx["c3.w"], fx["c3.b"], stride=stride, pad=pad, upsample2x=up)
    assert_close(out, fx[name], 1e-5)


# ---- tests/kernels.rs:86-116 (f64 direct definition across im2col bands)
def test_conv3x3_band_boundaries():
    n, h, w, c = 1, 40, 30, 1024
    x = hashed(n * h * w * c, 7919, 211, 211.0, 0.5).reshape(n, h, w, c)
    wt = (((np.arange(2 * 9 * c, dtype=np.int64) * 104_729) % 97).astype(np.float32) / np.float32(970.0)
          - np.float32(0.05)).astype(np.float32).reshape(2, 3, 3, c)
    out = oracle.conv3x3(x, wt, None)
    xp = np.zeros((h + 2, w + 2, c), np.float64)
    xp[1:-1, 1:-1] = x[0]
    want = np.zeros((1, h, w, 2), np.float64)
    for ky in range(3):
        for kx in range(3):
            want[0] += xp[ky:ky + h, kx:kx + w] @ wt[:, ky, kx, :].astype(np.float64).T
    assert_close(out, want.astype(np.float32), 2e-5)
    # the same through the im2col path (bands of 910 pixels)
    assert_close(oracle.conv3x3(x, wt, None, im2col=True), want.astype(np.float32), 2e-5)


# ---- tests/kernels.rs:118-128
def test_depthwise_epilogues(fx):
    x, w, b = fx["dw.x"], fx["dw.w"], fx["dw.b"]
    assert_close(oracle.depthwise3x3(x, w, b, "relu"), fx["dw.relu"], 1e-5)
    assert_close(oracle.depthwise3x3(x, w, b, "glu_silu"), fx["dw.glu"], 1e-5)


# ---- tests/kernels.rs:130-141
def test_group_norm_plain_and_fused(fx):
    x, g, b, add = fx["gn.x"], fx["gn.gamma"], fx["gn.beta"], fx["gn.add"]
    assert_close(oracle.group_norm(x, 32, 1e-6, g, b), fx["gn.y"], 1e-5)
    assert_close(oracle.group_norm(x, 32, 1e-5, g, b, add=add.reshape(-1), silu=True), fx["gn.y_add_silu"], 1e-5)


# ---- tests/kernels.rs:143-151
def test_layer_norm_tokens(fx):
    assert_close(oracle.layer_norm(fx["ln.x"], fx["ln.gamma"], fx["ln.beta"], 1e-5), fx["ln.y"], 1e-5)


# ---- tests/kernels.rs:153-170 (Winograd == im2col, odd sizes, f16 weights, upsample, big c_out)
@pytest.mark.parametrize("n,h,w,ci,co,up", [(2, 37, 23, 24, 40, False), (1, 9, 13, 16, 8, True),
                                            (1, 6, 5, 768, 720, False)])
def test_winograd_matches_direct_on_multiband_odd_sizes(n, h, w, ci, co, up):
    x = hashed(n * h * w * ci, 7919, 401, 401.0, 0.5).reshape(n, h, w, ci)
    wt = (((np.arange(co * 9 * ci, dtype=np.int64) * 104_729) % 113).astype(np.float32) / np.float32(1130.0)
          - np.float32(0.05)).astype(np.float32)
    wt = wt.astype(np.float16).astype(np.float32).reshape(co, 3, 3, ci)  # Param::f16_from then widened
    b = (np.arange(co, dtype=np.float32) * np.float32(0.01)).astype(np.float32)
    fast = oracle.conv3x3(x, wt, b, upsample2x=up)
    direct = oracle.conv3x3(x, wt, b, upsample2x=up, im2col=True)
    assert_close(fast, direct, 2e-5)


# ---- tests/kernels.rs:172-213 (f64 definition, all epilogues, odd widths, channel tails)
@pytest.mark.parametrize("h,w,c,ep", [(5, 7, 64, "relu"), (4, 9, 70, "none"), (3, 5, 140, "glu_silu"),
                                      (2, 4, 64, "glu_silu")])
def test_depthwise_register_blocks_and_tails(h, w, c, ep):
    x = hashed(h * w * c, 7919, 211, 211.0, 0.5).reshape(1, h, w, c)
    wt = hashed(9 * c, 31, 17, 17.0, 0.5).reshape(3, 3, c)
    b = (np.arange(c, dtype=np.float32) * np.float32(0.01) - np.float32(0.2)).astype(np.float32)
    out = oracle.depthwise3x3(x, wt, b, ep)
    xp = np.zeros((h + 2, w + 2, c), np.float64)
    xp[1:-1, 1:-1] = x[0]
    y = np.broadcast_to(b.astype(np.float64), (h, w, c)).copy()
    for ky in range(3):
        for kx in range(3):
            y += xp[ky:ky + h, kx:kx + w] * wt[ky, kx].astype(np.float64)
    if ep == "relu":
        want = np.maximum(y, 0.0)
    elif ep == "none":
        want = y
    else:
        half = c // 2
        g = y[..., half:]
        want = y[..., :half] * g / (1.0 + np.exp(-g))
    assert_close(out, want[None].astype(np.float32), 1e-5)


# ---- tests/kernels.rs:233-265 (GN(+SiLU) prologue == GN then conv; padding stays 0)
@pytest.mark.parametrize("n,h,w,ci,groups,co", [(2, 7, 9, 40, 8, 24), (2, 37, 23, 768, 32, 16)])
@pytest.mark.parametrize("up", [False, True])
def test_winograd_prologue_matches_group_norm_then_conv(n, h, w, ci, groups, co, up):
    rnd = Lcg(7 + ci)
    x = (rnd.take(n * h * w * ci) * np.float32(3.0) + np.float32(0.7)).reshape(n, h, w, ci)
    gamma = np.float32(1.0) + np.float32(0.5) * rnd.take(ci)
    beta = rnd.take(ci)
    wt = (rnd.take(co * 9 * ci) * np.float32(0.05)).astype(np.float16).astype(np.float32).reshape(co, 3, 3, ci)
    bias = (np.arange(co, dtype=np.float32) * np.float32(0.01)).astype(np.float32)
    a = oracle.group_norm(x, groups, 1e-6, gamma, beta, silu=True)
    want = oracle.conv3x3(a, wt, bias, upsample2x=up)
    sc, sh = oracle.group_norm_affine(x, groups, 1e-6, gamma, beta)
    got = oracle.conv3x3(x, wt, bias, upsample2x=up, prologue=(sc, sh, True))
    assert rel_l2(got, want) <= 1e-6


# ---- src/engine/math.rs:42-65
def test_exp_matches_f64():
    import ctypes

    xs = np.arange(-87.0, 88.0, 0.0137, dtype=np.float64).astype(np.float32)
    f = oracle.lib().orc_exp
    got = np.array([f(ctypes.c_float(v)) for v in xs], np.float64)
    want = np.exp(xs.astype(np.float64))
    assert np.max(np.abs((got - want) / want)) < 3e-7
    assert oracle.exp(-1000.0) == oracle.exp(-87.33655)
    assert np.isfinite(oracle.exp(1000.0))


def test_silu_matches_definition():
    xs = (np.arange(-2000, 2000, dtype=np.float32) * np.float32(0.01)).astype(np.float32)
    got = oracle.silu(xs).astype(np.float64)
    x64 = xs.astype(np.float64)
    want = x64 / (1.0 + np.exp(-x64))
    assert np.all(np.abs(got - want) <= 1e-6 * (1.0 + np.abs(want)))
    assert abs(oracle.silu_scalar(-200.0)) < 1e-30
    assert oracle.silu_scalar(200.0) == 200.0
    assert oracle.silu_scalar(0.0) == 0.0


# ---- src/engine/gemm.rs:139-187
def test_matmul_matches_naive_both_layouts():
    m, k, n = 7, 5, 3
    a = np.sin(np.arange(m * k, dtype=np.float32) * np.float32(0.37)).reshape(m, k).astype(np.float32)
    w = np.cos(np.arange(n * k, dtype=np.float32) * np.float32(0.11)).reshape(n, k).astype(np.float32)
    want = a.astype(np.float64) @ w.astype(np.float64).T
    got = oracle.matmul(a, w.T)
    assert np.max(np.abs(got - want)) < 1e-5
    oracle.matmul(a, w.T, got, accumulate=True)
    assert np.max(np.abs(got - 2 * want)) < 1e-5


def test_matmul_strided_operands_accumulate():
    m, k, n, planes = 67, 129, 45, 3
    a_buf = (((np.arange(m * planes * k, dtype=np.int64) * 37) % 101).astype(np.float32) / np.float32(101.0)
             - np.float32(0.5))
    w = (((np.arange(n * k, dtype=np.int64) * 53) % 97).astype(np.float32) / np.float32(97.0) - np.float32(0.5))
    w = w.reshape(n, k)
    a = a_buf.reshape(m, planes, k)[:, 1, :]  # plane 1 of 3: row stride planes*k
    want = a.astype(np.float64) @ w.astype(np.float64).T
    got = np.full((m, n), 0.5, np.float32)
    oracle.matmul(a, w.T, got, accumulate=True)
    assert np.max(np.abs(got - (want + 0.5))) < 1e-4
    oracle.matmul(a, w.T, got, accumulate=False)
    assert np.max(np.abs(got - want)) < 1e-4
    # transposed A (keys^T in softmax_lambda, src/unet/lambda.rs:353) and large k past one block
    k2 = 700
    at = np.sin(np.arange(k2 * m, dtype=np.float32)).reshape(k2, m).astype(np.float32)
    b2 = np.cos(np.arange(k2 * n, dtype=np.float32)).reshape(k2, n).astype(np.float32)
    got2 = oracle.matmul(at.T, b2)
    assert np.max(np.abs(got2 - at.T.astype(np.float64) @ b2.astype(np.float64))) < 1e-3


# ---- src/engine/tensor.rs:76-97
def test_concat_channels_interleaves_per_pixel():
    a = np.array([1, 2, 3, 4], np.float32).reshape(1, 1, 2, 2)
    b = np.array([10, 20, 30, 40, 50, 60], np.float32).reshape(1, 1, 2, 3)
    c = oracle.concat_channels(a, b)
    assert c.shape == (1, 1, 2, 5)
    assert c.reshape(-1).tolist() == [1, 2, 10, 20, 30, 3, 4, 40, 50, 60]


# ---- src/imaging/blend.rs:228-236
def test_to_u8_truncates_and_clamps():
    v = np.array([0.99999, 1.2, -0.1, 0.5, 1.0, 0.0, np.nan], np.float32)
    assert oracle.to_u8(v).tolist() == [254, 255, 0, 127, 255, 0, 0]


# ---- src/engine/conv.rs:170-191 (the cfg "broadcast bias + residual add" prefill)
def test_init_output_cases():
    r = np.arange(12, dtype=np.float32).reshape(3, 4)
    b = np.array([0.5, -1.0, 2.0, 0.25], np.float32)
    out, acc = oracle.init_output(3, 4)
    assert not acc
    out, acc = oracle.init_output(3, 4, bias=b)
    assert acc and np.array_equal(out, np.broadcast_to(b, (3, 4)))
    out, acc = oracle.init_output(3, 4, residual=r)
    assert acc and np.array_equal(out, r)
    out, acc = oracle.init_output(3, 4, bias=b, residual=r)
    assert acc and np.array_equal(out, r + b)


# ---- closed forms that pin what the fixtures leave open
def test_group_norm_closed_form_moments():
    """gamma=1, beta=0, no add/SiLU: each (item, group) slice has mean 0 and
    biased variance var/(var+eps)."""
    rng = np.random.default_rng(3)
    n, h, w, c, g, eps = 2, 13, 11, 96, 32, 1e-5
    x = (rng.standard_normal((n, h, w, c)) * 2.5 + 0.3).astype(np.float32)
    y = oracle.group_norm(x, g, eps, np.ones(c, np.float32), np.zeros(c, np.float32)).astype(np.float64)
    xs = x.reshape(n, h * w, g, c // g).astype(np.float64)
    ys = y.reshape(n, h * w, g, c // g)
    var = xs.var(axis=(1, 3))
    assert np.max(np.abs(ys.mean(axis=(1, 3)))) < 1e-6
    assert np.max(np.abs(ys.var(axis=(1, 3)) - var / (var + np.float64(np.float32(eps))))) < 1e-5


def test_group_norm_add_folds_into_shift():
    """GN(x + add) through the add argument equals GN of the materialised sum."""
    rng = np.random.default_rng(4)
    n, h, w, c = 2, 9, 7, 64
    x = rng.standard_normal((n, h, w, c)).astype(np.float32)
    add = rng.standard_normal((n, c)).astype(np.float32)
    gm = rng.standard_normal(c).astype(np.float32)
    bt = rng.standard_normal(c).astype(np.float32)
    got = oracle.group_norm(x, 32, 1e-5, gm, bt, add=add.reshape(-1))
    want = oracle.group_norm(x + add[:, None, None, :], 32, 1e-5, gm, bt)
    assert_close(got, want, 2e-6)


def test_conv_integer_inputs_bit_exact():
    """Small-integer activations and even-integer weights keep every partial sum
    an exact f32 integer (< 2^24): Winograd, im2col and the f64 definition agree
    bit for bit, and a transposed or shifted tap would not."""
    rng = np.random.default_rng(5)
    n, h, w, ci, co = 2, 11, 9, 24, 20
    x = rng.integers(-3, 4, (n, h, w, ci)).astype(np.float32)
    wt = (2 * rng.integers(-2, 3, (co, 3, 3, ci))).astype(np.float32)
    b = rng.integers(-5, 6, co).astype(np.float32)
    wino = oracle.conv3x3(x, wt, b)
    direct = oracle.conv3x3(x, wt, b, im2col=True)
    xp = np.zeros((n, h + 2, w + 2, ci), np.float64)
    xp[:, 1:-1, 1:-1] = x
    want = np.broadcast_to(b.astype(np.float64), (n, h, w, co)).copy()
    for ky in range(3):
        for kx in range(3):
            want += xp[:, ky:ky + h, kx:kx + w] @ wt[:, ky, kx, :].astype(np.float64).T
    assert np.array_equal(wino, want.astype(np.float32))
    assert np.array_equal(direct, want.astype(np.float32))


def test_torch_fp32_cross_check():
    """Independent library routine (torch CPU, fp32) on shapes the fixtures do
    not cover: 3x3 same/stride-2/upsample, depthwise, group norm, layer norm."""
    torch = pytest.importorskip("torch")
    F = torch.nn.functional
    rng = np.random.default_rng(6)
    x = rng.standard_normal((2, 16, 12, 64)).astype(np.float32)
    w = (rng.standard_normal((48, 3, 3, 64)) * 0.05).astype(np.float32)
    b = rng.standard_normal(48).astype(np.float32)
    xt = torch.from_numpy(x).permute(0, 3, 1, 2)
    wt = torch.from_numpy(w).permute(0, 3, 1, 2)
    bt = torch.from_numpy(b)

    def nhwc(t):
        return t.permute(0, 2, 3, 1).contiguous().numpy()

    assert_close(oracle.conv3x3(x, w, b), nhwc(F.conv2d(xt, wt, bt, padding=1)), 2e-5)
    assert_close(oracle.conv3x3(x, w, b, stride=2), nhwc(F.conv2d(xt, wt, bt, stride=2, padding=1)), 2e-5)
    assert_close(oracle.conv3x3(x, w, b, stride=2, pad=(0, 0, 1, 1)),
                 nhwc(F.conv2d(F.pad(xt, (0, 1, 0, 1)), wt, bt, stride=2)), 2e-5)
    assert_close(oracle.conv3x3(x, w, b, upsample2x=True),
                 nhwc(F.conv2d(F.interpolate(xt, scale_factor=2.0, mode="nearest"), wt, bt, padding=1)), 2e-5)
    dw = (rng.standard_normal((3, 3, 64)) * 0.3).astype(np.float32)
    db = rng.standard_normal(64).astype(np.float32)
    y = F.conv2d(xt, torch.from_numpy(dw).permute(2, 0, 1)[:, None], torch.from_numpy(db), padding=1, groups=64)
    assert_close(oracle.depthwise3x3(x, dw, db, "none"), nhwc(y), 1e-5)
    a, g = y.chunk(2, dim=1)
    assert_close(oracle.depthwise3x3(x, dw, db, "glu_silu"), nhwc(a * F.silu(g)), 1e-5)
    gm = rng.standard_normal(64).astype(np.float32)
    be = rng.standard_normal(64).astype(np.float32)
    gn = F.group_norm(xt, 32, torch.from_numpy(gm), torch.from_numpy(be), eps=1e-5)
    assert_close(oracle.group_norm(x, 32, 1e-5, gm, be, silu=True), nhwc(F.silu(gn)), 1e-5)
    ln = F.layer_norm(torch.from_numpy(x), (64,), torch.from_numpy(gm), torch.from_numpy(be), eps=1e-5)
    assert_close(oracle.layer_norm(x, gm, be, 1e-5), ln.numpy(), 1e-5)


@pytest.mark.parametrize("n,h,w,ci,co,up", [(2, 5, 7, 8, 12, False), (1, 4, 3, 6, 5, True), (1, 1, 1, 4, 3, False)])
def test_winograd_transforms_compose_to_the_direct_conv(n, h, w, ci, co, up):
    """The whole-map kernel, input and output transforms (src/engine/winograd.rs:
    254-352) composed through an f64 product equal the f64 direct conv, odd
    sizes (partial tiles) and the nearest-2x upsample included; and they are the
    same values the oracle's own Winograd conv uses."""
    from tests import ref_f64 as R

    rng = np.random.default_rng(n * 100 + h * 10 + w)
    x = rng.standard_normal((n, h, w, ci)).astype(np.float32)
    wt = rng.standard_normal((co, 3, 3, ci)).astype(np.float32)
    b = rng.standard_normal(co).astype(np.float32)
    u = oracle.wino_kernel_transform(wt)
    v = oracle.wino_input_transform(x, up)
    assert u.shape == (16, co, ci) and v.shape == (16, oracle.wino_tiles(n, h, w, up), ci)
    m = np.einsum("xtc,xoc->xto", v.astype(np.float64), u.astype(np.float64)).astype(np.float32)
    y = oracle.wino_output_transform(m, n, h, w, up, b)
    direct = R.conv3x3(x.astype(np.float64), wt.astype(np.float64), b.astype(np.float64), up=up)
    assert np.max(np.abs(y - direct)) <= 1e-5 * max(1.0, np.max(np.abs(direct)))
    assert np.max(np.abs(y - oracle.conv3x3(x, wt, b, upsample2x=up))) <= 1e-5 * max(1.0, np.max(np.abs(direct)))
    # integer inputs with even-integer weights: every transform and sum is exact
    xi = rng.integers(-4, 5, x.shape).astype(np.float32)
    wi = (2 * rng.integers(-3, 4, wt.shape)).astype(np.float32)
    mi = np.einsum("xtc,xoc->xto", oracle.wino_input_transform(xi, up).astype(np.float64),
                   oracle.wino_kernel_transform(wi).astype(np.float64)).astype(np.float32)
    yi = oracle.wino_output_transform(mi, n, h, w, up, None)
    assert np.array_equal(yi, R.conv3x3(xi.astype(np.float64), wi.astype(np.float64), 0.0, up=up).astype(np.float32))
