"""GPU parity of the Winograd F(2x2,3x3) conv (src/engine/winograd.rs), through
the C ABI: the kernel, input and output transforms bit for bit against the
oracle (they restate the reference's operation order), the whole conv against
the oracle at the f32 bar (max-abs <= 1e-4 * max|ref|), odd sizes (partial
tiles), the nearest-2x upsample and the GroupNorm prologue included, and in
FAST precision at the f16 bar (2e-2)."""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from moebius_cpu_amd import engine as E
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


@pytest.mark.parametrize("co,ci,f16", [(12, 8, False), (40, 64, False), (24, 20, True)])
def test_kernel_transform_bit_exact(ctx, co, ci, f16):
    rng = np.random.default_rng(co + ci)
    w = rng.standard_normal((co, 3, 3, ci)).astype(np.float32)
    p = E.Param(ctx, w, f16=f16)
    u = E.DeviceArray(ctx, (16, co, ci))
    E.check(E.lib().mh_winograd_weight_transform(ctx.h, p.ptr, p.dtype, co, ci, u.ptr))
    w_eff = w.astype(np.float16).astype(np.float32) if f16 else w  # f16 widened exactly first
    assert np.array_equal(u.numpy(), oracle.wino_kernel_transform(w_eff))


@pytest.mark.parametrize("n,h,w,c,up,pro", [(2, 5, 7, 8, False, False), (1, 4, 6, 16, True, False),
                                            (2, 9, 3, 64, False, True), (1, 3, 5, 32, True, True)])
def test_input_transform_bit_exact(ctx, n, h, w, c, up, pro):
    rng = np.random.default_rng(h * w + c)
    x = rng.standard_normal((n, h, w, c)).astype(np.float32)
    sc = (1 + 0.1 * rng.standard_normal(n * c)).astype(np.float32)
    sh = (0.1 * rng.standard_normal(n * c)).astype(np.float32)
    tiles = oracle.wino_tiles(n, h, w, up)
    v = E.DeviceArray(ctx, (16, tiles, c))
    scd, shd = D(ctx, sc), D(ctx, sh)
    E.check(E.lib().mh_winograd_input_transform(ctx.h, D(ctx, x).ptr, n, h, w, c, int(up),
                                                scd.ptr if pro else None, shd.ptr if pro else None, 1, v.ptr))
    want = oracle.wino_input_transform(x, up, (sc, sh, True) if pro else None)
    assert np.array_equal(v.numpy(), want)


@pytest.mark.parametrize("n,h,w,co,up,bias", [(2, 5, 7, 8, False, True), (1, 3, 3, 16, True, False),
                                              (1, 6, 4, 12, False, True)])
def test_output_transform_bit_exact(ctx, n, h, w, co, up, bias):
    rng = np.random.default_rng(co * 3 + h)
    tiles = oracle.wino_tiles(n, h, w, up)
    m = rng.standard_normal((16, tiles, co)).astype(np.float32)
    b = rng.standard_normal(co).astype(np.float32) if bias else None
    hu, wu = (2 * h, 2 * w) if up else (h, w)
    out = D(ctx, np.zeros((n, hu, wu, co), np.float32))
    bd = D(ctx, b) if bias else None
    E.check(E.lib().mh_winograd_output_transform(ctx.h, D(ctx, m).ptr, n, h, w, co, int(up),
                                                 bd.ptr if bias else None, out.ptr))
    assert np.array_equal(out.numpy(), oracle.wino_output_transform(m, n, h, w, up, b))


def wconv(ctx, x, w, b, up=False, prologue=None, f16=False):
    co, ci = w.shape[0], w.shape[3]
    conv = E.Conv3x3(ctx, ci, co, E.Param(ctx, w, f16=f16), b, upsample2x=up, winograd=True)
    out = E.Tensor(ctx)
    conv.forward_prologue(E.Tensor.from_numpy(ctx, x), prologue, out)
    return out.numpy()


@pytest.mark.parametrize("n,h,w,ci,co,up", [(2, 9, 11, 64, 48, False), (1, 7, 5, 32, 20, True),
                                            (2, 16, 16, 320, 320, False), (1, 8, 8, 1280, 1280, True),
                                            (2, 16, 16, 640, 640, True),
                                            (1, 64, 64, 320, 320, False)])  # the 64x64x320 conv bench.py times
def test_winograd_conv_matches_oracle(ctx, n, h, w, ci, co, up):
    rng = np.random.default_rng(ci + co + h)
    x = rng.standard_normal((n, h, w, ci)).astype(np.float32)
    wt = (rng.standard_normal((co, 3, 3, ci)) * np.sqrt(2.0 / (9 * ci))).astype(np.float32)
    b = (rng.standard_normal(co) * 0.02).astype(np.float32)
    got = wconv(ctx, x, wt, b, up)
    assert max_abs_rel(got, oracle.conv3x3(x, wt, b, upsample2x=up)) <= TOL


def test_winograd_conv_gn_prologue(ctx):
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((2, 7, 9, 64)) * 3 + 1).astype(np.float32)
    wt = (rng.standard_normal((32, 3, 3, 64)) * 0.05).astype(np.float32)
    gamma = (1 + 0.1 * rng.standard_normal(64)).astype(np.float32)
    beta = (0.1 * rng.standard_normal(64)).astype(np.float32)
    aff = E.GroupNorm(ctx, 32, 1e-6, gamma, beta).affine(E.Tensor.from_numpy(ctx, x), None, True)
    got = wconv(ctx, x, wt, None, prologue=aff)
    sc, sh = oracle.group_norm_affine(x, 32, 1e-6, gamma, beta)
    want = oracle.conv3x3(x, wt, None, prologue=(sc, sh, True))
    assert max_abs_rel(got, want) <= TOL


def test_winograd_conv_fast_precision(ctx):
    rng = np.random.default_rng(11)
    x = rng.standard_normal((2, 16, 16, 320)).astype(np.float32)
    wt = (rng.standard_normal((320, 3, 3, 320)) * np.sqrt(2.0 / 2880)).astype(np.float32)
    b = (rng.standard_normal(320) * 0.02).astype(np.float32)
    ctx.set_precision(True)
    try:
        got = wconv(ctx, x, wt, b, up=True, f16=True)
    finally:
        ctx.set_precision(False)
    assert max_abs_rel(got, oracle.conv3x3(x, wt, b, upsample2x=True)) <= 2e-2


def test_winograd_rejects_strided_or_padded_convs(ctx):
    w = np.zeros((8, 3, 3, 8), np.float32)
    with pytest.raises(E.MoebiusError):
        E.Conv3x3(ctx, 8, 8, E.Param(ctx, w), None, stride=2, winograd=True)
