"""The Winograd F(2x2,3x3) conv in one kernel (winograd_fused.hip: input
transform, the 16 plane products and the output transform of a 32-tile x
64-channel block kept on chip) against the oracle's conv (src/engine/
winograd.rs:48-120) at the f32 bar and against the three-kernel path
(transforms + batched GEMM; tuning "wino_fused" 0): odd sizes with partial
tiles, batch 2, the nearest-2x upsample, the GroupNorm prologue, the VAE's
and the UNet's channel counts, and shapes the kernel does not take (they fall
back), and maps with several work items per workgroup. The transforms restate the reference's operation order in both paths;
only the plane products' summation order differs."""
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


def conv(ctx, x, w, b, up=False, prologue=None, fused=True):
    co, ci = w.shape[0], w.shape[3]
    ctx.set_tuning("wino_fused", "1" if fused else "0")  # 1: wherever it fits
    try:
        cv = E.Conv3x3(ctx, ci, co, E.Param(ctx, w), b, upsample2x=up, winograd=True)
        out = E.Tensor(ctx)
        cv.forward_prologue(E.Tensor.from_numpy(ctx, x), prologue, out)
        return out.numpy()
    finally:
        ctx.set_tuning("wino_fused", None)


SHAPES = [(2, 9, 11, 64, 64, False), (1, 7, 5, 32, 64, True), (1, 64, 64, 128, 128, False),
          (1, 32, 32, 512, 512, False), (1, 24, 40, 256, 128, True), (2, 16, 16, 640, 640, True),
          (1, 8, 8, 1280, 1280, True), (1, 9, 7, 48, 64, False), (1, 9, 7, 64, 40, True),
          # several work items per workgroup (one workgroup per CU), partial last tile block
          (1, 200, 180, 32, 128, False), (1, 130, 250, 64, 64, True)]


@pytest.mark.parametrize("n,h,w,ci,co,up", SHAPES)
def test_fused_conv_matches_oracle_and_the_three_kernel_path(ctx, n, h, w, ci, co, up):
    rng = np.random.default_rng(ci * 7 + co + h)
    x = rng.standard_normal((n, h, w, ci)).astype(np.float32)
    wt = (rng.standard_normal((co, 3, 3, ci)) * np.sqrt(2.0 / (9 * ci))).astype(np.float32)
    b = (rng.standard_normal(co) * 0.02).astype(np.float32)
    print(f"wino fused {n}x{h}x{w} {ci}->{co} up={up}", flush=True)
    got = conv(ctx, x, wt, b, up, fused=True)
    want = oracle.conv3x3(x, wt, b, upsample2x=up)
    assert max_abs_rel(got, want) <= TOL
    three = conv(ctx, x, wt, b, up, fused=False)
    assert np.abs(got - three).max() <= 1e-5 * np.abs(three).max()
    assert np.array_equal(got, conv(ctx, x, wt, b, up, fused=True))  # deterministic


def test_fused_conv_gn_prologue(ctx):
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((2, 7, 9, 64)) * 3 + 1).astype(np.float32)
    wt = (rng.standard_normal((64, 3, 3, 64)) * 0.05).astype(np.float32)
    gamma = (1 + 0.1 * rng.standard_normal(64)).astype(np.float32)
    beta = (0.1 * rng.standard_normal(64)).astype(np.float32)
    aff = E.GroupNorm(ctx, 32, 1e-6, gamma, beta).affine(E.Tensor.from_numpy(ctx, x), None, True)
    got = conv(ctx, x, wt, None, prologue=aff)
    sc, sh = oracle.group_norm_affine(x, 32, 1e-6, gamma, beta)
    want = oracle.conv3x3(x, wt, None, prologue=(sc, sh, True))
    assert max_abs_rel(got, want) <= TOL
