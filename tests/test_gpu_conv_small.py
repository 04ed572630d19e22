"""The direct 3x3 conv for a handful of output channels (conv_small.hip: the
reference's Conv3x3, src/engine/conv.rs:60-102, where c_out <= 8, as the VAE
decoder's 128 -> 3 image conv) against the oracle's conv at the f32 bar, with
and without the GroupNorm+SiLU prologue (padding stays 0), f32 and f16
weights, channel counts that are not a multiple of the 16-channel chunk, odd
map sizes with partial 16x16 tiles; and a map below the kernel's 65536-pixel
threshold, which the implicit GEMM takes, against the same oracle."""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from moebius_cpu_amd import engine as E
from tests.util import max_abs_rel, rel_l2

pytestmark = pytest.mark.gpu
F32_TOL = 1e-4


@pytest.fixture(scope="module")
def ctx():
    c = E.Context(0)
    yield c
    c.synchronize()
    c.close()


def conv3(ctx, x, w, b, prologue=None, f16=False):
    co, ci = w.shape[0], w.shape[3]
    conv = E.Conv3x3(ctx, ci, co, E.Param(ctx, w, f16=f16), b)
    out = E.Tensor(ctx)
    conv.forward_prologue(E.Tensor.from_numpy(ctx, x), prologue, out)
    return out.numpy()


CASES = [(1, 257, 300, 128, 3, False, False), (1, 257, 300, 128, 3, True, False), (2, 181, 200, 20, 8, True, True),
         (1, 256, 256, 4, 1, False, True), (1, 300, 222, 36, 5, True, False), (1, 100, 100, 64, 3, True, False)]


@pytest.mark.parametrize("n,h,w,ci,co,pro,f16", CASES)
def test_small_channel_conv_matches_the_oracle(ctx, n, h, w, ci, co, pro, f16):
    rng = np.random.default_rng(ci * 31 + co + h)
    x = (rng.standard_normal((n, h, w, ci)) * 2 + 0.5).astype(np.float32)
    wt = (rng.standard_normal((co, 3, 3, ci)) * np.sqrt(2.0 / (9 * ci))).astype(np.float32)
    b = (rng.standard_normal(co) * 0.02).astype(np.float32)
    wr = wt.astype(np.float16).astype(np.float32) if f16 else wt
    print(f"small conv {n}x{h}x{w} {ci}->{co} prologue={pro} f16={f16}", flush=True)
    if pro:
        groups = 4 if ci % 4 == 0 else 1
        gamma = (1 + 0.1 * rng.standard_normal(ci)).astype(np.float32)
        beta = (0.1 * rng.standard_normal(ci)).astype(np.float32)
        aff = E.GroupNorm(ctx, groups, 1e-6, gamma, beta).affine(E.Tensor.from_numpy(ctx, x), None, True)
        sc, sh = oracle.group_norm_affine(x, groups, 1e-6, gamma, beta)
        got = conv3(ctx, x, wt, b, prologue=aff, f16=f16)
        want = oracle.conv3x3(x, wr, b, prologue=(sc, sh, True))
    else:
        got = conv3(ctx, x, wt, b, f16=f16)
        want = oracle.conv3x3(x, wr, b)
    assert got.shape == (n, h, w, co)
    assert max_abs_rel(got, want) <= F32_TOL and rel_l2(got, want) <= 5e-6
