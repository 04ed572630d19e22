"""GPU parity at the benchmark workloads' full sizes, through the C ABI,
against the oracle on identical seeded inputs (max-abs <= 1e-4 * max|ref| for
f32; the depthwise and GroupNorm-apply kernels restate the CPU arithmetic and
are compared bit for bit where their inputs are identical)."""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from moebius_cpu_amd import engine as E
from moebius_cpu_amd import workloads as W
from tests.util import max_abs_rel

pytestmark = pytest.mark.gpu
TOL = 1e-4


@pytest.fixture(scope="module")
def ctx():
    c = E.Context(0)
    yield c
    c.synchronize()
    c.close()


def T(ctx, a):
    return E.Tensor.from_numpy(ctx, a)


def test_conv3x3_gn_silu_64x64x320(ctx):
    wl = W.conv3x3_gn_silu()
    conv = E.Conv3x3.same(ctx, 320, 320, E.Param(ctx, wl.w), wl.b)
    y, z = E.Tensor(ctx), E.Tensor(ctx)
    conv.forward(T(ctx, wl.x), y)
    E.GroupNorm(ctx, wl.groups, wl.eps, wl.gamma, wl.beta).forward(y, None, True, z)
    ref_y = oracle.conv3x3(wl.x, wl.w, wl.b)
    ref_z = oracle.group_norm(ref_y, wl.groups, wl.eps, wl.gamma, wl.beta, silu=True)
    assert max_abs_rel(y.numpy(), ref_y) <= TOL
    assert max_abs_rel(z.numpy(), ref_z) <= TOL
    # GN+SiLU on the same (device) conv output is the reference arithmetic to f64 rounding
    z2 = oracle.group_norm(y.numpy(), wl.groups, wl.eps, wl.gamma, wl.beta, silu=True)
    assert max_abs_rel(z.numpy(), z2) <= 1e-6


@pytest.mark.parametrize("s,c", W.SWEEP)
@pytest.mark.parametrize("f16", [False, True])
def test_kernel_sweep(ctx, s, c, f16):
    p = W.sweep_point(s, c)
    x = T(ctx, p.x)
    # 1x1 conv-as-GEMM C -> C (f16: stored f16, widened exactly)
    w_eff = p.w1.astype(np.float16).astype(np.float32) if f16 else p.w1
    out = E.Tensor(ctx)
    E.Conv1x1(ctx, c, c, E.Param(ctx, p.w1, f16=f16), p.b1).forward(x, out)
    assert max_abs_rel(out.numpy(), oracle.conv1x1(p.x, w_eff, p.b1)) <= TOL
    # depthwise 3x3 (f32 weights in every mode, as the reference)
    E.depthwise3x3(x, p.dw_w, p.dw_b, "none", out)
    assert np.array_equal(out.numpy(), oracle.depthwise3x3(p.x, p.dw_w, p.dw_b, "none"))
    # GroupNorm(32) + SiLU
    E.GroupNorm(ctx, 32, 1e-5, p.gamma, p.beta).forward(x, None, True, out)
    assert max_abs_rel(out.numpy(), oracle.group_norm(p.x, 32, 1e-5, p.gamma, p.beta, silu=True)) <= 1e-6
    # broadcast bias + residual add: (r + b) + x
    E.bias_residual_add(x, p.bias, T(ctx, p.residual), out)
    pre, _ = oracle.init_output(s * s, c, p.bias, p.residual.reshape(-1, c))
    assert np.array_equal(out.numpy().reshape(-1, c), oracle.add(pre, p.x.reshape(-1, c)))


def _resnet_gpu(ctx, wl: W.ResnetBlock, winograd=True):
    """The device chain bench.py times (workloads.ResnetBlockGpu), run twice: a
    second call on the same buffers gives the same bits."""
    blk = W.ResnetBlockGpu(ctx, wl, winograd=winograd)
    first = blk.forward().numpy()
    assert np.array_equal(blk.forward().numpy(), first)
    return first


def _resnet_oracle(wl: W.ResnetBlock):
    sc, sh = oracle.group_norm_affine(wl.x, 32, wl.eps, wl.gn1_g, wl.gn1_b)
    h = oracle.conv3x3(wl.x, wl.w1, wl.b1, prologue=(sc, sh, True))
    tp = oracle.conv1x1(oracle.silu(wl.temb).reshape(1, 1, 1, -1), wl.lin_w, wl.lin_b).reshape(-1)
    sc2, sh2 = oracle.group_norm_affine(h, 32, wl.eps, wl.gn2_g, wl.gn2_b, add=tp)
    out = oracle.conv3x3(h, wl.w2, wl.b2, prologue=(sc2, sh2, True))
    return oracle.conv1x1(wl.x, wl.ws, wl.bs, residual=out)


@pytest.mark.parametrize("winograd", [True, False])
def test_resnet_block_32x32_320_to_640(ctx, winograd):
    wl = W.resnet_block()
    got = _resnet_gpu(ctx, wl, winograd)
    want = _resnet_oracle(wl)
    assert max_abs_rel(got, want) <= TOL


def test_resnet_block_matches_unfused_composition(ctx):
    """The GN prologue + folded temb add equal materialising GN(h + tp) first."""
    wl = W.resnet_block(seed=3100, s=16, c_in=64, c_out=128, temb_dim=256)
    got = _resnet_gpu(ctx, wl)
    tp = oracle.conv1x1(oracle.silu(wl.temb).reshape(1, 1, 1, -1), wl.lin_w, wl.lin_b).reshape(-1)
    a = oracle.group_norm(wl.x, 32, wl.eps, wl.gn1_g, wl.gn1_b, silu=True)
    h = oracle.conv3x3(a, wl.w1, wl.b1, im2col=True)
    a2 = oracle.group_norm(h + tp[None, None, None, :], 32, wl.eps, wl.gn2_g, wl.gn2_b, silu=True)
    out = oracle.conv3x3(a2, wl.w2, wl.b2, im2col=True)
    want = oracle.conv1x1(wl.x, wl.ws, wl.bs) + out
    assert max_abs_rel(got, want) <= TOL
