"""Pins the oracle's UNet restatement (oracle/unet.cpp) to float64 restatements
of the blocks' mathematical definitions (tests/ref_f64.py: the lambda layers
in their unfolded upstream form, the norms and convs from their formulas) and
to invariants of the whole network. CPU only."""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from moebius_cpu_amd import synthetic as S
from moebius_cpu_amd import unet_params as U
from tests import ref_f64 as R
from tests.util import max_abs_rel

TOL = 2e-5  # f32 oracle vs f64 definition, max-abs / max|ref|


def block_params(specs, seed, std=0.05):
    out = {}
    for i, s in enumerate(specs):
        mean = 1.0 if s.kind == "norm_w" else 0.0
        out[s.name] = S.normal(seed * 1000 + i, s.shape, std=std, mean=mean)
    return out


def cond_specs():
    specs = [U.Spec("embedding_layer.weight", (20, U.EHS), "weight", False)]
    U._lin(specs, "diff_model.encoder_hid_proj", U.EHS, U.XDIM)
    return specs


def test_timestep_sinusoid_layout_and_values():
    for t in (1, 17, 442, 999):
        got = oracle.timestep_sinusoid(t).astype(np.float64)
        want = R.timestep_embedding_sinusoid(t)
        # f32 argument rounding: |d arg| <= ~1 ulp(999) = 6.1e-5
        assert np.max(np.abs(got - want)) < 2e-4
        assert np.allclose(got[:160] ** 2 + got[160:] ** 2, 1.0, atol=1e-6)  # [cos | sin] of one argument


def test_softmax_lambda_matches_definition():
    rng = np.random.default_rng(1)
    for rows, k in ((10, 40), (300, 8), (4096, 40)):
        keys = (rng.standard_normal((rows, k)) * 3).astype(np.float32)
        v = rng.standard_normal((rows, k)).astype(np.float32)
        got = oracle.softmax_lambda(keys, v)
        kd = keys.astype(np.float64)
        sk = np.exp(kd - kd.max(axis=0))
        sk /= sk.sum(axis=0)
        assert max_abs_rel(got, sk.T @ v.astype(np.float64)) < 1e-5


def test_tap_filter_window_geometry():
    rng = np.random.default_rng(2)
    hh, ww, vd = 11, 9, 8
    a = rng.standard_normal((hh * ww, 8, 226)).astype(np.float32)
    v = rng.standard_normal((hh * ww, vd)).astype(np.float32)
    o = rng.standard_normal((hh * ww, 8 * vd)).astype(np.float32)
    got = oracle.tap_filter(a, v, o, hh, ww)
    vp = np.zeros((hh + 14, ww + 14, vd))
    vp[7:7 + hh, 7:7 + ww] = v.reshape(hh, ww, vd)
    want = o.astype(np.float64).reshape(hh, ww, 8, vd) + a[..., 225].reshape(hh, ww, 8, 1)
    ar = a.astype(np.float64).reshape(hh, ww, 8, 226)
    for dy in range(15):
        for dx in range(15):
            want += ar[..., dy * 15 + dx, None] * vp[dy:dy + hh, dx:dx + ww, None, :]
    assert max_abs_rel(got, want.reshape(hh * ww, 8 * vd)) < 1e-5


def test_dot8_lane_order():
    a = np.arange(40, dtype=np.float32) * np.float32(0.37)
    b = np.cos(np.arange(40, dtype=np.float32)).astype(np.float32)
    assert abs(oracle.dot8(a, b) - float(a.astype(np.float64) @ b.astype(np.float64))) < 1e-4


def test_self_lambda_matches_unfolded_definition():
    c, p = 64, "blk.attn1"
    k = c // 8
    specs = []
    U._lin(specs, p + ".to_q", c, c)
    U._lin(specs, p + ".to_k", c, k, bias=False)
    U._lin(specs, p + ".to_v", c, k)
    specs += [U.Spec(p + ".pos_conv.weight", (k, 225), "weight", False),
              U.Spec(p + ".pos_conv.bias", (k,), "bias", False)]
    params = block_params(specs, 7, std=0.2)
    x = S.normal(8, (2, 12, 10, c))
    got = oracle.block_forward("self_lambda", params, p, x)
    want = R.self_lambda(params, p, x.astype(np.float64))
    assert max_abs_rel(got, want) < TOL


@pytest.mark.parametrize("branches", [(0, 1), (1,)])
def test_cross_lambda_matches_unfolded_definition(branches):
    c, p = 320, "blk.attn2"
    k = c // 8
    specs = cond_specs() + [U.Spec(p + ".rel_pos_emb", (4096, 10, k), "weight", False)]
    U._lin(specs, p + ".to_q", c, c)
    specs += [U.Spec(p + ".to_k.weight", (k, U.XDIM), "weight", True),
              U.Spec(p + ".to_v.weight", (k, U.XDIM), "weight", True),
              U.Spec(p + ".to_v.bias", (k,), "bias", False)]
    params = block_params(specs, 9, std=0.05)
    x = S.normal(10, (len(branches), 64, 64, c))
    got = oracle.block_forward("cross_lambda", params, p, x, branches=branches)
    want = R.cross_lambda(params, p, x.astype(np.float64), branches)
    assert max_abs_rel(got, want) < TOL


@pytest.mark.parametrize("ci,co", [(64, 96), (96, 96)])
def test_resnet_block_matches_definition(ci, co):
    p = "blk"
    specs = []
    U._resnet(specs, p, ci, co)
    params = block_params(specs, 11, std=0.1)
    x = S.normal(12, (2, 9, 7, ci))
    temb = S.normal(13, (2, 1280))
    got = oracle.block_forward("resnet", params, p, x, c_out=co, temb=temb)
    want = R.resnet(params, p, x.astype(np.float64), temb.astype(np.float64), ci, co)
    assert max_abs_rel(got, want) < TOL


def test_dwconv2d_matches_definition():
    p = "blk"
    specs = []
    U._dwconv(specs, p, 9, 32)
    params = block_params(specs, 14, std=0.3)
    x = S.normal(15, (2, 8, 8, 9))
    got = oracle.block_forward("dwconv", params, p, x, c_out=32)
    assert max_abs_rel(got, R.dwconv2d(params, p, x.astype(np.float64), 9, 32)) < TOL


def test_transformer_block_matches_definition():
    c, p = 320, "blk"
    specs = cond_specs()
    U._transformer(specs, p, c)
    params = block_params(specs, 16, std=0.05)
    x = S.normal(17, (2, 64, 64, c))
    got = oracle.block_forward("transformer", params, p, x, branches=(0, 1))
    want = R.transformer(params, p, x.astype(np.float64), (0, 1))
    assert max_abs_rel(got, want) < TOL


@pytest.fixture(scope="module")
def unet():
    return oracle.UNet(U.random_unet(seed=4000))


def test_unet_cfg_cond_item_equals_cond_only_forward(unet):
    """Batch items never mix: the cond item of a CFG step is the CondOnly step,
    bit for bit, and the uncond item differs only through the cross-lambda branch."""
    inp = U.unet_input(seed=5000)
    eps2 = unet.forward(inp.x, inp.timestep, cfg=True)
    eps1 = unet.forward(inp.x, inp.timestep, cfg=False)
    assert eps2.shape == (2, 64, 64, 4) and eps1.shape == (1, 64, 64, 4)
    assert np.array_equal(eps2[1], eps1[0])
    assert not np.array_equal(eps2[0], eps2[1])
    assert np.isfinite(eps2).all()


def test_unet_trace_names_and_shapes(unet):
    inp = U.unet_input(seed=5001)
    _, tr = unet.forward(inp.x, inp.timestep, cfg=False, trace=True)
    names = list(tr)
    assert names[0] == "unet.temb" and names[1] == "unet.conv_in" and names[-1] == "unet.out"
    assert tr["unet.down.0.res.0"].shape == (1, 64, 64, 320)
    assert tr["unet.down.1.out"].shape == (1, 16, 16, 640)
    assert tr["unet.down.2.attn.1"].shape == (1, 16, 16, 1280)
    assert tr["unet.up.0.out"].shape == (1, 32, 32, 1280)
    assert tr["unet.up.2.attn.2"].shape == (1, 64, 64, 320)
    assert len([n for n in names if ".res." in n]) == 6 + 9
    # the time embedding is sinusoid -> linear -> SiLU -> linear (src/unet/embed.rs:48-66)
    P = U.random_unet(seed=4000)
    s = oracle.timestep_sinusoid(inp.timestep)
    a1 = s @ P["diff_model.time_embedding.linear_1.weight"].T + P["diff_model.time_embedding.linear_1.bias"]
    a2 = R.silu(a1.astype(np.float64)) @ P["diff_model.time_embedding.linear_2.weight"].T.astype(np.float64)
    a2 += P["diff_model.time_embedding.linear_2.bias"]
    assert max_abs_rel(tr["unet.temb"].reshape(-1), a2) < 1e-5
