"""Pins the oracle's UNet restatement (oracle/unet.cpp) to float64 restatements
of the blocks' mathematical definitions (tests/ref_f64.py: the lambda layers
in their unfolded upstream form, the norms and convs from their formulas) and
to invariants of the whole network. CPU only."""
from __future__ import annotations

import ast
import os

import numpy as np
import pytest

import oracle
from moebius_cpu_amd import synthetic as S
from moebius_cpu_amd import unet_params as U
from moebius_cpu_amd import vae_params as V
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


# ---- the whole network against the reference's published model facts

MANIFEST = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "weights-manifest.txt")
BN_TARGETS = {"bn1": "conv_dw", "bn2": "conv_pw", "norm_q": "to_q", "norm_v": "to_v"}
BN_KEYS = ("weight", "bias", "running_mean", "running_var", "num_batches_tracked")


def read_manifest():
    """{section: {name: shape}} of the reference's docs/weights-manifest.txt (a copy in tests/golden)."""
    sections, cur = {}, None
    for line in open(MANIFEST, encoding="utf-8"):
        line = line.rstrip("\n")
        if not line or line.startswith("#"):
            continue
        if line.startswith("["):
            cur = sections.setdefault(line.strip("[]"), {})
            continue
        name, shape = line.split("\t")
        cur[name] = tuple(ast.literal_eval(shape))
    return sections


def converted_shapes(upstream):
    """The converter's rewrites of an upstream state dict's names and shapes
    (tools/convert_weights.py:13-33): eval BatchNorms (found by their
    running_var) are dropped and folded into the layer beside them, which gains
    a bias; 1x1 [o,i,1,1] -> [o,i]; dense 3x3 [o,i,3,3] -> [o,3,3,i];
    depthwise [c,1,3,3] -> [3,3,c]; pos_conv [k,1,1,15,15] -> [k,225];
    rel_pos_emb [N,10,k,1] -> [N,10,k]."""
    bns = {}
    for name in upstream:
        mod, _, leaf = name.rpartition(".")
        if leaf == "running_var":
            parent, _, bn = mod.rpartition(".")
            assert bn in BN_TARGETS, f"BatchNorm {mod} has no fold target"
            bns[mod] = f"{parent}.{BN_TARGETS[bn]}"
    skip = {f"{bn}.{k}" for bn in bns for k in BN_KEYS}
    out = {}
    for name, shape in upstream.items():
        if name in skip:
            continue
        mod, _, leaf = name.rpartition(".")
        if mod in bns.values() and leaf == "weight":
            out[f"{mod}.bias"] = (shape[0],)
        if leaf == "rel_pos_emb":
            assert len(shape) == 4 and shape[-1] == 1
            shape = shape[:3]
        elif leaf == "weight" and len(shape) == 5:
            assert shape[1:3] == (1, 1)
            shape = (shape[0], shape[3] * shape[4])
        elif leaf == "weight" and len(shape) == 4:
            o, i, kh, kw = shape
            if (kh, kw) == (1, 1):
                shape = (o, i)
            elif i == 1:
                shape = (kh, kw, o)
            else:
                shape = (o, kh, kw, i)
        out[name] = tuple(shape)
    return out


def test_unet_tensor_set_is_the_manifest_after_conversion():
    """The converted UNet tensor set (names and layouts the oracle and the device
    load) equals the reference's manifest [unet] section after the converter's
    rewrites: 1 203 upstream entries, 124 BatchNorms folded."""
    up = read_manifest()["unet"]
    assert len(up) == 1203
    want = converted_shapes(up)
    got = {s.name: tuple(s.shape) for s in U.unet_specs()}
    assert sorted(set(want) - set(got)) == [] and sorted(set(got) - set(want)) == []
    bad = {k: (got[k], want[k]) for k in want if got[k] != want[k]}
    assert not bad, f"shape differences: {list(bad.items())[:5]}"


def test_vae_tensor_set_is_the_manifest_after_conversion():
    up = read_manifest()["vae"]
    want = converted_shapes(up)
    got = {s.name: tuple(s.shape) for s in V.vae_specs()}
    assert got == want


def test_unet_parameter_count_is_226_0_million():
    """docs/PLAN.md:30: 226.0 M parameters (the upstream module's parameters:
    no token embedding, BatchNorm affine included, running statistics not).
    The converted set holds exactly those minus the folded BatchNorm affines,
    plus the biases the folds add, plus the embedding table."""
    up = read_manifest()["unet"]
    numel = {k: int(np.prod(v, dtype=np.int64)) for k, v in up.items()}
    module = sum(n for k, n in numel.items()
                 if not k.startswith("embedding_layer.") and not k.rsplit(".", 1)[1].startswith(("running_", "num_")))
    assert round(module / 1e6, 1) == 226.0
    bn = [k.rsplit(".", 1)[0] for k in up if k.endswith(".running_var")]
    bn_affine = sum(2 * up[f"{m}.weight"][0] for m in bn)
    added_bias = sum(up[f"{m}.weight"][0] for m in bn
                     if f"{m.rsplit('.', 1)[0]}.{BN_TARGETS[m.rsplit('.', 1)[1]]}.bias" not in up)
    assert U.param_count() == module - bn_affine + added_bias + numel["embedding_layer.weight"]


def test_unet_step_flops_match_the_published_split(unet):
    """docs/PLAN.md:56: one CFG step (batch 2) is 632 GFLOP, 1x1 62.5%, dense 3x3
    19.1%, lambda pos-conv 14.0%, stride-2 1.2%, depthwise 0.5%
    (tools/count_flops.py's categories). The oracle tallies each layer's FLOPs
    at the shapes it runs (the unfolded lambda's products where it runs the
    folded form), so this checks the wiring it executes: which layers run, at
    which level and with which channel counts."""
    inp = U.unet_input(seed=5000)
    oracle.UNet.flops_reset()
    unet.forward(inp.x, inp.timestep, cfg=True)
    f = oracle.UNet.flops()
    total = sum(f.values())
    assert round(total / 1e9) == 632
    share = {k: round(100.0 * v / total, 1) for k, v in f.items()}
    assert share["1x1"] == 62.5
    assert share["3x3 dense"] == 19.1
    assert share["lambda pos_conv"] == 14.0
    assert share["3x3 stride 2"] == 1.2
    assert share["depthwise"] == 0.5
    # the device's FLOP model (bench.py's step roofline) is the folded count of the same layers
    mine = U.step_flops(2)
    temb_proj = sum(2 * 2 * s.shape[1] * s.shape[0] for s in U.unet_specs() if s.name.endswith("time_emb_proj.weight"))
    assert abs(mine["gemm_1x1"] - f["1x1"] - temb_proj) < 1e6
    assert abs(mine["conv3x3"] - f["3x3 dense"] - f["3x3 stride 2"]) < 1e6
    assert abs(mine["depthwise"] - f["depthwise"]) < 1e6
    # cond-only runs half of every per-item product
    oracle.UNet.flops_reset()
    unet.forward(inp.x, inp.timestep, cfg=False)
    assert abs(sum(oracle.UNet.flops().values()) - total / 2) < 1e-9 * total
