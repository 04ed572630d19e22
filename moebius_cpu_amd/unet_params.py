"""The UNet's converted tensor set (names, shapes, storage) and a seeded
random initialisation of it.

Names and layouts are those the reference's loader asks for
(src/unet/load.rs:51-97, blocks.rs:31-113, transformer.rs:65-87,
lambda.rs:86-104, 205-249 / 335-378, embed.rs:40-83, mod.rs:86-140) after the
converter (tools/convert_weights.py:13-33): BatchNorms folded into conv_dw /
conv_pw / to_q / to_v biases, 1x1 [o, i], dense 3x3 [o, 3, 3, i], depthwise
[3, 3, c], pos_conv [k, 225], rel_pos_emb [N, 10, k].
"""
from __future__ import annotations

import functools
from dataclasses import dataclass

import numpy as np

from . import synthetic as S

CH = (320, 640, 1280)
LAYERS = 2
HEADS = 8
TIME_PROJ = 320
TIME_EMBED = 1280
EHS = 3072
XDIM = 768
TOKENS = 10


@dataclass(frozen=True)
class Spec:
    name: str
    shape: tuple
    kind: str  # "weight" | "bias" | "norm_w" | "norm_b"
    gemm: bool  # f16-eligible GEMM weight (converter step 4)


def _lin(out, p, ci, co, bias=True):
    out.append(Spec(p + ".weight", (co, ci), "weight", True))
    if bias:
        out.append(Spec(p + ".bias", (co,), "bias", False))


def _norm(out, p, c):
    out.append(Spec(p + ".weight", (c,), "norm_w", False))
    out.append(Spec(p + ".bias", (c,), "norm_b", False))


def _dwconv(out, p, ci, co):
    out.append(Spec(p + ".conv_dw.weight", (3, 3, ci), "weight", False))
    out.append(Spec(p + ".conv_dw.bias", (ci,), "bias", False))
    _lin(out, p + ".conv_pw", ci, co)


def _resnet(out, p, ci, co):
    _norm(out, p + ".norm1", ci)
    _dwconv(out, p + ".conv1", ci, co)
    _lin(out, p + ".time_emb_proj", TIME_EMBED, co)
    _norm(out, p + ".norm2", co)
    _dwconv(out, p + ".conv2", co, co)
    if ci != co:
        _lin(out, p + ".conv_shortcut", ci, co)


def _transformer(out, p, c):
    k = c // HEADS
    hidden = int(c * 2.5)
    n = (64 * 320 // c) ** 2
    b = p + ".transformer_blocks.0"
    _norm(out, p + ".norm", c)
    _lin(out, p + ".proj_in", c, c)
    _norm(out, b + ".norm1", c)
    _lin(out, b + ".attn1.to_q", c, c)
    _lin(out, b + ".attn1.to_k", c, k, bias=False)
    _lin(out, b + ".attn1.to_v", c, k)
    out.append(Spec(b + ".attn1.pos_conv.weight", (k, 225), "weight", False))
    out.append(Spec(b + ".attn1.pos_conv.bias", (k,), "bias", False))
    _norm(out, b + ".norm2", c)
    out.append(Spec(b + ".attn2.rel_pos_emb", (n, TOKENS, k), "weight", False))
    _lin(out, b + ".attn2.to_q", c, c)
    out.append(Spec(b + ".attn2.to_k.weight", (k, XDIM), "weight", True))
    out.append(Spec(b + ".attn2.to_v.weight", (k, XDIM), "weight", True))
    out.append(Spec(b + ".attn2.to_v.bias", (k,), "bias", False))
    _norm(out, b + ".norm3", c)
    _lin(out, b + ".ff.inverted_conv.conv", c, 2 * hidden)
    out.append(Spec(b + ".ff.depth_conv.conv.weight", (3, 3, 2 * hidden), "weight", False))
    out.append(Spec(b + ".ff.depth_conv.conv.bias", (2 * hidden,), "bias", False))
    _lin(out, b + ".ff.point_conv.conv", hidden, c, bias=False)
    _lin(out, p + ".proj_out", c, c)


def unet_specs() -> list[Spec]:
    out: list[Spec] = [Spec("embedding_layer.weight", (20, EHS), "weight", False)]
    d = "diff_model"
    _lin(out, d + ".encoder_hid_proj", EHS, XDIM)
    _lin(out, d + ".time_embedding.linear_1", TIME_PROJ, TIME_EMBED)
    _lin(out, d + ".time_embedding.linear_2", TIME_EMBED, TIME_EMBED)
    _dwconv(out, d + ".conv_in", 9, CH[0])
    c_prev = CH[0]
    for i, c in enumerate(CH):
        l = f"{d}.down_blocks.{i}"
        for j in range(LAYERS):
            _resnet(out, f"{l}.resnets.{j}", c_prev if j == 0 else c, c)
            _transformer(out, f"{l}.attentions.{j}", c)
        if i + 1 < len(CH):
            out.append(Spec(f"{l}.downsamplers.0.conv.weight", (c, 3, 3, c), "weight", True))
            out.append(Spec(f"{l}.downsamplers.0.conv.bias", (c,), "bias", False))
        c_prev = c
    skips = [CH[0]]
    for i, c in enumerate(CH):
        skips += [c] * LAYERS
        if i + 1 < len(CH):
            skips.append(c)
    h_c = CH[-1]
    for i, c in enumerate(reversed(CH)):
        l = f"{d}.up_blocks.{i}"
        for j in range(LAYERS + 1):
            _resnet(out, f"{l}.resnets.{j}", h_c + skips.pop(), c)
            _transformer(out, f"{l}.attentions.{j}", c)
            h_c = c
        if i + 1 < len(CH):
            out.append(Spec(f"{l}.upsamplers.0.conv.weight", (c, 3, 3, c), "weight", True))
            out.append(Spec(f"{l}.upsamplers.0.conv.bias", (c,), "bias", False))
    assert not skips
    _norm(out, d + ".conv_norm_out", CH[0])
    _dwconv(out, d + ".conv_out", CH[0], 4)
    return out


@functools.lru_cache(maxsize=2)
def random_unet(seed: int = 4000, std: float = 0.02) -> dict[str, np.ndarray]:
    """Random init of every tensor: weights and biases N(0, std), norm gamma
    1 + N(0, std), beta N(0, std); one seed per tensor (seed + index).
    Cached per (seed, std): treat the arrays as read-only."""
    import concurrent.futures as cf
    import os

    specs = unet_specs()

    def gen(i):
        s = specs[i]
        return S.normal(seed * 100003 + i, s.shape, std=std, mean=1.0 if s.kind == "norm_w" else 0.0)

    # numpy releases the GIL inside its ufuncs: generate tensors in parallel.
    with cf.ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 1)) as ex:
        arrays = list(ex.map(gen, range(len(specs))))
    return {s.name: a for s, a in zip(specs, arrays)}


def param_count() -> int:
    return sum(int(np.prod(s.shape)) for s in unet_specs())


def step_flops(batch: int = 2, winograd: bool = False, cfg_shared: bool = False) -> dict:
    """Algorithmic FLOPs of one denoise step (multiply-add = 2), by kernel
    family, for the architecture above at a 64x64 latent: the GEMM-shaped
    work (1x1 convs and linears, the dense 3x3 convs, the lambda GEMMs) and
    the vector work (depthwise, tap filter, position term). winograd: count
    the two upsample convs as the Winograd F(2x2,3x3) GEMM work this build
    executes (else as direct convs). cfg_shared: count the part both CFG
    branches share (conv_in, the first resnet, and the first transformer up to
    its self-lambda, everything before the text conditioning enters) once, as
    the device runs it, instead of per item as the algorithm states it."""
    f = {"gemm_1x1": 0.0, "conv3x3": 0.0, "lambda_gemm": 0.0, "depthwise": 0.0, "tap_filter": 0.0,
         "position_term": 0.0}
    shared = cfg_shared and batch > 1

    def res(p, ci, co):
        f["depthwise"] += 18 * p * (ci + co)
        f["gemm_1x1"] += 2 * p * (ci * co + co * co) + 2 * batch * TIME_EMBED * co
        if ci != co:
            f["gemm_1x1"] += 2 * p * ci * co

    def tr(p, c, p_self=None):
        """p_self: the pixels the part before the cross-lambda runs over (GroupNorm,
        proj_in, LayerNorm 1, the self-lambda), when that differs from p."""
        k = c // HEADS
        hid = int(c * 2.5)
        ps = p if p_self is None else p_self
        f["gemm_1x1"] += 2 * ps * (2 * c * c + 2 * c * k) + 2 * p * (2 * c * c + c * 2 * hid + hid * c)
        f["lambda_gemm"] += 2 * ps * (k * k + HEADS * k * k + HEADS * k * 226) + 2 * p * HEADS * k * k
        f["tap_filter"] += 2 * ps * HEADS * 225 * k
        f["position_term"] += p * HEADS * TOKENS * 4 * k
        f["depthwise"] += 18 * p * 2 * hid

    side = [64, 32, 16]
    b_in = 1 if shared else batch
    f["depthwise"] += 18 * b_in * 4096 * 9 + 18 * batch * 4096 * CH[0]
    f["gemm_1x1"] += 2 * b_in * 4096 * 9 * CH[0] + 2 * batch * 4096 * CH[0] * 4
    c_prev = CH[0]
    for i, c in enumerate(CH):
        p = batch * side[i] ** 2
        for j in range(LAYERS):
            first = shared and i == 0 and j == 0
            if first:  # (res counts the time projection per item: it still runs at the batch)
                res(side[i] ** 2, c_prev, c)
                tr(p, c, p_self=side[i] ** 2)
            else:
                res(p, c_prev if j == 0 else c, c)
                tr(p, c)
        if i + 1 < 3:
            f["conv3x3"] += 2 * (p // 4) * 9 * c * c
        c_prev = c
    skips = [CH[0]]
    for i, c in enumerate(CH):
        skips += [c] * LAYERS
        if i + 1 < 3:
            skips.append(c)
    h_c = CH[-1]
    for i, c in enumerate(reversed(CH)):
        p = batch * side[2 - i] ** 2
        for j in range(LAYERS + 1):
            res(p, h_c + skips.pop(), c)
            tr(p, c)
            h_c = c
        if i + 1 < 3:
            # upsample conv: 4p output pixels; as Winograd F(2x2,3x3), 16 plane
            # GEMMs over p tiles (32 p c^2) instead of the direct 72 p c^2
            f["conv3x3"] += 32 * p * c * c if winograd else 2 * (4 * p) * 9 * c * c
    f["total"] = sum(f.values())
    return f


@dataclass
class UNetInput:
    x: np.ndarray       # [1, 64, 64, 9] = noisy(4) | mask(1) | masked-image latent(4)
    timestep: int


def unet_input(seed: int = 5000) -> UNetInput:
    """Inpainting latent stack: noisy latent ~N(0,1), binary mask with a random
    axis-aligned rectangle covering 10-40% of the 64x64 area, masked-image
    latent ~N(0,1); timestep uniform in 1..999."""
    u = S.uniform(seed, 8)
    area = 0.10 + 0.30 * u[0]
    aspect = 0.5 + 1.5 * u[1]
    rh = int(np.clip(round(np.sqrt(area * 4096 / aspect)), 1, 64))
    rw = int(np.clip(round(area * 4096 / rh), 1, 64))
    y0 = int(u[2] * (64 - rh + 1))
    x0 = int(u[3] * (64 - rw + 1))
    mask = np.zeros((64, 64), np.float32)
    mask[y0:y0 + rh, x0:x0 + rw] = 1.0
    noisy = S.normal(seed + 1, (64, 64, 4))
    masked = S.normal(seed + 2, (64, 64, 4))
    x = np.concatenate([noisy, mask[..., None], masked], axis=-1)[None].astype(np.float32)
    t = 1 + int(u[4] * 999)
    return UNetInput(x=np.ascontiguousarray(x), timestep=min(t, 999))
