"""The VAE's converted tensor set (names, shapes) and a seeded random
initialisation of it.

Names are diffusers' AutoencoderKL names at the file root, as the reference's
loader asks for them (src/vae/mod.rs:174-189, 227-236, 297-312;
encoder.rs:47-73; decoder.rs:44-70); layouts after the converter
(tools/convert_weights.py:26-29): 1x1 and linear [o, i], dense 3x3 [o, 3, 3, i].
"""
from __future__ import annotations

import functools

import numpy as np

from . import synthetic as S
from .unet_params import Spec

CH = (128, 256, 512, 512)   # src/config.rs:54
LAYERS = 2                  # src/vae/encoder.rs:23 (up levels: LAYERS + 1)
LATENT_C = 4
IMAGE_C = 3
SCALING = 0.13025           # src/config.rs:58


def _conv3(out, p, ci, co):
    out.append(Spec(p + ".weight", (co, 3, 3, ci), "weight", True))
    out.append(Spec(p + ".bias", (co,), "bias", False))


def _lin(out, p, ci, co):
    out.append(Spec(p + ".weight", (co, ci), "weight", True))
    out.append(Spec(p + ".bias", (co,), "bias", False))


def _norm(out, p, c):
    out.append(Spec(p + ".weight", (c,), "norm_w", False))
    out.append(Spec(p + ".bias", (c,), "norm_b", False))


def _resnet(out, p, ci, co):
    _norm(out, p + ".norm1", ci)
    _conv3(out, p + ".conv1", ci, co)
    _norm(out, p + ".norm2", co)
    _conv3(out, p + ".conv2", co, co)
    if ci != co:
        _lin(out, p + ".conv_shortcut", ci, co)


def _mid(out, p, c):
    a = p + ".attentions.0"
    _norm(out, a + ".group_norm", c)
    for t in ("to_q", "to_k", "to_v", "to_out.0"):
        _lin(out, f"{a}.{t}", c, c)
    _resnet(out, p + ".resnets.0", c, c)
    _resnet(out, p + ".resnets.1", c, c)


def vae_specs() -> list[Spec]:
    out: list[Spec] = []
    e = "encoder"
    _conv3(out, e + ".conv_in", IMAGE_C, CH[0])
    c_prev = CH[0]
    for i, c in enumerate(CH):
        for j in range(LAYERS):
            _resnet(out, f"{e}.down_blocks.{i}.resnets.{j}", c_prev if j == 0 else c, c)
        if i + 1 < len(CH):
            _conv3(out, f"{e}.down_blocks.{i}.downsamplers.0.conv", c, c)
        c_prev = c
    _mid(out, e + ".mid_block", CH[-1])
    _norm(out, e + ".conv_norm_out", CH[-1])
    _conv3(out, e + ".conv_out", CH[-1], 2 * LATENT_C)
    _lin(out, "quant_conv", 2 * LATENT_C, 2 * LATENT_C)
    _lin(out, "post_quant_conv", LATENT_C, LATENT_C)
    d = "decoder"
    _conv3(out, d + ".conv_in", LATENT_C, CH[-1])
    _mid(out, d + ".mid_block", CH[-1])
    c_prev = CH[-1]
    for i, c in enumerate(reversed(CH)):
        for j in range(LAYERS + 1):
            _resnet(out, f"{d}.up_blocks.{i}.resnets.{j}", c_prev if j == 0 else c, c)
        if i + 1 < len(CH):
            _conv3(out, f"{d}.up_blocks.{i}.upsamplers.0.conv", c, c)
        c_prev = c
    _norm(out, d + ".conv_norm_out", CH[0])
    _conv3(out, d + ".conv_out", CH[0], IMAGE_C)
    return out


@functools.lru_cache(maxsize=2)
def random_vae(seed: int = 6000, bias_std: float = 0.02, norm_std: float = 0.05) -> dict[str, np.ndarray]:
    """Random init of every tensor, as the VAE benchmark configuration states it:
    Kaiming-normal weights (std sqrt(2 / fan_in), fan_in = 9 * c_in for the 3x3
    convs and c_in for the 1x1 convs and the attention projections, which are
    the same [o, i] GEMMs), GroupNorm gamma = 1 + N(0, norm_std) and
    beta = N(0, norm_std); the configuration leaves biases open, they are
    N(0, bias_std). Cached per argument set: treat the arrays as read-only."""
    import concurrent.futures as cf
    import os

    specs = vae_specs()

    def gen(i):
        s = specs[i]
        if s.kind == "weight":
            return S.kaiming(seed * 100003 + i, s.shape, int(np.prod(s.shape[1:])))
        std = norm_std if s.kind in ("norm_w", "norm_b") else bias_std
        return S.normal(seed * 100003 + i, s.shape, std=std, mean=1.0 if s.kind == "norm_w" else 0.0)

    with cf.ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 1)) as ex:
        arrays = list(ex.map(gen, range(len(specs))))
    return {s.name: a for s, a in zip(specs, arrays)}


def param_count() -> int:
    return sum(int(np.prod(s.shape)) for s in vae_specs())


def _conv3_flops(px: int, ci: int, co: int, winograd: bool, same: bool = True) -> float:
    """FLOPs of a 3x3 conv with px output pixels: the direct count 2*px*9*ci*co,
    or, for the stride-1 convs this build runs as Winograd F(2x2,3x3) (both
    channel counts multiples of 4), the 16 plane GEMMs over px/4 tiles:
    32 * (px/4) * ci * co = 8*px*ci*co (transforms not counted)."""
    if winograd and same and ci % 4 == 0 and co % 4 == 0:
        return 8.0 * px * ci * co
    return 2.0 * px * 9 * ci * co


def decode_flops(h: int = 64, w: int = 64, winograd: bool = False) -> float:
    """FLOPs of one decode of an h x w latent (multiply-add = 2): the 3x3 and 1x1
    convs and the mid attention's two products. winograd: count the stride-1
    3x3 convs as the Winograd GEMM work this build executes (else direct)."""
    f = 0.0
    p = h * w
    f += 2 * p * LATENT_C * LATENT_C + _conv3_flops(p, LATENT_C, CH[-1], winograd)

    def res(px, ci, co):
        return (_conv3_flops(px, ci, co, winograd) + _conv3_flops(px, co, co, winograd)
                + (2 * px * ci * co if ci != co else 0))

    f += 2 * res(p, CH[-1], CH[-1]) + 2 * p * 4 * CH[-1] ** 2 + 4 * p * p * CH[-1]
    c_prev = CH[-1]
    for i, c in enumerate(reversed(CH)):
        for j in range(LAYERS + 1):
            f += res(p, c_prev if j == 0 else c, c)
        if i + 1 < len(CH):
            p *= 4
            f += _conv3_flops(p, c, c, winograd)
        c_prev = c
    f += _conv3_flops(p, CH[0], IMAGE_C, winograd)
    return f


def encode_flops(b: int = 2, h: int = 512, w: int = 512, winograd: bool = False) -> float:
    """FLOPs of encoding b images of h x w (see decode_flops for winograd)."""
    f = 0.0
    p = h * w
    f += _conv3_flops(p, IMAGE_C, CH[0], winograd)

    def res(px, ci, co):
        return (_conv3_flops(px, ci, co, winograd) + _conv3_flops(px, co, co, winograd)
                + (2 * px * ci * co if ci != co else 0))

    c_prev = CH[0]
    for i, c in enumerate(CH):
        for j in range(LAYERS):
            f += res(p, c_prev if j == 0 else c, c)
        if i + 1 < len(CH):
            p //= 4
            f += _conv3_flops(p, c, c, winograd, same=False)  # stride-2 downsample
        c_prev = c
    f += 2 * res(p, CH[-1], CH[-1]) + 2 * p * 4 * CH[-1] ** 2 + 4 * p * p * CH[-1]
    f += _conv3_flops(p, CH[-1], 2 * LATENT_C, winograd) + 2 * p * 64
    return b * f


def vae_images(seed: int = 7000, b: int = 2, h: int = 512, w: int = 512) -> np.ndarray:
    """Synthetic RGB batch in [-1, 1]: uniform, [b, h, w, 3]."""
    return S.uniform_range(seed, (b, h, w, 3), -1.0, 1.0)
