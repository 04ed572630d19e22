"""The benchmark workloads as concrete seeded inputs (shared by tests and
bench.py). Shapes and distributions follow the five workload definitions of
the conv/norm path:

1. conv3x3_gn_silu: NHWC 3x3 conv 64x64x320 -> 320 (stride 1, pad 1), then
   GroupNorm(32, eps 1e-5) + SiLU.
2. kernel sweep: (S, C) in (64,320), (32,640), (16,1280), (8,1280): 1x1 C->C,
   depthwise 3x3, GroupNorm(32)+SiLU, broadcast bias + residual add; f32 and
   f16-stored GEMM weights.
3. resnet block 32x32: GN+SiLU -> 3x3 320->640 -> + Linear(SiLU(temb)) ->
   GN+SiLU -> 3x3 640->640, plus 1x1 skip 320->640 and the residual add.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from . import synthetic as S

SWEEP = ((64, 320), (32, 640), (16, 1280), (8, 1280))


@dataclass
class ConvGnSilu:
    x: np.ndarray
    w: np.ndarray
    b: np.ndarray
    gamma: np.ndarray
    beta: np.ndarray
    groups: int = 32
    eps: float = 1e-5

    @property
    def flops(self) -> float:
        n, h, w, ci = self.x.shape
        return 2.0 * n * h * w * 9 * ci * self.w.shape[0]


def conv3x3_gn_silu(seed: int = 1000, n=1, s=64, c_in=320, c_out=320) -> ConvGnSilu:
    return ConvGnSilu(
        x=S.normal(seed, (n, s, s, c_in)),
        w=S.kaiming(seed + 1, (c_out, 3, 3, c_in), 9 * c_in),
        b=S.normal(seed + 2, (c_out,), std=0.02),
        gamma=S.normal(seed + 3, (c_out,), std=0.1, mean=1.0),
        beta=S.normal(seed + 4, (c_out,), std=0.1),
    )


@dataclass
class SweepPoint:
    s: int
    c: int
    x: np.ndarray
    w1: np.ndarray       # 1x1 [C, C]
    b1: np.ndarray
    dw_w: np.ndarray     # [3, 3, C]
    dw_b: np.ndarray
    gamma: np.ndarray
    beta: np.ndarray
    bias: np.ndarray     # broadcast bias [C]
    residual: np.ndarray


def sweep_point(s: int, c: int, seed: int = 2000) -> SweepPoint:
    seed = seed + 100 * s + c
    return SweepPoint(
        s=s, c=c,
        x=S.normal(seed, (1, s, s, c)),
        w1=S.kaiming(seed + 1, (c, c), c),
        b1=S.normal(seed + 2, (c,), std=0.02),
        dw_w=S.kaiming(seed + 3, (3, 3, c), 9),
        dw_b=S.normal(seed + 4, (c,), std=0.02),
        gamma=S.normal(seed + 5, (c,), std=0.1, mean=1.0),
        beta=S.normal(seed + 6, (c,), std=0.1),
        bias=S.normal(seed + 7, (c,), std=0.02),
        residual=S.normal(seed + 8, (1, s, s, c)),
    )


@dataclass
class ResnetBlock:
    x: np.ndarray
    temb: np.ndarray
    gn1_g: np.ndarray
    gn1_b: np.ndarray
    w1: np.ndarray
    b1: np.ndarray
    lin_w: np.ndarray
    lin_b: np.ndarray
    gn2_g: np.ndarray
    gn2_b: np.ndarray
    w2: np.ndarray
    b2: np.ndarray
    ws: np.ndarray
    bs: np.ndarray
    eps: float = 1e-5

    @property
    def flops(self) -> float:
        n, h, w, ci = self.x.shape
        co = self.w1.shape[0]
        p = n * h * w
        return 2.0 * p * (9 * ci * co + 9 * co * co + ci * co) + 2.0 * self.lin_w.size


def resnet_block(seed: int = 3000, s=32, c_in=320, c_out=640, temb_dim=1280) -> ResnetBlock:
    return ResnetBlock(
        x=S.normal(seed, (1, s, s, c_in)),
        temb=S.normal(seed + 1, (1, temb_dim)),
        gn1_g=S.normal(seed + 2, (c_in,), std=0.1, mean=1.0),
        gn1_b=S.normal(seed + 3, (c_in,), std=0.1),
        w1=S.kaiming(seed + 4, (c_out, 3, 3, c_in), 9 * c_in),
        b1=S.normal(seed + 5, (c_out,), std=0.02),
        lin_w=S.normal(seed + 6, (c_out, temb_dim), std=0.02),
        lin_b=S.normal(seed + 7, (c_out,), std=0.02),
        gn2_g=S.normal(seed + 8, (c_out,), std=0.1, mean=1.0),
        gn2_b=S.normal(seed + 9, (c_out,), std=0.1),
        w2=S.kaiming(seed + 10, (c_out, 3, 3, c_out), 9 * c_out),
        b2=S.normal(seed + 11, (c_out,), std=0.02),
        ws=S.kaiming(seed + 12, (c_out, c_in), c_in),
        bs=S.normal(seed + 13, (c_out,), std=0.02),
    )
