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


class ResnetBlockGpu:
    """ResNet block 32x32 on the device: GN1+SiLU applied inside the Winograd conv1
    (the reference's forward_prologue), time projection Linear(SiLU(temb)) folded
    into GN2's shift, GN2+SiLU inside conv2, 1x1 skip with conv2's output as its
    residual. Buffers are allocated once; a call allocates nothing."""

    def __init__(self, ctx, wl, winograd=True):
        from . import engine as E

        self.E, self.ctx, self.wl = E, ctx, wl
        c_in, c_out = wl.w1.shape[3], wl.w1.shape[0]
        self.c_out = c_out
        self.x = E.Tensor.from_numpy(ctx, wl.x)
        self.gn1 = E.GroupNorm(ctx, 32, wl.eps, wl.gn1_g, wl.gn1_b)
        self.gn2 = E.GroupNorm(ctx, 32, wl.eps, wl.gn2_g, wl.gn2_b)
        self.conv1 = E.Conv3x3.same(ctx, c_in, c_out, E.Param(ctx, wl.w1), wl.b1, winograd=winograd)
        self.conv2 = E.Conv3x3.same(ctx, c_out, c_out, E.Param(ctx, wl.w2), wl.b2, winograd=winograd)
        self.lin = E.Conv1x1(ctx, wl.lin_w.shape[1], c_out, E.Param(ctx, wl.lin_w), wl.lin_b)
        self.skip = E.Conv1x1(ctx, c_in, c_out, E.Param(ctx, wl.ws), wl.bs)
        self.temb = E.Tensor.from_numpy(ctx, wl.temb.reshape(1, 1, 1, -1))
        self.t = E.Tensor(ctx, *self.temb.shape)
        self.tp, self.h, self.out, self.res = E.Tensor(ctx), E.Tensor(ctx), E.Tensor(ctx), E.Tensor(ctx)
        n = self.x.n
        self.aff1 = E.Affine(E.DeviceArray(ctx, (n * c_in,)), E.DeviceArray(ctx, (n * c_in,)), True)
        self.aff2 = E.Affine(E.DeviceArray(ctx, (n * c_out,)), E.DeviceArray(ctx, (n * c_out,)), True)

    def forward(self):
        E, ctx = self.E, self.ctx
        L = E.lib()
        x, g1, g2 = self.x, self.gn1, self.gn2
        E.check(L.mh_group_norm_affine(ctx.h, x.ptr, x.n, x.h, x.w, x.c, 32, g1.eps, g1.gamma.ptr, g1.beta.ptr,
                                       None, self.aff1.scale.ptr, self.aff1.shift.ptr))
        self.conv1.forward_prologue(x, self.aff1, self.h)
        E.check(L.mh_math_eval(ctx.h, 1, self.temb.ptr, self.temb.nbytes // 4, self.t.ptr))  # SiLU(temb)
        self.lin.forward(self.t, self.tp)
        h = self.h
        E.check(L.mh_group_norm_affine(ctx.h, h.ptr, h.n, h.h, h.w, h.c, 32, g2.eps, g2.gamma.ptr, g2.beta.ptr,
                                       self.tp.ptr, self.aff2.scale.ptr, self.aff2.shift.ptr))
        self.conv2.forward_prologue(h, self.aff2, self.out)
        self.skip.forward(x, self.res, self.out)
        return self.res
