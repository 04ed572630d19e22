"""GroupNorm statistics written by the GEMM epilogue (gn_tile_partials in
gemm_kernel.hpp, shared by the f32 and f16 kernels), checked directly: for
every tiling the planner can be forced to, in EXACT and FAST precision, the
scale/shift folded from a 1x1 conv's epilogue partials
(mh_conv1x1_gn_partials + mh_group_norm_affine_partials) against
mh_group_norm_affine reading the conv's output (the reference's GroupNorm::affine,
src/engine/norm.rs:57-105), with and without the time-embedding add folded in,
at 1e-6; and against the oracle's GroupNorm of the same output. Tilings that
split K write no partials and say so (rows 0)."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

import oracle
from moebius_cpu_amd import engine as E
from tests.util import max_abs_rel

pytestmark = pytest.mark.gpu

PLANS = ["32,32,1", "32,64,1", "64,32,1", "64,64,1", "128,64,1", "64,128,1", "128,128,1", "64,64,2", None,
         # wide wave layouts (f32 kernel; FAST keeps its own tiles): partials summed from LDS
         "64,80,1,4,1,1,1", "64,80,1,4,1,1", "128,80,1,4,1,1,1", "64,160,1,2,2,1,1", "32,80,1,2,1,2,1",
         "32,80,1,2,1,2", "160,64,1,2,2,1,1", "160,64,1,2,2,1,1,16", "64,80,1,4,1,1,0,16", "128,128,1,2,2,1,1,16"]


@pytest.fixture(scope="module")
def ctx():
    c = E.Context(0)
    yield c
    c.synchronize()
    c.close()


@pytest.mark.parametrize("with_add", [False, True])
@pytest.mark.parametrize("fast", [False, True])
@pytest.mark.parametrize("plan", PLANS)
def test_epilogue_partials_fold_to_the_group_norm_of_the_output(ctx, plan, fast, with_add):
    n, h, w, c_in, c_out, groups, eps = 2, 32, 32, 96, 128, 32, 1e-5
    rng = np.random.default_rng(11 + c_in + (7 if fast else 0))
    x = rng.standard_normal((n, h, w, c_in)).astype(np.float32)
    wt = (rng.standard_normal((c_out, c_in)) / np.sqrt(c_in)).astype(np.float32)
    b = (rng.standard_normal(c_out) * 0.1 + 0.3).astype(np.float32)
    r = rng.standard_normal((n, h, w, c_out)).astype(np.float32)
    gamma = (1 + 0.1 * rng.standard_normal(c_out)).astype(np.float32)
    beta = (0.1 * rng.standard_normal(c_out)).astype(np.float32)
    add = (rng.standard_normal(n * c_out) * 0.5).astype(np.float32)
    ctx.set_precision(fast)
    ctx.set_tuning("gemm_plan", plan)
    try:
        param = E.Param(ctx, wt, f16=fast)
        dev = {k: E.DeviceArray.from_numpy(ctx, v) for k, v in dict(x=x, b=b, r=r, g=gamma, be=beta, a=add).items()}
        out = E.DeviceArray(ctx, (n, h, w, c_out))
        part = E.DeviceArray(ctx, ((n * h * w + 31) // 32 * c_out * 2,))
        rows = ctypes.c_uint32(99)
        print(f"partials plan={plan} fast={fast} add={with_add}", flush=True)
        E.check(E.lib().mh_conv1x1_gn_partials(ctx.h, dev["x"].ptr, n, h, w, c_in, param.ptr, param.dtype, c_out,
                                               dev["b"].ptr, dev["r"].ptr, out.ptr, part.ptr, ctypes.byref(rows)))
        y = out.numpy()
        parts = [int(v) for v in plan.split(",")] if plan else []
        if parts and parts[2] > 1:
            assert rows.value == 0  # a K split: the partial sums are not final in any one workgroup
            return
        if parts and not fast and (h * w) % parts[0]:
            assert rows.value == 0  # tiles would straddle two items: no partials
            return
        assert rows.value in (32, 64, 128) and (h * w) % rows.value == 0
        a_ptr = dev["a"].ptr if with_add else None
        sc, sh = E.DeviceArray(ctx, (n * c_out,)), E.DeviceArray(ctx, (n * c_out,))
        E.check(E.lib().mh_group_norm_affine_partials(ctx.h, part.ptr, rows.value, n, h, w, c_out, groups, eps,
                                                      dev["g"].ptr, dev["be"].ptr, a_ptr, sc.ptr, sh.ptr))
        want_sc, want_sh = E.DeviceArray(ctx, (n * c_out,)), E.DeviceArray(ctx, (n * c_out,))
        E.check(E.lib().mh_group_norm_affine(ctx.h, out.ptr, n, h, w, c_out, groups, eps, dev["g"].ptr, dev["be"].ptr,
                                             a_ptr, want_sc.ptr, want_sh.ptr))
        got = np.concatenate([sc.numpy(), sh.numpy()])
        dev_want = np.concatenate([want_sc.numpy(), want_sh.numpy()])
        assert max_abs_rel(got, dev_want) <= 1e-6
        # GN(y + add) = y . scale + shift: the oracle's shift for y + add, plus add . scale
        ya = y + add.reshape(n, 1, 1, c_out) if with_add else y
        o_sc, o_sh = oracle.group_norm_affine(np.ascontiguousarray(ya, dtype=np.float32), groups, eps, gamma, beta)
        if with_add:
            o_sh = (o_sh.astype(np.float64) + add.astype(np.float64) * o_sc).astype(np.float32)
        assert max_abs_rel(got, np.concatenate([o_sc, o_sh])) <= 1e-6
    finally:
        ctx.set_tuning("gemm_plan", None)
        ctx.set_precision(False)
