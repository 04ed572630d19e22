"""The GEMM launch timing behind bench.py's in-step figures (tuning key
"gemm_time", mh_context_gemm_times): one record per kernel configuration with
the launch count and 2.M.N.K per launch, cleared when read, nothing recorded
while the key is off, and the timed launches' results unchanged."""
from __future__ import annotations

import numpy as np
import pytest

from moebius_cpu_amd import engine as E
from moebius_cpu_amd import synthetic as S

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    c = E.Context(0)
    yield c
    c.synchronize()
    c.close()


def test_gemm_times_count_launches_and_flops(ctx):
    x = E.Tensor.from_numpy(ctx, S.normal(1, (2, 32, 32, 320)))
    conv = E.Conv1x1(ctx, 320, 640, E.Param(ctx, S.normal(2, (640, 320), 0.05)), S.normal(3, (640,), 0.02))
    y, z = E.Tensor(ctx), E.Tensor(ctx)
    conv.forward(x, y)
    want = y.numpy()
    assert ctx.gemm_times() == []  # off by default
    ctx.set_tuning("gemm_time", 1)
    try:
        print("gemm_time: three timed launches", flush=True)
        for _ in range(3):
            conv.forward(x, z)
        recs = ctx.gemm_times()
    finally:
        ctx.set_tuning("gemm_time", None)
    assert np.array_equal(z.numpy(), want)
    assert len(recs) == 1, recs
    rec = recs[0]
    assert rec["launches"] == 3
    assert rec["flops"] == 3 * 2.0 * (2 * 32 * 32) * 640 * 320
    assert 0 < rec["us"] < 3 * 10000
    assert rec["config"].startswith(("f32 ", "f32p "))
    assert ctx.gemm_times() == []  # cleared when read
    conv.forward(x, z)
    assert ctx.gemm_times() == []  # off again
