"""The allocation-free GroupNorm forward (mh_group_norm_forward_noalloc) against
mh_group_norm_forward through the C ABI: the same kernels over a fixed device
scratch array, so the outputs must be bit-identical, call after call, including
a second, smaller call that reuses the array the first one left behind. The
noalloc calls run first, on a fresh context, with the library's device-allocation
count read around them: it must not move."""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from moebius_cpu_amd import _lib
from moebius_cpu_amd import engine as E
from tests.util import max_abs_rel

pytestmark = pytest.mark.gpu

SCRATCH_FLOATS = 1 << 18  # the array's size, stated in include/moebius_hip.h


@pytest.fixture
def ctx():
    """A fresh context per test: its workspace has never been grown."""
    c = E.Context(0)
    yield c
    c.synchronize()
    c.close()


def _gn_inputs(seed, n, h, w, c, use_add):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((n, h, w, c)) * 1.3 + 0.2).astype(np.float32)
    gamma = (1 + 0.1 * rng.standard_normal(c)).astype(np.float32)
    beta = (0.1 * rng.standard_normal(c)).astype(np.float32)
    add = (0.5 * rng.standard_normal((n, c))).astype(np.float32) if use_add else None
    return x, gamma, beta, add


class _Call:
    """Device operands of one GroupNorm call, uploaded up front so that issuing
    the call itself allocates nothing on the Python side either."""

    def __init__(self, ctx, x, gamma, beta, add, groups, eps, silu):
        self.ctx, self.shape, self.groups, self.eps, self.silu = ctx, x.shape, groups, eps, int(silu)
        self.dx = E.DeviceArray.from_numpy(ctx, x)
        self.dg, self.db = E.DeviceArray.from_numpy(ctx, gamma), E.DeviceArray.from_numpy(ctx, beta)
        self.da = E.DeviceArray.from_numpy(ctx, add) if add is not None else None
        self.out = E.DeviceArray(ctx, x.shape)

    def issue(self, entry):
        n, h, w, c = self.shape
        fn = getattr(_lib.lib(), entry)
        _lib.check(fn(self.ctx.h, self.dx.ptr, n, h, w, c, self.groups, self.eps, self.dg.ptr, self.db.ptr,
                      self.da.ptr if self.da else None, self.silu, self.out.ptr))

    def run(self, entry):
        self.issue(entry)
        return self.out.numpy()


def _run(ctx, entry, x, gamma, beta, add, groups, eps, silu):
    return _Call(ctx, x, gamma, beta, add, groups, eps, silu).run(entry)


# Two calls in a row, the second on a smaller input: the UNet's resnet GroupNorm
# (2 x 64x64x320, add folded, SiLU), then a 1 x 16x16x64 map; and the VAE's
# 512x512x128 GroupNorm followed by the UNet's 16x16x1280 level.
CASES = [
    (((2, 64, 64, 320), True, True, 1e-5), ((1, 16, 16, 64), False, False, 1e-6)),
    (((1, 512, 512, 128), False, True, 1e-6), ((2, 16, 16, 1280), True, True, 1e-5)),
]


@pytest.mark.parametrize("first,second", CASES)
def test_noalloc_matches_group_norm_forward(ctx, first, second):
    inputs, calls = [], []
    for i, (shape, use_add, silu, eps) in enumerate((first, second)):
        x, gamma, beta, add = _gn_inputs(11 + i + shape[3], *shape, use_add)
        inputs.append((x, gamma, beta, add, eps, silu))
        calls.append(_Call(ctx, x, gamma, beta, add, 32, eps, silu))
    before = E.device_allocations()
    got = []
    for i, call in enumerate(calls):
        print(f"noalloc GroupNorm call {i}: shape {call.shape}", flush=True)
        got.append(call.run("mh_group_norm_forward_noalloc"))
    assert E.device_allocations() == before, "the noalloc entry point allocated device memory"
    for i, (x, gamma, beta, add, eps, silu) in enumerate(inputs):
        want = _run(ctx, "mh_group_norm_forward", x, gamma, beta, add, 32, eps, silu)
        assert np.array_equal(got[i], want), f"call {i}: differs from mh_group_norm_forward"
        if x.shape[0] * x.shape[1] * x.shape[2] <= 8192:
            ref = oracle.group_norm(x, 32, eps, gamma, beta, add=add, silu=silu)
            assert max_abs_rel(got[i], ref) <= 1e-4


def test_noalloc_calls_from_two_contexts_do_not_overlap(ctx):
    """Two contexts on one GPU share the array: the large VAE-size call is queued
    on one stream and a smaller call on the other right after it, without a host
    synchronisation between; the second waits for the first on the device, so
    both keep mh_group_norm_forward's bits."""
    other = E.Context(0)
    try:
        big = _gn_inputs(31, 1, 512, 512, 128, False)
        small = _gn_inputs(32, 2, 16, 16, 1280, True)
        a = _Call(ctx, *big, 32, 1e-6, True)
        b = _Call(other, *small, 32, 1e-5, True)
        print("noalloc across two contexts", flush=True)
        for _ in range(3):
            a.issue("mh_group_norm_forward_noalloc")
            b.issue("mh_group_norm_forward_noalloc")
        got_a, got_b = a.out.numpy(), b.out.numpy()
        other.synchronize()
        assert np.array_equal(got_a, _run(ctx, "mh_group_norm_forward", *big, 32, 1e-6, True))
        assert np.array_equal(got_b, _run(other, "mh_group_norm_forward", *small, 32, 1e-5, True))
    finally:
        other.synchronize()
        other.close()


def test_noalloc_rejects_shapes_beyond_the_scratch(ctx):
    """2 x 1x1 x 40960 needs 4 * n * c = 327680 floats > 262144: refused on the
    host with a clear error, before any kernel is queued."""
    n, c = 2, 40960
    x = np.zeros((n, 1, 1, c), np.float32)
    g, b = np.ones(c, np.float32), np.zeros(c, np.float32)
    with pytest.raises(_lib.MoebiusError) as e:
        _run(ctx, "mh_group_norm_forward_noalloc", x, g, b, None, 32, 1e-5, False)
    assert e.value.code == _lib.ERR_INVALID_ARGUMENT
    assert "fixed" in e.value.msg and str(SCRATCH_FLOATS) in e.value.msg
    # the context is still usable
    x2, g2, b2, _ = _gn_inputs(3, 1, 4, 4, 64, False)
    got = _run(ctx, "mh_group_norm_forward_noalloc", x2, g2, b2, None, 32, 1e-5, True)
    want = _run(ctx, "mh_group_norm_forward", x2, g2, b2, None, 32, 1e-5, True)
    assert np.array_equal(got, want)
