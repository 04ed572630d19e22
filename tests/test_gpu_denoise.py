"""The denoise loop on the device (mh_unet_denoise) and its samplers
(mh_scheduler_*), through the C ABI: the update kernels against the
reference's own expected values (src/scheduler.rs:202-255) and bit for bit
against the oracle's samplers, then whole trajectories (DDIM with CFG on every
step; DPM-Solver++(2M) on a trailing schedule with CFG for the first step
only) against the oracle's loop over the oracle UNet."""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from moebius_cpu_amd import _lib
from moebius_cpu_amd import engine as E
from moebius_cpu_amd import synthetic as S
from moebius_cpu_amd import unet_params as U
from moebius_cpu_amd.unet import Scheduler, UNet, denoise
from tests.util import max_abs_rel

pytestmark = pytest.mark.gpu
TOL = 1e-4


@pytest.fixture(scope="module")
def ctx():
    c = E.Context(0)
    yield c
    c.synchronize()
    c.close()


def D(ctx, a):
    return E.DeviceArray.from_numpy(ctx, np.ascontiguousarray(a, np.float32))


def close(got, want, rel):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    assert np.all(np.abs(got - want) <= rel * np.maximum(np.abs(want), 1e-3)), (got, want)


def test_ddim_step_and_add_noise_match_diffusers(ctx):
    """src/scheduler.rs:236-255 on the device."""
    s = Scheduler(ctx, 20, 0.99, "leading", length=3)
    x = np.array([0.5, -1.25, 2.0], np.float32)
    eps = D(ctx, [0.1, -0.3, 0.7])
    for t, want in ((900, [6.129949689e-01, -1.518200040e+00, 2.366255760e+00]),
                    (50, [4.927129745e-01, -1.221965790e+00, 1.911952496e+00]),
                    (0, [4.972958863e-01, -1.241781354e+00, 1.980433226e+00])):
        xd = D(ctx, x)
        s.ddim_step(eps, None, 0.0, t, xd)
        close(xd.numpy(), want, 1e-5)
    out = E.DeviceArray(ctx, (3,))
    s.add_noise(D(ctx, x), eps, 900, out)
    close(out.numpy(), [1.587691903e-01, -4.465679526e-01, 9.329465032e-01], 1e-5)


def test_dpm_solver_matches_diffusers(ctx):
    """src/scheduler.rs:202-219 on the device: first order, second order, then the
    final step to the data prediction."""
    s = Scheduler(ctx, 5, 1.0, "trailing", length=3)
    assert s.timesteps == [999, 799, 599, 399, 199]
    want = [[1.228850083e+00, -2.980257470e+00, 4.364194085e+00],
            [2.418310907e+00, -5.782050465e+00, 8.090883333e+00],
            [3.814012762e+00, -9.051524459e+00, 1.235500469e+01],
            [4.986929961e+00, -1.177817121e+01, 1.581279684e+01],
            [5.635935287e+00, -1.324560079e+01, 1.747831563e+01]]
    x = D(ctx, [0.5, -1.25, 2.0])
    for i, w in enumerate(want):
        k = np.float32(1.0) + np.float32(0.2) * np.float32(i)
        s.dpm_step(D(ctx, [np.float32(0.1) * k, np.float32(-0.3) * k, np.float32(0.7) * k]), None, 0.0, i, x)
        close(x.numpy(), w, 2e-5)


@pytest.mark.parametrize("solver", ["ddim", "dpm"])
@pytest.mark.parametrize("cfg", [False, True])
def test_guided_steps_bit_exact_to_the_oracle(ctx, solver, cfg):
    """Every step of a 6-step schedule on 64x64x4 values: the device's CFG combine
    and update give the oracle's bits (the same f32 operations in the same order);
    DPM restarts once, as the Fast preset does where CFG stops."""
    steps, spacing = (6, "trailing") if solver == "dpm" else (20, "leading")
    strength = 1.0 if solver == "dpm" else 0.3
    dev = Scheduler(ctx, steps, strength, spacing)
    ref = oracle.Scheduler(steps, strength, spacing)
    assert dev.timesteps == ref.timesteps
    rng = np.random.default_rng(11 + cfg)
    x = rng.standard_normal(64 * 64 * 4).astype(np.float32)
    xd = D(ctx, x)
    g = np.float32(2.5)
    for i, t in enumerate(ref.timesteps):
        u = rng.standard_normal(x.size).astype(np.float32)
        c = rng.standard_normal(x.size).astype(np.float32)
        eps = (u + g * (c - u)).astype(np.float32) if cfg else u
        if solver == "dpm" and i == 2:
            dev.dpm_restart()
            ref.dpm_restart()
        if solver == "ddim":
            dev.ddim_step(D(ctx, u), D(ctx, c) if cfg else None, g, t, xd)
            x = ref.ddim_step(eps, t, x)
        else:
            dev.dpm_step(D(ctx, u), D(ctx, c) if cfg else None, g, i, xd)
            x = ref.dpm_step(eps, i, x)
        assert np.array_equal(xd.numpy(), x), f"step {i} (t={t})"


@pytest.fixture(scope="module")
def params():
    return U.random_unet(seed=4000)


@pytest.fixture(scope="module")
def gnet(ctx, params):
    return UNet(ctx, params)


@pytest.fixture(scope="module")
def onet(params):
    return oracle.UNet(params)


def _inputs(seed):
    inp = U.unet_input(seed=seed)
    mask = inp.x[..., 4:5]
    z_masked = inp.x[..., 5:9]
    z_img = S.normal(seed + 11, (1, 64, 64, 4))
    init = S.normal(seed + 12, (1, 64, 64, 4))
    return z_img, init, mask, z_masked


@pytest.mark.parametrize("case", [
    dict(steps=20, strength=0.15, spacing="leading", solver="ddim", cfg_steps=None),   # t = 100, 50, 0 with CFG
    dict(steps=10, strength=0.3, spacing="trailing", solver="dpm", cfg_steps=1),       # Fast-preset shape
])
def test_denoise_trajectory_matches_the_oracle(gnet, onet, case):
    z_img, init, mask, z_masked = _inputs(6000)
    print(f"denoise trajectory {case}", flush=True)
    seen = []
    got = denoise(gnet, z_img, init, mask, z_masked, guidance=2.5, progress=lambda d, t: seen.append((d, t)), **case)
    want = oracle.denoise(onet, z_img, init, mask, z_masked, guidance=2.5, **case)
    n = len(oracle.Scheduler(case["steps"], case["strength"], case["spacing"]).timesteps)
    assert seen == [(i, n) for i in range(1, n + 1)]
    err = max_abs_rel(got, want)
    print(f"  final latents max-abs/max|ref| = {err:.3e}")
    assert err <= TOL


def test_denoise_pure_noise_start_needs_no_image_latents(gnet, onet):
    """strength >= 1 starts from init alone (src/pipeline.rs:305-309): z_img may be NULL."""
    _, init, mask, z_masked = _inputs(6100)
    case = dict(steps=2, strength=1.0, spacing="trailing", solver="dpm", cfg_steps=0)
    got = denoise(gnet, None, init, mask, z_masked, guidance=2.5, **case)
    want = oracle.denoise(onet, np.zeros_like(init), init, mask, z_masked, guidance=2.5, **case)
    assert max_abs_rel(got, want) <= TOL


def test_denoise_cancel_leaves_the_output_untouched(ctx, gnet):
    """Cancelling from the progress callback returns MH_ERR_CANCELLED after the
    step it reports; the output buffer keeps its contents."""
    z_img, init, mask, z_masked = _inputs(6200)
    arrs = [D(ctx, a) for a in (z_img, init, mask, z_masked)]
    sentinel = np.full((1, 64, 64, 4), 7.0, np.float32)
    out = D(ctx, sentinel)
    prm = _lib.DenoiseParams(strength=0.15, guidance=2.5, steps=20, spacing=0, solver=0, cfg_steps=-1, reserved=0)
    calls = []

    def cb(_u, done, total):
        calls.append(done)
        return 1 if done == 1 else 0

    fn = _lib.STEP_FN(cb)
    import ctypes
    st = _lib.lib().mh_unet_denoise(gnet.h, arrs[0].ptr, arrs[1].ptr, arrs[2].ptr, arrs[3].ptr, ctypes.byref(prm),
                                    fn, None, out.ptr)
    assert st == _lib.ERR_CANCELLED and calls == [1]
    assert np.array_equal(out.numpy(), sentinel)


def test_denoise_rejects_bad_parameters(ctx, gnet):
    z_img, init, mask, z_masked = _inputs(6300)
    with pytest.raises(_lib.MoebiusError) as e:
        denoise(gnet, z_img, init, mask, z_masked, steps=0)
    assert e.value.code == _lib.ERR_INVALID_ARGUMENT
    with pytest.raises(_lib.MoebiusError) as e:
        denoise(gnet, z_img, init, mask, z_masked, steps=20, strength=0.01)  # int(20 * 0.01) = 0 timesteps
    assert "no timestep" in e.value.msg
    with pytest.raises(_lib.MoebiusError) as e:
        denoise(gnet, None, init, mask, z_masked, steps=20, strength=0.5)
    assert "z_img" in e.value.msg
