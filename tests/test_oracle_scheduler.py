"""The oracle's samplers (oracle/pipeline.cpp) against the values the
reference's own tests pin (src/scheduler.rs:171-256, from diffusers via
tools/dump_ddim_reference.py and tools/dump_dpm_reference.py), plus closed
forms of the schedule. CPU only."""
from __future__ import annotations

import numpy as np

import oracle


def close(got, want, rel):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    assert np.all(np.abs(got - want) <= rel * np.maximum(np.abs(want), 1e-3)), (got, want)


def test_timesteps_match_diffusers():
    """src/scheduler.rs:179-191"""
    d = oracle.Scheduler(20, 0.99, "leading")
    assert d.timesteps == [i * 50 for i in range(18, -1, -1)]
    assert not d.pure_noise_start
    assert oracle.Scheduler(7, 0.99, "leading").timesteps == [710, 568, 426, 284, 142, 0]
    full = oracle.Scheduler(20, 1.0, "leading")
    assert len(full.timesteps) == 20 and full.timesteps[0] == 950 and full.pure_noise_start
    assert oracle.Scheduler(4, 1.0, "trailing").timesteps == [999, 749, 499, 249]
    # the Fast preset: 10 trailing steps at strength 0.99 keep the last 9
    assert oracle.Scheduler(10, 0.99, "trailing").timesteps == [899, 799, 699, 599, 499, 399, 299, 199, 99]


def test_alphas_cumprod_match_diffusers():
    """src/scheduler.rs:193-198"""
    a = oracle.alphas_cumprod()
    close(a[[0, 1, 500, 900, 999]], [9.991499782e-01, 9.982960224e-01, 2.763324678e-01, 1.415113267e-02,
                                      4.660095088e-03], 1e-5)
    # closed form: the f64 product of (1 - beta_i) of the scaled-linear betas
    betas = np.linspace(np.sqrt(0.00085), np.sqrt(0.012), 1000) ** 2
    assert np.max(np.abs(a - np.cumprod(1 - betas)) / np.cumprod(1 - betas)) < 2e-5
    assert np.all(np.diff(a) < 0)


def test_dpm_solver_matches_diffusers():
    """src/scheduler.rs:202-219: first order, then second order, then the final
    step straight to the data prediction."""
    d = oracle.Scheduler(5, 1.0, "trailing")
    assert d.timesteps == [999, 799, 599, 399, 199]
    want = [[1.228850083e+00, -2.980257470e+00, 4.364194085e+00],
            [2.418310907e+00, -5.782050465e+00, 8.090883333e+00],
            [3.814012762e+00, -9.051524459e+00, 1.235500469e+01],
            [4.986929961e+00, -1.177817121e+01, 1.581279684e+01],
            [5.635935287e+00, -1.324560079e+01, 1.747831563e+01]]
    x = np.array([0.5, -1.25, 2.0], np.float32)
    for i, w in enumerate(want):
        k = np.float32(1.0) + np.float32(0.2) * np.float32(i)
        eps = np.array([np.float32(0.1) * k, np.float32(-0.3) * k, np.float32(0.7) * k], np.float32)
        x = d.dpm_step(eps, i, x)
        close(x, w, 2e-5)


def test_dpm_restart_makes_the_next_step_first_order():
    """src/scheduler.rs:221-234"""
    eps = np.array([0.1, -0.3, 0.7], np.float32)
    fresh, restarted = oracle.Scheduler(5, 1.0, "trailing"), oracle.Scheduler(5, 1.0, "trailing")
    a = np.array([0.5, -1.25, 2.0], np.float32)
    restarted.dpm_step(eps, 0, np.array([1.0, 2.0, 3.0], np.float32))
    restarted.dpm_restart()
    assert np.array_equal(fresh.dpm_step(eps, 1, a), restarted.dpm_step(eps, 1, a))


def test_ddim_step_and_add_noise_match_diffusers():
    """src/scheduler.rs:236-255"""
    d = oracle.Scheduler(20, 0.99, "leading")
    x = np.array([0.5, -1.25, 2.0], np.float32)
    eps = np.array([0.1, -0.3, 0.7], np.float32)
    for t, want in ((900, [6.129949689e-01, -1.518200040e+00, 2.366255760e+00]),
                    (50, [4.927129745e-01, -1.221965790e+00, 1.911952496e+00]),
                    (0, [4.972958863e-01, -1.241781354e+00, 1.980433226e+00])):
        close(d.ddim_step(eps, t, x), want, 1e-5)
    close(d.add_noise(x, eps, 900), [1.587691903e-01, -4.465679526e-01, 9.329465032e-01], 1e-5)


def test_ddim_step_closed_form():
    """With eps equal to the noise that add_noise mixed in, a DDIM step from t to
    t - r lands on add_noise(x0, eps, t - r): the deterministic sampler's fixed
    point (f32 rounding aside)."""
    d = oracle.Scheduler(20, 1.0, "leading")
    rng = np.random.default_rng(0)
    x0 = rng.standard_normal(1000).astype(np.float32)
    n = rng.standard_normal(1000).astype(np.float32)
    xt = d.add_noise(x0, n, 500)
    assert np.max(np.abs(d.ddim_step(n, 500, xt) - d.add_noise(x0, n, 450))) < 2e-5
