"""The library's host-side schedule (mh_schedule_timesteps,
mh_schedule_alphas_cumprod) against the values the reference's tests pin
(src/scheduler.rs:179-198) and against the oracle, bit for bit. No GPU."""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from moebius_cpu_amd import _lib
from moebius_cpu_amd.unet import schedule_alphas_cumprod, schedule_timesteps


def test_timesteps_match_diffusers():
    assert schedule_timesteps(20, 0.99, "leading") == ([i * 50 for i in range(18, -1, -1)], False)
    assert schedule_timesteps(7, 0.99, "leading")[0] == [710, 568, 426, 284, 142, 0]
    ts, pure = schedule_timesteps(20, 1.0, "leading")
    assert len(ts) == 20 and ts[0] == 950 and pure
    assert schedule_timesteps(4, 1.0, "trailing")[0] == [999, 749, 499, 249]
    assert schedule_timesteps(5, 1.0, "trailing")[0] == [999, 799, 599, 399, 199]


@pytest.mark.parametrize("steps,strength,spacing", [(20, 0.99, "leading"), (10, 0.99, "trailing"), (1, 1.0, "leading"),
                                                    (1000, 0.5, "trailing"), (3, 0.2, "leading"), (33, 0.71, "trailing")])
def test_timesteps_equal_the_oracle(steps, strength, spacing):
    s = oracle.Scheduler(steps, strength, spacing)
    assert schedule_timesteps(steps, strength, spacing) == (s.timesteps, s.pure_noise_start)


def test_alphas_cumprod_bit_exact_to_the_oracle_and_diffusers():
    a = schedule_alphas_cumprod()
    assert np.array_equal(a, oracle.alphas_cumprod())
    want = np.array([9.991499782e-01, 9.982960224e-01, 2.763324678e-01, 1.415113267e-02, 4.660095088e-03])
    assert np.all(np.abs(a[[0, 1, 500, 900, 999]] - want) <= 1e-5 * want)


def test_bad_schedule_is_an_argument_error():
    with pytest.raises(_lib.MoebiusError) as e:
        schedule_timesteps(0, 0.99)
    assert e.value.code == _lib.ERR_INVALID_ARGUMENT and "steps must be 1..=1000" in e.value.msg
    with pytest.raises(_lib.MoebiusError):
        schedule_timesteps(1001, 0.99)
