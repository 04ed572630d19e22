"""Host-side checks of the whole-pipeline C ABI (include/moebius_engine.h):
parameter resolution as in the reference's FFI tests (src/ffi.rs:271-282),
argument errors before any device work (src/ffi.rs:254-264), the noise
generator, and engine creation failing cleanly without a GPU."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from moebius_cpu_amd import _lib
from moebius_cpu_amd import synthetic as S
from moebius_cpu_amd.pipeline import InpaintParams, NoiseSet, Preset

EXACT = dict(steps=20, strength=0.99, spacing="leading", solver="ddim", guidance=2.5, seed=0, cfg_steps=None,
             roi_encode=False, roi_decode=False, paste="feather", mask_dilate=0, precision="exact")


def test_exact_preset_matches_the_reference_defaults():
    # src/preset.rs:62-75
    p = Preset.EXACT.params()
    for k, v in EXACT.items():
        assert getattr(p, k) == v, k
    assert p.noise_offset == np.float32(0.0357)


def test_fast_preset_changes_only_the_sampling_fields():
    # src/preset.rs:76-82: 10 trailing DPM-Solver++(2M) steps, CFG for 3, ROI encode
    p = Preset.FAST.params()
    want = dict(EXACT, steps=10, spacing="trailing", solver="dpm", cfg_steps=3, roi_encode=True)
    for k, v in want.items():
        assert getattr(p, k) == v, k


def test_zeroed_params_are_exact_defaults_and_overrides_apply():
    # src/ffi.rs:271-282 zeroed_params_are_exact_defaults
    L = _lib.lib()
    z, c = _lib.MoebiusParams(), _lib.InpaintParams()
    assert L.mh_inpaint_params(ctypes.byref(z), ctypes.byref(c)) == _lib.OK
    assert InpaintParams.from_c(c) == Preset.EXACT.params()
    assert L.mh_inpaint_params(None, ctypes.byref(c)) == _lib.OK
    assert InpaintParams.from_c(c) == Preset.EXACT.params()
    r = InpaintParams.resolve(preset=1, steps=9)
    assert (r.steps, r.roi_encode) == (9, True)
    r = InpaintParams.resolve(preset=0, guidance=4.0, seed=77, paste="feather_compensate", mask_dilate=5)
    assert (r.guidance, r.seed, r.paste, r.mask_dilate) == (4.0, 77, "feather_compensate", 5)
    r = InpaintParams.resolve(preset=0, guidance=-1.0)  # <= 0: the preset's
    assert r.guidance == 2.5


@pytest.mark.parametrize("bad,msg", [(dict(preset=7), b"unknown preset 7"),
                                     (dict(paste=9), b"unknown paste mode 9")])
def test_unknown_preset_or_paste_is_invalid_argument(bad, msg):
    L = _lib.lib()
    m, c = _lib.MoebiusParams(**bad), _lib.InpaintParams()
    assert L.mh_inpaint_params(ctypes.byref(m), ctypes.byref(c)) == _lib.ERR_INVALID_ARGUMENT
    assert msg in L.moebius_last_error()


def test_invalid_arguments_are_reported_before_any_device_work():
    # src/ffi.rs:254-264: a null engine is rejected first
    L = _lib.lib()
    px = np.zeros(12, np.uint8)
    m = np.zeros(4, np.uint8)
    rc = L.moebius_inpaint(None, px.ctypes.data, 2, 2, 6, 3, m.ctypes.data, 2, None, None, None, None)
    assert rc == _lib.ERR_INVALID_ARGUMENT
    assert L.moebius_last_error() == b"null argument"
    assert L.mh_last_error() == b"null argument"  # one message per thread for both prefixes
    # dimensions and strides are checked before the engine is touched
    fake = ctypes.create_string_buffer(64)
    for w, h, stride, c, ms in [(0, 2, 6, 3, 2), (2, 0, 6, 3, 2), (2, 2, 5, 3, 2), (2, 2, 6, 3, 1)]:
        rc = L.moebius_inpaint(ctypes.addressof(fake), px.ctypes.data, w, h, stride, c, m.ctypes.data, ms, None,
                               None, None, None)
        assert rc == _lib.ERR_INVALID_ARGUMENT
        assert L.moebius_last_error() == b"bad dimensions or stride"
    noise = np.zeros(_lib.NOISE_FLOATS, np.float32)
    cp = Preset.EXACT.params().to_c()
    rc = L.mh_inpaint_with_noise(ctypes.addressof(fake), px.ctypes.data, 2, 2, 6, 3, m.ctypes.data, 2, None,
                                 noise.ctypes.data, None, None, None, None)
    assert rc == _lib.ERR_INVALID_ARGUMENT and L.mh_last_error() == b"null argument"
    rc = L.mh_inpaint_with_noise(ctypes.addressof(fake), px.ctypes.data, 2, 2, 6, 3, m.ctypes.data, 2,
                                 ctypes.byref(cp), None, None, None, None, None)
    assert rc == _lib.ERR_INVALID_ARGUMENT and L.mh_last_error() == b"null argument"


def test_engine_create_reports_null_and_missing_device():
    L = _lib.lib()
    out = ctypes.c_void_p(123)
    assert L.moebius_engine_create(None, 0, ctypes.byref(out)) == _lib.ERR_INVALID_ARGUMENT
    assert L.moebius_engine_create(b"/nonexistent", 0, None) == _lib.ERR_INVALID_ARGUMENT
    L.moebius_engine_destroy(None)  # ignored
    assert L.moebius_abi_version() == 1


def test_engine_create_without_a_gpu_fails_cleanly():
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    L = _lib.lib()
    out = ctypes.c_void_p(123)
    rc = L.moebius_engine_create(b"/nonexistent", 0, ctypes.byref(out))
    assert rc != _lib.OK and out.value is None
    assert L.moebius_last_error()


def test_noise_is_the_documented_generator_in_noiseset_order():
    # splitmix64 -> 53-bit uniforms -> Box-Muller (f64) -> f32, one stream of
    # 3 * 16384 + 4 normals: vae_img, vae_masked, init, offset
    n = NoiseSet.sample(1234)
    flat = n.flat()
    want = S.normal(1234, (_lib.NOISE_FLOATS,))
    # numpy's and the C library's cos / sin / log1p may differ in the last f64 bit
    assert np.abs(flat - want).max() <= 1e-6
    assert np.mean(flat == want) > 0.999
    assert n.offset.shape == (1, 1, 1, 4) and np.array_equal(n.offset.ravel(), want[-4:])
    assert np.array_equal(NoiseSet.sample(1234).flat(), flat)
    assert not np.array_equal(NoiseSet.sample(1235).flat(), flat)
    assert abs(float(flat.mean())) < 0.02 and abs(float(flat.std()) - 1.0) < 0.02


def test_noise_shape_is_checked():
    n = NoiseSet.sample(1)
    n.offset = np.zeros((1, 1, 1, 3), np.float32)
    with pytest.raises(_lib.MoebiusError, match="noise.offset has shape"):
        n.flat()
