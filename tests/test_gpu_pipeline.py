"""The whole inpainting run on the GPU (include/moebius_engine.h) against the
oracle's restatement of src/pipeline.rs (oracle/inpaint.py): window crop
with edge replication, Lanczos resampling both ways, VAE encode (whole frame
or the Fast preset's ROI encode), the denoise loop, decode (whole frame or ROI),
8-bit truncation and the paste. Models come from safetensors files written as
the converter writes them (f16 GEMM weights for the UNet), loaded through
moebius_engine_create.

Bars: the device resampler is byte-exact to the oracle's; the final latents
agree to rel-L2 2e-5 (f32 arithmetic in a different order through the VAE
encoder, then the denoise loop); the pasted image to within 3 levels on at
most 1% of its bytes (an f32 difference moves a value across an 8-bit
truncation step), and bytes outside the changed rectangle, and alpha, are
untouched. The feathered pastes use the library's host paste on the oracle's
window, which the reference's blend fixtures pin separately."""
from __future__ import annotations

import ctypes
import dataclasses
import os

import numpy as np
import pytest

import oracle
from oracle import inpaint as OI
from moebius_cpu_amd import _lib
from moebius_cpu_amd import engine as E
from moebius_cpu_amd import synthetic as S
from moebius_cpu_amd import unet_params as U
from moebius_cpu_amd import vae_params as V
from moebius_cpu_amd.pipeline import Control, Engine, InpaintParams, NoiseSet, Preset, Rect, Stage
from moebius_cpu_amd.weights_io import write_weights
from tests.util import rel_l2

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def weights(tmp_path_factory):
    d = tmp_path_factory.mktemp("weights")
    up = U.random_unet(seed=4100)
    gemm = {s.name for s in U.unet_specs() if s.gemm}
    write_weights(str(d / "unet.safetensors"), up, sorted(gemm), f16=True)
    vp = V.random_vae()
    write_weights(str(d / "vae.safetensors"), vp, metadata={"scaling_factor": "0.13025"})
    # the oracle sees exactly the stored values: f16 GEMM weights widened to f32
    uo = {k: (v.astype(np.float16).astype(np.float32) if k in gemm else v) for k, v in up.items()}
    return d, uo, vp


@pytest.fixture(scope="module")
def engine(weights):
    print("engine: moebius_engine_create", flush=True)
    e = Engine.load(str(weights[0]))
    yield e
    e.close()


@pytest.fixture(scope="module")
def omodels(weights):
    return oracle.UNet(weights[1]), oracle.Vae(weights[2])


def image(seed, h, w, c):
    """A smooth gradient with noise, so the resampler sees structure."""
    y, x = np.mgrid[0:h, 0:w]
    base = np.stack([(x * 255 // max(w - 1, 1)), (y * 255 // max(h - 1, 1)), ((x + y) * 3) % 256], -1)
    noise = S.uniform_range(seed, (h, w, 3), -20, 20)
    rgb = np.clip(base + noise, 0, 255).astype(np.uint8)
    if c == 4:
        rgb = np.concatenate([rgb, (S.uniform_range(seed + 1, (h, w, 1), 0, 256)).astype(np.uint8)], -1)
    return np.ascontiguousarray(rgb)


def rect_mask(h, w, x0, y0, x1, y1, value=255):
    m = np.zeros((h, w), np.uint8)
    m[y0:y1, x0:x1] = value
    return m


def ellipse_mask(h, w, cx, cy, rx, ry):
    y, x = np.mgrid[0:h, 0:w]
    return np.where(((x - cx) / rx) ** 2 + ((y - cy) / ry) ** 2 <= 1.0, 255, 0).astype(np.uint8)



def oracle_inpaint(omodels, img, mask, p: InpaintParams, noise: NoiseSet):
    out = img.copy()
    r = OI.run(omodels[0], omodels[1], img, mask, p, noise)
    if r is None:
        return out, Rect(), None
    result, plan, lat = r
    if p.paste == "none":
        rect = OI.paste_none(out, result, plan)
    else:
        m = OI.dilate(mask, p.mask_dilate) if p.mask_dilate > 0 else mask
        rect = host_paste(out, m, result, plan, p.paste)
    return out, Rect(*rect), lat


def host_paste(img, mask, result, plan, mode):
    h, w, c = img.shape
    r = (ctypes.c_uint32 * 4)()
    _lib.check(_lib.lib().mh_paste(img.ctypes.data, w, h, w * c, c, np.ascontiguousarray(mask).ctypes.data, w,
                                   np.ascontiguousarray(result).ctypes.data, plan.x, plan.y, plan.side,
                                   _lib.PASTE[mode], r))
    return tuple(r)


def compare(got_img, want_img, orig, rect: Rect):
    assert got_img.shape == want_img.shape
    d = np.abs(got_img.astype(np.int16) - want_img.astype(np.int16))
    print(f"  image: max diff {d.max()}, {np.mean(d > 0):.2e} of the bytes differ", flush=True)
    assert d.max() <= 3, f"max diff {d.max()}"
    assert np.mean(d > 0) <= 0.01, f"{np.mean(d > 0):.4f} of the bytes differ"
    outside = np.ones(orig.shape[:2], bool)
    outside[rect.y:rect.y + rect.h, rect.x:rect.x + rect.w] = False
    assert np.array_equal(got_img[outside], orig[outside])
    if orig.shape[2] == 4:
        assert np.array_equal(got_img[..., 3], orig[..., 3])


CASES = {
    # window past the bottom and top edges (edge replication), 300 -> 512 -> 300 resampling, raw paste
    "exact_edge_none": dict(hwc=(200, 300, 3), mask=("rect", 250, 20, 290, 60), preset=Preset.EXACT,
                            over=dict(steps=2, paste="none")),
    # a 512 window in a larger RGBA image (no resampling), ROI encode, DPM with CFG on the first step,
    # dilation and the feathered paste
    "fast_roi_encode_feather": dict(hwc=(480, 640, 4), mask=("ellipse", 300, 260, 40, 25), preset=Preset.FAST,
                                    over=dict(steps=3, cfg_steps=1, mask_dilate=5)),
    # upsampled 200 -> 512 window, partial strength (add_noise start), ROI decode, compensated paste
    "roi_decode_compensate": dict(hwc=(200, 200, 3), mask=("rect", 60, 90, 110, 130), preset=Preset.EXACT,
                                  over=dict(steps=2, strength=0.5, spacing="trailing", roi_decode=True,
                                            paste="feather_compensate")),
    # The presets unchanged on the benchmark's call: a 1024x768 RGB image with a 400x300 mask, so an
    # 800 px window resampled to 512 and back. Exact: 19 leading DDIM steps (20 at strength 0.99), CFG
    # 2.5 on every step, feathered paste. Fast: 9 trailing DPM-Solver++(2M) steps, CFG on the first 3,
    # the ROI encode (the mask's latent box plus its margin is 48x40 of the 64x64 latents).
    "exact_full_preset": dict(hwc=(768, 1024, 3), mask=("rect", 312, 234, 712, 534), preset=Preset.EXACT,
                              over=dict()),
    "fast_full_preset": dict(hwc=(768, 1024, 3), mask=("rect", 312, 234, 712, 534), preset=Preset.FAST,
                             over=dict()),
}


@pytest.mark.parametrize("name", list(CASES))
def test_inpaint_matches_the_oracle_pipeline(engine, omodels, name):
    case = CASES[name]
    h, w, c = case["hwc"]
    img = image(7000 + len(name), h, w, c)
    kind, *a = case["mask"]
    mask = rect_mask(h, w, *a) if kind == "rect" else ellipse_mask(h, w, *a)
    p = dataclasses.replace(case["preset"].params(), **case["over"])
    noise = NoiseSet.from_flat(S.normal(7100 + len(name), (_lib.NOISE_FLOATS,)))
    print(f"pipeline case {name}: {h}x{w}x{c} {p}", flush=True)
    got = img.copy()
    rect, lat = engine.inpaint_traced(got, mask, p, noise, latents=True)
    want, wrect, wlat = oracle_inpaint(omodels, img, mask, p, noise)
    assert rect == wrect
    err = rel_l2(lat, wlat)
    print(f"  latents rel-L2 {err:.3e}", flush=True)
    assert err <= 2e-5
    compare(got, want, img, rect)


def test_progress_stages_and_cancellation_leave_the_image_untouched(engine):
    img = image(7200, 256, 256, 3)
    mask = rect_mask(256, 256, 100, 100, 140, 150)
    p = dataclasses.replace(Preset.EXACT.params(), steps=3)  # strength 0.99: int(3 * 0.99) = 2 timesteps
    seen = []

    def record(pr):
        seen.append((int(pr.stage), pr.done, pr.total))
        return Control.CONTINUE

    out = img.copy()
    engine.inpaint(out, mask, p, progress=record)
    assert seen == [(0, 0, 1), (0, 1, 1), (1, 1, 2), (1, 2, 2), (2, 0, 1), (2, 1, 1)]
    for stop in [(Stage.ENCODE, 1), (Stage.DENOISE, 2), (Stage.DECODE, 1)]:
        out = img.copy()

        def cancel(pr, stop=stop):
            return Control.CANCEL if (pr.stage, pr.done) == stop else Control.CONTINUE

        with pytest.raises(_lib.MoebiusError) as e:
            engine.inpaint(out, mask, p, progress=cancel)
        assert e.value.code == _lib.ERR_CANCELLED
        assert np.array_equal(out, img), f"image changed after a cancel at {stop}"


def test_empty_mask_changes_nothing_and_reports_no_progress(engine):
    img = image(7300, 64, 96, 4)
    mask = np.full((64, 96), 127, np.uint8)  # below the 128 threshold everywhere
    calls = []
    out = img.copy()
    rect = engine.inpaint(out, mask, progress=lambda pr: calls.append(pr) or Control.CONTINUE)
    assert rect == Rect() and not calls and np.array_equal(out, img)


def test_seeded_c_api_equals_the_same_noise_given_explicitly(engine):
    img = image(7400, 300, 220, 3)
    mask = rect_mask(300, 220, 30, 200, 90, 260)
    L = _lib.lib()
    mp = _lib.MoebiusParams(preset=1, steps=2, guidance=0.0, seed=99, paste=0, mask_dilate=0)
    a = img.copy()
    rect = _lib.MoebiusRect()
    _lib.check(L.moebius_inpaint(engine._h, a.ctypes.data, 220, 300, 220 * 3, 3, mask.ctypes.data, 220,
                                 ctypes.byref(mp), None, None, ctypes.byref(rect)))
    b = img.copy()
    r2 = engine.inpaint_with_noise(b, mask, InpaintParams.resolve(preset=1, steps=2, seed=99), NoiseSet.sample(99))
    assert np.array_equal(a, b) and (rect.x, rect.y, rect.width, rect.height) == (r2.x, r2.y, r2.w, r2.h)
    assert not np.array_equal(a, img)
    # the models' pools, the frames and the loop state stay resident: a repeated
    # call makes no device allocation at all
    before, allocs = engine.memory(), E.device_allocations()
    engine.inpaint_with_noise(img.copy(), mask, InpaintParams.resolve(preset=1, steps=2, seed=99),
                              NoiseSet.sample(99))
    assert engine.memory() == before
    assert E.device_allocations() == allocs, "a repeated inpaint call allocated device memory"
    # released on request, allocated again by the next call, same result
    engine.release_scratch()
    assert engine.memory()[1] < before[1] and engine.memory()[0] == before[0]
    c = img.copy()
    engine.inpaint_with_noise(c, mask, InpaintParams.resolve(preset=1, steps=2, seed=99), NoiseSet.sample(99))
    assert np.array_equal(c, a)


@pytest.fixture(scope="module")
def ctx():
    c = E.Context(0)
    yield c
    c.synchronize()
    c.close()


@pytest.mark.parametrize("src_hw,dst_hw,c", [((300, 300), (512, 512), 3), ((512, 512), (300, 300), 3),
                                             ((200, 200), (512, 512), 1), ((480, 640), (200, 320), 4),
                                             ((5, 7), (3, 13), 3), ((512, 512), (512, 512), 3)])
def test_device_resize_is_byte_exact_to_the_oracle(ctx, src_hw, dst_hw, c):
    (fh, fw), (th, tw) = src_hw, dst_hw
    shape = (fh, fw) if c == 1 else (fh, fw, c)
    src = S.uniform_range(7500 + fh + c, shape, 0, 256).astype(np.uint8)
    src[: fh // 2] = np.minimum(src[: fh // 2], 40)  # hard edges for the negative lobes
    want = oracle.resize_u8(src, tw, th)
    d_src = E.DeviceArray.from_numpy(ctx, src)
    d_dst = E.DeviceArray(ctx, want.shape, np.uint8)
    print(f"resize {src_hw} -> {dst_hw} x{c}", flush=True)
    _lib.check(_lib.lib().mh_resize_u8(ctx.h, d_src.ptr, fw, fh, tw, th, c, d_dst.ptr))
    assert np.array_equal(d_dst.numpy(), want)


def _pillow_cases():
    import json
    import os

    golden = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "lanczos.json")
    with open(golden, encoding="utf-8") as f:
        return [c for c in json.load(f)["cases"] if c["from"] != c["to"]]


@pytest.mark.parametrize("case", _pillow_cases(), ids=lambda c: f"{c['kind']}-{c['from'][0]}x{c['from'][1]}-"
                                                             f"{c['to'][0]}x{c['to'][1]}-c{c['channels']}")
def test_device_resize_matches_pillow_lanczos(ctx, case):
    """The device resampler against Pillow's LANCZOS bytes directly (SHA-256 of the
    output; tests/golden/lanczos.json), on the reference's pixel types U8 and U8x3."""
    import hashlib
    import sys

    sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden"))
    from make_lanczos_fixture import image

    (fw, fh), (tw, th), c = case["from"], case["to"], case["channels"]
    src = image(case["kind"], case["seed"], fw, fh, c)
    d_src = E.DeviceArray.from_numpy(ctx, src)
    d_dst = E.DeviceArray(ctx, (th, tw) if c == 1 else (th, tw, c), np.uint8)
    print(f"pillow case {case['kind']} {fw}x{fh} -> {tw}x{th} x{c}", flush=True)
    _lib.check(_lib.lib().mh_resize_u8(ctx.h, d_src.ptr, fw, fh, tw, th, c, d_dst.ptr))
    got = d_dst.numpy().tobytes()
    assert got[:48].hex() == case["head"]
    assert hashlib.sha256(got).hexdigest() == case["sha256"]
