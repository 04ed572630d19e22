"""The library's host imaging steps (src/imaging, src/vae/mod.rs roi_window)
through the C ABI, against the reference's own unit tests
(src/imaging/mod.rs:90-131, crop.rs:68-134, blend.rs:216-341,
vae/mod.rs:325-352) and its fixtures: Pillow 10.4's GaussianBlur
(tests/fixtures/blur.safetensors) and upstream paste_compensate
(tests/fixtures/compensate.safetensors), byte for byte. No GPU."""
from __future__ import annotations

import ctypes
import os

import numpy as np
import pytest

from moebius_cpu_amd import _lib

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
L = _lib.lib()


def bbox(m):
    h, w = m.shape
    m = np.ascontiguousarray(m, np.uint8)
    r = (ctypes.c_uint32 * 4)()
    f = ctypes.c_uint32()
    _lib.check(L.mh_mask_bbox(m.ctypes.data, w, h, w, r, ctypes.byref(f)))
    return tuple(r) if f.value else None


def dilate(m, k):
    h, w = m.shape
    m = np.ascontiguousarray(m, np.uint8)
    out = np.empty((h, w), np.uint8)
    _lib.check(L.mh_mask_dilate(m.ctypes.data, w, h, w, k, out.ctypes.data))
    return out


def plan(b, iw, ih):
    x, y, s = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_uint32()
    _lib.check(L.mh_crop_plan((ctypes.c_uint32 * 4)(*b), iw, ih, ctypes.byref(x), ctypes.byref(y), ctypes.byref(s)))
    return x.value, y.value, s.value


def blur(m, radius=3.0):
    h, w = m.shape
    m = np.ascontiguousarray(m, np.uint8)
    out = np.empty_like(m)
    _lib.check(L.mh_gaussian_blur(m.ctypes.data, w, h, radius, out.ctypes.data))
    return out


def paste(image, mask, result, px, py, side, mode):
    img = np.array(image, np.uint8, copy=True)
    h, w, c = img.shape
    mask = np.ascontiguousarray(mask, np.uint8)
    result = np.ascontiguousarray(result, np.uint8)
    r = (ctypes.c_uint32 * 4)()
    _lib.check(L.mh_paste(img.ctypes.data, w, h, w * c, c, mask.ctypes.data, w, result.ctypes.data, px, py, side,
                          mode, r))
    return img, tuple(r)


def roi(points, margin):
    m = np.zeros(64 * 64, np.float32)
    for x, y in points:
        m[y * 64 + x] = 1.0
    r = (ctypes.c_uint32 * 4)()
    f = ctypes.c_uint32()
    _lib.check(L.mh_roi_window(m.ctypes.data, margin, r, ctypes.byref(f)))
    return tuple(r) if f.value else None


def test_mask_bbox():
    """src/imaging/mod.rs:94-104"""
    m = np.zeros((5, 6), np.uint8)
    assert bbox(m) is None
    m[1, 2] = 255
    m[3, 4] = 200
    m[2, 1] = 127
    assert bbox(m) == (2, 1, 3, 3)


def test_dilate_matches_cv2_anchor():
    """src/imaging/mod.rs:106-130"""
    m = np.zeros((7, 9), np.uint8)
    m[3, 4] = 255
    m[0, 0] = 200
    d = dilate(m, 3)
    assert (d == 255).sum() == 9 + 4 and d[2, 3] == 255 and d[4, 5] == 255 and d[2, 6] == 0
    d = dilate(m, 2)
    assert d[3, 4] == 255 and d[2, 3] == 0 and d[4, 5] == 255
    assert (dilate(m, 1) == 255).sum() == 2
    assert (dilate(np.full((7, 9), 127, np.uint8), 3) == 0).all()


def test_dilate_equals_a_brute_force_max_filter():
    rng = np.random.default_rng(5)
    m = (rng.random((31, 23)) > 0.97).astype(np.uint8) * 255
    for k in (2, 3, 4, 7):
        b, a = k // 2, k - 1 - k // 2
        want = np.zeros_like(m)
        for y in range(31):
            for x in range(23):
                want[y, x] = m[max(0, y - b):y + a + 1, max(0, x - b):x + a + 1].max()
        assert np.array_equal(dilate(m, k), want), k


def test_crop_plans():
    """src/imaging/crop.rs:75-119"""
    assert plan((100, 100, 40, 40), 2000, 2000) == (0, 0, 512)
    assert plan((900, 900, 40, 40), 2000, 2000) == (664, 664, 512)
    for b in ((0, 0, 512, 512), (100, 100, 300, 300), (5, 5, 2, 2)):
        assert plan(b, 512, 512) == (0, 0, 512)
    assert plan((100, 100, 600, 600), 800, 800) == (0, 0, 800)
    assert plan((200, 50, 500, 300), 1000, 400)[2::-2] == (1000, 0)
    assert plan((500, 500, 600, 400), 2000, 1500) == (200, 100, 1200)
    assert plan((1900, 10, 80, 80), 2000, 2000) == (1488, 0, 512)
    assert plan((100, 50, 100, 100), 300, 200) == (0, -50, 300)


def test_window_always_contains_the_mask():
    """src/imaging/crop.rs:113-133 (the same xorshift case generator)."""
    seed = 0x9E3779B97F4A7C15
    mask64 = (1 << 64) - 1

    def nxt(m):
        nonlocal seed
        seed ^= (seed << 13) & mask64
        seed ^= seed >> 7
        seed ^= (seed << 17) & mask64
        return seed % m

    for _ in range(2000):
        iw, ih = 1 + nxt(3000), 1 + nxt(3000)
        x, y = nxt(iw), nxt(ih)
        b = (x, y, 1 + nxt(iw - x), 1 + nxt(ih - y))
        px, py, side = plan(b, iw, ih)
        assert px <= b[0] and py <= b[1]
        assert px + side >= b[0] + b[2] and py + side >= b[1] + b[3]


def _fixture(name):
    from safetensors.numpy import load_file

    return load_file(os.path.join(GOLDEN, name))


@pytest.mark.parametrize("case", ["a", "b", "c"])
def test_gaussian_blur_is_byte_exact_vs_pillow(case):
    f = _fixture("blur.safetensors")
    m = f[f"{case}.mask"].astype(np.uint8)
    assert np.array_equal(blur(m), f[f"{case}.blurred"].astype(np.uint8))


def test_feather_paste_keeps_outside_and_blends_edge():
    """src/imaging/blend.rs:244-262"""
    w, h = 40, 30
    data = np.full((h, w, 3), 10, np.uint8)
    m = np.zeros((h, w), np.uint8)
    m[5:25, 10:30] = 255
    out, r = paste(data, m, np.full((40, 40, 3), 250, np.uint8), 0, 0, 40, _lib_mode("feather"))
    assert r == (0, 0, 40, 30)
    assert out[0, 0, 0] == 10 and out[15, 20, 0] == 250 and 10 < out[15, 9, 0] < 250


def _lib_mode(name):
    return {"none": 1, "feather": 2, "compensate": 3}[name]


def _paste_at_origin(image, result, mask, mode):
    h, w, _ = image.shape
    side = max(w, h)
    padded = np.zeros((side, side, 3), np.uint8)
    padded[:h, :w] = result
    return paste(image, mask, padded, 0, 0, side, _lib_mode(mode))[0]


@pytest.mark.parametrize("case", ["a", "b", "c"])
def test_compensated_paste_is_byte_exact_vs_upstream(case):
    """src/imaging/blend.rs:286-303"""
    f = _fixture("compensate.safetensors")
    image, result = f[f"{case}.image"].astype(np.uint8), f[f"{case}.result"].astype(np.uint8)
    mask, want = f[f"{case}.mask"].astype(np.uint8), f[f"{case}.out"].astype(np.uint8)
    got = _paste_at_origin(image, result, mask, "compensate")
    assert np.array_equal(got, want)
    assert not np.array_equal(_paste_at_origin(image, result, mask, "feather"), got)


def test_compensation_falls_back_to_feather():
    """src/imaging/blend.rs:305-340: no ring (mask everywhere) or no mask."""
    w, h = 24, 20
    image = (np.arange(w * h * 3) * 7 % 251).astype(np.uint8).reshape(h, w, 3)
    result = (np.arange(w * h * 3) * 13 % 241).astype(np.uint8).reshape(h, w, 3)
    full = np.full((h, w), 255, np.uint8)
    assert np.array_equal(_paste_at_origin(image, result, full, "compensate"),
                          _paste_at_origin(image, result, full, "feather"))
    image, result, empty = np.full((16, 16, 3), 90, np.uint8), np.full((16, 16, 3), 200, np.uint8), \
        np.zeros((16, 16), np.uint8)
    assert np.array_equal(_paste_at_origin(image, result, empty, "compensate"),
                          _paste_at_origin(image, result, empty, "feather"))


def test_paste_none_copies_the_window():
    rng = np.random.default_rng(1)
    image = rng.integers(0, 256, (30, 50, 4), dtype=np.uint8)
    result = rng.integers(0, 256, (50, 50, 3), dtype=np.uint8)
    out, r = paste(image, np.zeros((30, 50), np.uint8), result, 0, -10, 50, _lib_mode("none"))
    assert r == (0, 0, 50, 30)
    assert np.array_equal(out[..., :3], result[10:40]) and np.array_equal(out[..., 3], image[..., 3])


def test_roi_window():
    """src/vae/mod.rs:325-351"""
    assert roi([], 8) is None
    assert roi([(0, 0), (63, 63)], 8) == (0, 0, 64, 64)
    assert roi([(20, 30), (24, 31)], 8) == (12, 22, 21, 18)
    assert roi([(0, 0), (2, 1)], 8) == (0, 0, 11, 10)
    assert roi([(62, 63)], 8) == (54, 55, 10, 9)
    assert roi([(5, 6)], 0) == (5, 6, 1, 1)


def test_bad_arguments():
    m = np.zeros((4, 4), np.uint8)
    assert L.mh_mask_bbox(m.ctypes.data, 4, 4, 3, (ctypes.c_uint32 * 4)(), None) == _lib.ERR_INVALID_ARGUMENT
    assert L.mh_crop_plan((ctypes.c_uint32 * 4)(0, 0, 5, 1), 4, 4, ctypes.byref(ctypes.c_int64()),
                          ctypes.byref(ctypes.c_int64()), ctypes.byref(ctypes.c_uint32())) == _lib.ERR_INVALID_ARGUMENT
