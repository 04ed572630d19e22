"""The oracle's window resampling (oracle/imaging.cpp: PIL's LANCZOS in 22-bit
fixed point, the formulation src/imaging/resize.rs's fast_image_resize 6.1.0
follows) pinned byte for byte to Pillow's LANCZOS on the reference's pixel
types (U8 and U8x3, up and down, 800 <-> 512 among them; fixture written by
tests/golden/make_lanczos_fixture.py), by the reference's resize tests
(src/imaging/resize.rs:66-147), by closed forms (a constant image stays exactly
constant; same size is a copy) and by an f64 separable Lanczos3 convolution
(within one 8-bit level per pass). Per-byte equality with fast_image_resize
itself is not pinned: the crate is not vendored. CPU only."""
from __future__ import annotations

import hashlib
import json
import math
import os
import sys

import numpy as np
import pytest

import oracle

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
sys.path.insert(0, GOLDEN)
from make_lanczos_fixture import image  # noqa: E402

PILLOW_CASES = json.load(open(os.path.join(GOLDEN, "lanczos.json"), encoding="utf-8"))["cases"]


@pytest.mark.parametrize("case", PILLOW_CASES, ids=lambda c: f"{c['kind']}-{c['from'][0]}x{c['from'][1]}-"
                                                          f"{c['to'][0]}x{c['to'][1]}-c{c['channels']}")
def test_matches_pillow_lanczos_byte_for_byte(case):
    """Pillow's LANCZOS output (SHA-256 of its bytes) for seeded L and RGB images."""
    img = image(case["kind"], case["seed"], *case["from"], case["channels"])
    got = oracle.resize_u8(img, *case["to"]).tobytes()
    assert got[:48].hex() == case["head"]
    assert hashlib.sha256(got).hexdigest() == case["sha256"]


def test_same_size_is_a_copy():
    img = (np.arange(512 * 512 * 3) * 7 % 256).astype(np.uint8).reshape(512, 512, 3)
    assert np.array_equal(oracle.resize_u8(img, 512, 512), img)


@pytest.mark.parametrize("frm,to", [(100, 512), (512, 100), (1200, 512), (512, 2000), (37, 23)])
@pytest.mark.parametrize("value", [0, 1, 40, 127, 200, 255])
def test_constant_images_stay_constant(frm, to, value):
    img = np.full((frm, frm, 3), value, np.uint8)
    assert (oracle.resize_u8(img, to, to) == value).all()


def test_reference_resize_cases():
    """src/imaging/resize.rs:117-145: a flat colour through a padded window stays
    flat; (0.5 -> 127) resized 512 -> 100 stays 127; 0.999 -> 254 at 512."""
    flat = np.tile(np.array([40, 120, 200], np.uint8), (100, 100, 1))
    assert (oracle.resize_u8(flat, 512, 512) == flat[0, 0]).all()
    half = np.full((512, 512, 3), 127, np.uint8)
    assert (oracle.resize_u8(half, 100, 100) == 127).all()


def _lanczos_f64(img, to_w, to_h):
    def axis(a, out, ax):
        n = a.shape[ax]
        scale = n / out
        fs = max(scale, 1.0)
        sup = 3.0 * fs
        res = []
        for xx in range(out):
            c = (xx + 0.5) * scale
            lo, hi = max(int(c - sup + 0.5), 0), min(int(c + sup + 0.5), n)
            xs = np.arange(lo, hi)
            t = (xs - c + 0.5) / fs
            w = np.where(np.abs(t) < 3, np.sinc(t) * np.sinc(t / 3), 0.0)
            w = w / w.sum()
            res.append(np.tensordot(w, np.take(a, xs, axis=ax), axes=([0], [ax])))
        r = np.stack(res, axis=ax)
        return np.clip(np.floor(r + 0.5), 0, 255)

    a = img.astype(np.float64)
    return axis(axis(a, to_w, 1), to_h, 0)


@pytest.mark.parametrize("frm,to", [(64, 41), (41, 96), (300, 512)])
def test_matches_f64_lanczos3_within_one_level_per_pass(frm, to):
    rng = np.random.default_rng(frm + to)
    img = rng.integers(0, 256, (frm, frm, 3), dtype=np.uint8)
    got = oracle.resize_u8(img, to, to).astype(np.int32)
    want = _lanczos_f64(img, to, to)
    assert np.abs(got - want).max() <= 2
    assert np.mean(got != want) < 0.05
