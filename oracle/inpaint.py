"""Oracle restatement of the reference's end-to-end inpainting run
(src/pipeline.rs:160-392, src/imaging/{mod,crop,resize}.rs) over the oracle's
resampler, VAE, UNet and denoise loop. Test infrastructure only, like the rest
of this package.

`run` returns the window-sized 8-bit result that the reference hands to
`paste` (src/pipeline.rs:209-212) together with the crop plan and the final
latents; `paste_none` restates the raw paste (src/imaging/blend.rs:166-173).
The feathered pastes are not restated here: they are pinned on their own
against the reference's blend fixtures.
"""
from __future__ import annotations

import dataclasses

import numpy as np

from . import Vae, denoise, resize_u8, to_u8

IMAGE_SIZE, LATENT, DOWN, ROI_MARGIN = 512, 64, 8, 8


@dataclasses.dataclass(frozen=True)
class Plan:
    x: int
    y: int
    side: int


def bbox(mask: np.ndarray):
    """src/imaging/mod.rs:31-46: (x, y, w, h) of the pixels >= 128, or None."""
    ys, xs = np.nonzero(mask >= 128)
    if ys.size == 0:
        return None
    return int(xs.min()), int(ys.min()), int(xs.max() - xs.min() + 1), int(ys.max() - ys.min() + 1)


def dilate(mask: np.ndarray, k: int) -> np.ndarray:
    """src/imaging/mod.rs:48-77: binarise (>= 128 -> 255), then the max over
    [i - k/2, i + k - 1 - k/2] per axis, out-of-range ignored."""
    cur = np.where(mask >= 128, 255, 0).astype(np.uint8)
    if k <= 1:
        return cur
    before, after = k // 2, k - 1 - k // 2
    h, w = cur.shape
    tmp = np.zeros_like(cur)
    for x in range(w):
        tmp[:, x] = cur[:, max(0, x - before):min(w - 1, x + after) + 1].max(axis=1)
    out = np.zeros_like(cur)
    for y in range(h):
        out[y] = tmp[max(0, y - before):min(h - 1, y + after) + 1].max(axis=0)
    return out


def _place(start: int, length: int, side: int, extent: int) -> int:
    """src/imaging/crop.rs:51-60."""
    if side <= extent:
        centred = (2 * start + length) // 2 - side // 2
        return min(max(centred, 0), extent - side)
    return -((side - extent) // 2)


def crop_plan(bb, img_w: int, img_h: int) -> Plan:
    """src/imaging/crop.rs:28-38."""
    x, y, w, h = bb
    long, img_long = max(w, h), max(img_w, img_h)
    side = min(max(long + 2 * (long // 2), min(IMAGE_SIZE, img_long)), img_long)
    return Plan(_place(x, w, side, img_w), _place(y, h, side, img_h), side)


def source_rect(p: Plan, img_w: int, img_h: int):
    """src/imaging/crop.rs:41-48."""
    x0, y0 = max(p.x, 0), max(p.y, 0)
    return x0, y0, min(p.x + p.side, img_w) - x0, min(p.y + p.side, img_h) - y0


def to_model(img: np.ndarray, mask: np.ndarray, p: Plan):
    """src/imaging/resize.rs:34-63: window (edge-replicated image, zero mask
    outside) -> 512x512 rgb in [-1, 1] (f64 arithmetic, f32) and a 0/255 mask."""
    h, w = mask.shape
    ys, xs = np.arange(p.side) + p.y, np.arange(p.side) + p.x
    yc, xc = np.clip(ys, 0, h - 1), np.clip(xs, 0, w - 1)
    win = img[yc[:, None], xc[None, :], :3]
    inside = ((ys >= 0) & (ys < h))[:, None] & ((xs >= 0) & (xs < w))[None, :]
    binw = np.where(inside & (mask[yc[:, None], xc[None, :]] >= 128), 255, 0).astype(np.uint8)
    rgb8 = win if p.side == IMAGE_SIZE else resize_u8(win, IMAGE_SIZE, IMAGE_SIZE)
    bin8 = binw if p.side == IMAGE_SIZE else resize_u8(binw, IMAGE_SIZE, IMAGE_SIZE)
    bin8 = np.where(bin8 >= 128, 255, 0).astype(np.uint8)
    rgb = (rgb8.astype(np.float64) / 255.0 * 2.0 - 1.0).astype(np.float32)
    return rgb, bin8


def roi_window(mask_lat: np.ndarray, margin: int):
    """src/vae/mod.rs:60-78: (x, y, w, h) of the latent mask's bbox grown by margin, or None."""
    ys, xs = np.nonzero(mask_lat.reshape(LATENT, LATENT) > 0.5)
    if ys.size == 0:
        return None
    x0, y0 = max(int(xs.min()) - margin, 0), max(int(ys.min()) - margin, 0)
    x1, y1 = min(int(xs.max()) + margin, LATENT - 1), min(int(ys.max()) + margin, LATENT - 1)
    return x0, y0, x1 - x0 + 1, y1 - y0 + 1


def run(unet, vae: Vae, img: np.ndarray, mask: np.ndarray, params, noise):
    """src/pipeline.rs:186-345 + 350-392 up to the paste. img [h,w,3|4] uint8,
    mask [h,w] uint8; params with the fields of the reference's InpaintParams
    (spacing / solver as "leading" / "trailing", "ddim" / "dpm"; cfg_steps None
    = every step); noise with vae_img, vae_masked, init [1,64,64,4] and offset
    [1,1,1,4]. Returns (result [side,side,3] uint8, plan, latents) or None for
    an empty mask."""
    if params.mask_dilate > 0:
        mask = dilate(mask, params.mask_dilate)
    bb = bbox(mask)
    if bb is None:
        return None
    plan = crop_plan(bb, img.shape[1], img.shape[0])
    rgb, bin8 = to_model(img, mask, plan)
    keep = np.where(bin8 >= 128, 0.0, 1.0).astype(np.float32)[..., None]
    masked = rgb * keep
    mask_lat = np.where(bin8[::DOWN, ::DOWN] >= 128, 1.0, 0.0).astype(np.float32).reshape(1, LATENT, LATENT, 1)

    win = roi_window(mask_lat, ROI_MARGIN)
    if win is not None and not (win[2] < LATENT or win[3] < LATENT):
        win = None
    if params.roi_encode and win is not None:
        x, y, w, h = win
        z_masked = vae.encode(masked[None], noise.vae_masked)
        crop = rgb[y * DOWN:(y + h) * DOWN, x * DOWN:(x + w) * DOWN][None]
        part = vae.encode(np.ascontiguousarray(crop), np.ascontiguousarray(noise.vae_img[:, y:y + h, x:x + w]))
        ix, iy, iw, ih = roi_window(mask_lat, ROI_MARGIN // 2)
        z_img = z_masked.copy()
        z_img[:, iy:iy + ih, ix:ix + iw] = part[:, iy - y:iy - y + ih, ix - x:ix - x + iw]
    else:
        z = vae.encode(np.stack([rgb, masked]), np.concatenate([noise.vae_img, noise.vae_masked]))
        z_img, z_masked = z[:1], z[1:]

    init = (noise.init + np.float32(params.noise_offset) * noise.offset).astype(np.float32)
    lat = denoise(unet, z_img, init, mask_lat, z_masked, params.steps, params.strength, params.spacing,
                  params.solver, params.guidance, params.cfg_steps)

    roi = roi_window(mask_lat, ROI_MARGIN) if params.roi_decode else None
    if roi is not None and (roi[2] < LATENT or roi[3] < LATENT):
        x, y, w, h = roi
        part = vae.decode(np.ascontiguousarray(lat[:, y:y + h, x:x + w]))
        dec = ((rgb + np.float32(1.0)) * np.float32(0.5))[None]
        dec[:, y * DOWN:(y + h) * DOWN, x * DOWN:(x + w) * DOWN] = part
    else:
        dec = vae.decode(lat)
    u8 = to_u8(dec[0])
    result = u8 if plan.side == IMAGE_SIZE else resize_u8(u8, plan.side, plan.side)
    return result, plan, lat


def paste_none(img: np.ndarray, result: np.ndarray, plan: Plan):
    """src/imaging/blend.rs:155-173 (Paste::None): the window's in-image part
    over img (RGB channels; alpha kept). Returns the rectangle written."""
    x, y, w, h = source_rect(plan, img.shape[1], img.shape[0])
    ox, oy = x - plan.x, y - plan.y
    img[y:y + h, x:x + w, :3] = result[oy:oy + h, ox:ox + w]
    return x, y, w, h
