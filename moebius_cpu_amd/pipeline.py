"""End-to-end inpainting on the GPU, mirroring the reference's `Engine`
(src/pipeline.rs:113-213) and presets (src/preset.rs) over the C ABI of
include/moebius_engine.h.

    eng = Engine.load("weights/")                  # unet.safetensors + vae.safetensors
    rect = eng.inpaint(img, mask)                  # img: HxWx3|4 uint8, edited in place
    rect = eng.inpaint(img, mask, Preset.FAST.params())

Host arrays in, host arrays out; everything between the mask's window and the
paste runs on the device. Errors raise MoebiusError (ERR_CANCELLED when the
progress callback returns Control.CANCEL; the image is then untouched).
"""
from __future__ import annotations

import ctypes
import dataclasses
import enum
from typing import Callable, Optional

import numpy as np

from . import _lib


class Preset(enum.IntEnum):
    """src/preset.rs:8-12."""
    EXACT = 0
    FAST = 1

    def params(self) -> "InpaintParams":
        """src/preset.rs:60-82 Preset::params."""
        return InpaintParams.resolve(preset=int(self))


class Stage(enum.IntEnum):
    """src/pipeline.rs:53-58."""
    ENCODE = 0
    DENOISE = 1
    DECODE = 2


class Control(enum.IntEnum):
    """src/pipeline.rs:60-65."""
    CONTINUE = 0
    CANCEL = 1


@dataclasses.dataclass(frozen=True)
class Progress:
    stage: Stage
    done: int
    total: int


@dataclasses.dataclass(frozen=True)
class Rect:
    x: int = 0
    y: int = 0
    w: int = 0
    h: int = 0


@dataclasses.dataclass
class InpaintParams:
    """src/preset.rs:34-58 (cfg_steps None = CFG on every step), plus the
    UNet's arithmetic (`precision`: "exact" f32 MFMA, "fast" f16 MFMA)."""
    steps: int
    strength: float
    spacing: str
    solver: str
    guidance: float
    noise_offset: float
    seed: int
    cfg_steps: Optional[int]
    roi_encode: bool
    roi_decode: bool
    paste: str
    mask_dilate: int
    precision: str = "exact"

    @staticmethod
    def resolve(preset: int = 0, steps: int = 0, guidance: float = 0.0, seed: int = 0, paste: str = "default",
                mask_dilate: int = 0) -> "InpaintParams":
        """src/ffi.rs:227-250: a preset with the C API's overrides."""
        m = _lib.MoebiusParams(preset, steps, guidance, seed, _lib.PASTE[paste], mask_dilate)
        c = _lib.InpaintParams()
        _lib.check(_lib.lib().mh_inpaint_params(ctypes.byref(m), ctypes.byref(c)))
        return InpaintParams.from_c(c)

    @staticmethod
    def from_c(c: "_lib.InpaintParams") -> "InpaintParams":
        inv = lambda d, v: next(k for k, x in d.items() if x == v)  # noqa: E731
        return InpaintParams(
            steps=c.steps, strength=c.strength, spacing=inv(_lib.SPACING, c.spacing),
            solver=inv(_lib.SOLVER, c.solver), guidance=c.guidance, noise_offset=c.noise_offset, seed=c.seed,
            cfg_steps=None if c.cfg_steps < 0 else c.cfg_steps, roi_encode=bool(c.roi_encode),
            roi_decode=bool(c.roi_decode), paste=inv(_lib.PASTE, c.paste), mask_dilate=c.mask_dilate,
            precision="fast" if c.precision == _lib.PRECISION_FAST else "exact")

    def to_c(self) -> "_lib.InpaintParams":
        return _lib.InpaintParams(
            steps=self.steps, spacing=_lib.SPACING[self.spacing], solver=_lib.SOLVER[self.solver],
            cfg_steps=-1 if self.cfg_steps is None else self.cfg_steps, strength=self.strength,
            guidance=self.guidance, noise_offset=self.noise_offset, seed=self.seed,
            roi_encode=int(self.roi_encode), roi_decode=int(self.roi_decode), paste=_lib.PASTE[self.paste],
            mask_dilate=self.mask_dilate,
            precision=_lib.PRECISION_FAST if self.precision == "fast" else _lib.PRECISION_EXACT, reserved=0)


@dataclasses.dataclass
class NoiseSet:
    """src/pipeline.rs:64-111: the normals one inpaint consumes, NHWC f32."""
    vae_img: np.ndarray     # [1,64,64,4]
    vae_masked: np.ndarray  # [1,64,64,4]
    init: np.ndarray        # [1,64,64,4]
    offset: np.ndarray      # [1,1,1,4]

    @staticmethod
    def sample(seed: int) -> "NoiseSet":
        """The library's seeded generator (not the CPU engine's StdRng stream)."""
        buf = np.empty(_lib.NOISE_FLOATS, np.float32)
        _lib.check(_lib.lib().mh_sample_noise(seed, buf.ctypes.data))
        return NoiseSet.from_flat(buf)

    @staticmethod
    def from_flat(buf: np.ndarray) -> "NoiseSet":
        n = 64 * 64 * 4
        return NoiseSet(buf[:n].reshape(1, 64, 64, 4), buf[n:2 * n].reshape(1, 64, 64, 4),
                        buf[2 * n:3 * n].reshape(1, 64, 64, 4), buf[3 * n:].reshape(1, 1, 1, 4))

    def flat(self) -> np.ndarray:
        parts = (self.vae_img, self.vae_masked, self.init, self.offset)
        shapes = ((1, 64, 64, 4),) * 3 + ((1, 1, 1, 4),)
        for name, p, s in zip(("vae_img", "vae_masked", "init", "offset"), parts, shapes):
            if tuple(p.shape) != s:  # src/pipeline.rs:94-110 NoiseSet::check
                raise _lib.MoebiusError(_lib.ERR_INVALID_ARGUMENT,
                                        f"noise.{name} has shape {list(p.shape)}, expected {list(s)}")
        return np.ascontiguousarray(np.concatenate([np.asarray(p, np.float32).ravel() for p in parts]))


def _views(img: np.ndarray, mask: np.ndarray):
    if img.dtype != np.uint8 or img.ndim != 3 or mask.dtype != np.uint8 or mask.ndim != 2:
        raise _lib.MoebiusError(_lib.ERR_INVALID_ARGUMENT, "image must be HxWxC uint8 and mask HxW uint8")
    if img.strides[2] != 1 or img.strides[1] != img.shape[2] or mask.strides[1] != 1:
        raise _lib.MoebiusError(_lib.ERR_INVALID_ARGUMENT, "pixels and mask rows must be packed")
    h, w, c = img.shape
    return w, h, img.strides[0], c, mask.strides[0]


class Engine:
    """src/pipeline.rs:113-138: UNet + VAE resident on one GPU."""

    def __init__(self, handle: int):
        self._h = ctypes.c_void_p(handle)

    @staticmethod
    def load(weights_dir: str, threads: int = 0, device: Optional[int] = None) -> "Engine":
        """`weights_dir` holds unet.safetensors and vae.safetensors; `threads` is
        accepted for the reference's signature and ignored."""
        out = ctypes.c_void_p()
        L = _lib.lib()
        d = weights_dir.encode()
        if device is None:
            st = L.moebius_engine_create(d, threads, ctypes.byref(out))
        else:
            st = L.mh_engine_create(device, d, ctypes.byref(out))
        _lib.check(st)
        return Engine(out.value)

    def close(self) -> None:
        if self._h:
            _lib.lib().moebius_engine_destroy(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def memory(self):
        wb, pb = ctypes.c_uint64(), ctypes.c_uint64()
        _lib.check(_lib.lib().mh_engine_memory(self._h, ctypes.byref(wb), ctypes.byref(pb)))
        return wb.value, pb.value

    def release_scratch(self) -> None:
        """Frees the activation pools and workspace until the next call."""
        _lib.check(_lib.lib().mh_engine_release_scratch(self._h))

    @staticmethod
    def _progress(fn: Optional[Callable[[Progress], Control]]):
        if fn is None:
            return None

        def cb(_user, stage, done, total):
            r = fn(Progress(Stage(stage), done, total))
            return 1 if r == Control.CANCEL else 0
        return _lib.PROGRESS_FN(cb)

    def inpaint(self, img: np.ndarray, mask: np.ndarray, params: Optional[InpaintParams] = None,
                progress: Optional[Callable[[Progress], Control]] = None) -> Rect:
        """src/pipeline.rs:140-149: in place where mask >= 128; noise from params.seed."""
        p = params or Preset.EXACT.params()
        return self.inpaint_with_noise(img, mask, p, NoiseSet.sample(p.seed), progress)

    def inpaint_with_noise(self, img, mask, params: InpaintParams, noise: NoiseSet, progress=None) -> Rect:
        """src/pipeline.rs:151-161."""
        return self.inpaint_traced(img, mask, params, noise, progress)[0]

    def inpaint_traced(self, img, mask, params: InpaintParams, noise: NoiseSet, progress=None, latents=False):
        """src/pipeline.rs:163-213: (rect, final scaled latents [1,64,64,4] or None)."""
        w, h, stride, c, mstride = _views(img, mask)
        if mask.shape != img.shape[:2]:
            raise _lib.MoebiusError(_lib.ERR_INVALID_ARGUMENT, "image and mask sizes differ")
        flat = noise.flat()
        lat = np.empty((1, 64, 64, 4), np.float32) if latents else None
        rect = _lib.MoebiusRect()
        cp = params.to_c()
        cb = self._progress(progress)
        _lib.check(_lib.lib().mh_inpaint_with_noise(
            self._h, img.ctypes.data, w, h, stride, c, mask.ctypes.data, mstride, ctypes.byref(cp),
            flat.ctypes.data, cb, None, ctypes.byref(rect), None if lat is None else lat.ctypes.data))
        return Rect(rect.x, rect.y, rect.width, rect.height), lat
