"""The device UNet over the C ABI (mh_unet_*), mirroring src/unet/mod.rs
`UNet::{load, forward, forward_traced}`."""
from __future__ import annotations

import ctypes

import numpy as np

from . import _lib
from ._lib import check, lib
from .engine import Context, DeviceArray
from .unet_params import unet_specs


class UNet:
    """Weights copied to HBM at construction; `forward*` run one denoise step."""

    def __init__(self, ctx: Context, params: dict, f16_gemm: bool = False):
        """params: converter tensors as f32 arrays; f16_gemm stores the GEMM
        weights (2-D linears / 1x1 and dense 3x3) as f16, as the converter's
        --dtype f16 does (tools/convert_weights.py:27-30)."""
        self.ctx = ctx
        gemm = {s.name for s in unet_specs() if s.gemm}
        keep = []
        arr = (_lib.NamedTensor * len(params))()
        for i, (name, v) in enumerate(params.items()):
            if f16_gemm and name in gemm:
                a = np.ascontiguousarray(v, dtype=np.float16)
                dt = _lib.DTYPE_F16
            else:
                a = np.ascontiguousarray(v, dtype=np.float32)
                dt = _lib.DTYPE_F32
            keep.append(a)
            arr[i].name = name.encode()
            arr[i].data = a.ctypes.data
            arr[i].dtype = dt
            arr[i].numel = a.size
        h = ctypes.c_void_p()
        check(lib().mh_unet_create(ctx.h, arr, len(params), ctypes.byref(h)))
        self.h = h
        ctx.adopt(self)

    @classmethod
    def from_file(cls, ctx: Context, path: str) -> "UNet":
        """Loads a converter safetensors file (mh_unet_create_from_file): format-tag and shape checked."""
        self = cls.__new__(cls)
        self.ctx = ctx
        h = ctypes.c_void_p()
        check(lib().mh_unet_create_from_file(ctx.h, str(path).encode(), ctypes.byref(h)))
        self.h = h
        ctx.adopt(self)
        return self

    def close(self):
        if getattr(self, "h", None):
            lib().mh_unet_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @staticmethod
    def _guidance(cfg: bool) -> int:
        return _lib.GUIDANCE_CFG if cfg else _lib.GUIDANCE_COND_ONLY

    def forward_host(self, x: np.ndarray, timestep: int, cfg: bool = True) -> np.ndarray:
        """x [1,64,64,9] host -> eps [b,64,64,4] host."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        assert x.shape == (1, 64, 64, 9), "UNet input is [1, 64, 64, 9]"
        eps = np.empty((2 if cfg else 1, 64, 64, 4), np.float32)
        check(lib().mh_unet_forward_host(self.h, x.ctypes.data, int(timestep), self._guidance(cfg), eps.ctypes.data))
        return eps

    def forward(self, x_dev: DeviceArray, timestep: int, cfg: bool, eps_dev: DeviceArray):
        """Device in / device out, asynchronous on the context stream."""
        check(lib().mh_unet_forward(self.h, x_dev.ptr, int(timestep), self._guidance(cfg), eps_dev.ptr))

    def forward_traced(self, x: np.ndarray, timestep: int, cfg: bool = True):
        """(eps, {block name: host copy}) with the reference's trace names."""
        xd = DeviceArray.from_numpy(self.ctx, np.ascontiguousarray(x, dtype=np.float32))
        eps = DeviceArray(self.ctx, (2 if cfg else 1, 64, 64, 4))
        traced = {}

        def cb(_user, name, dev, n, h, w, c):
            out = np.empty((n, h, w, c), np.float32)
            check(lib().mh_memcpy_d2h(self.ctx.h, out.ctypes.data, dev, out.nbytes))
            traced[name.decode()] = out

        fn = _lib.TRACE_FN(cb)
        check(lib().mh_unet_forward_traced(self.h, xd.ptr, int(timestep), self._guidance(cfg), eps.ptr, fn, None))
        return eps.numpy(), traced

    def memory(self):
        w, p = ctypes.c_uint64(), ctypes.c_uint64()
        check(lib().mh_unet_memory(self.h, ctypes.byref(w), ctypes.byref(p)))
        return int(w.value), int(p.value)


class Scheduler:
    """src/scheduler.rs `Ddim` + `Dpm2M` on device arrays of `length` floats
    (mh_scheduler_*): timesteps and alphas on the host, updates on the device."""

    def __init__(self, ctx: Context, steps: int, strength: float, spacing: str = "leading", length: int = 64 * 64 * 4):
        self.ctx = ctx
        h = ctypes.c_void_p()
        check(lib().mh_scheduler_create(ctx.h, int(steps), float(strength), _lib.SPACING[spacing], int(length),
                                        ctypes.byref(h)))
        self.h = h
        self.timesteps, self.pure_noise_start = schedule_timesteps(steps, strength, spacing)
        ctx.adopt(self)

    def close(self):
        if getattr(self, "h", None):
            lib().mh_scheduler_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def add_noise(self, x0: DeviceArray, noise: DeviceArray, t: int, out: DeviceArray):
        check(lib().mh_scheduler_add_noise(self.h, x0.ptr, noise.ptr, int(t), out.ptr))

    def ddim_step(self, eps_u: DeviceArray, eps_c, guidance: float, t: int, x: DeviceArray):
        check(lib().mh_scheduler_ddim_step(self.h, eps_u.ptr, eps_c.ptr if eps_c is not None else None,
                                           float(guidance), int(t), x.ptr))

    def dpm_step(self, eps_u: DeviceArray, eps_c, guidance: float, i: int, x: DeviceArray):
        check(lib().mh_scheduler_dpm_step(self.h, eps_u.ptr, eps_c.ptr if eps_c is not None else None,
                                          float(guidance), int(i), x.ptr))

    def dpm_restart(self):
        check(lib().mh_scheduler_dpm_restart(self.h))


def schedule_timesteps(steps: int, strength: float, spacing: str = "leading"):
    """(timesteps, pure_noise_start) of src/scheduler.rs:30-76, computed by the library on the host."""
    out = (ctypes.c_uint32 * 1000)()
    n, pure = ctypes.c_uint32(), ctypes.c_uint32()
    check(lib().mh_schedule_timesteps(int(steps), float(strength), _lib.SPACING[spacing], out, ctypes.byref(n),
                                      ctypes.byref(pure)))
    return [int(out[i]) for i in range(n.value)], bool(pure.value)


def schedule_alphas_cumprod() -> np.ndarray:
    out = np.empty(1000, np.float32)
    check(lib().mh_schedule_alphas_cumprod(out.ctypes.data))
    return out


def denoise(net: "UNet", z_img, init, mask_lat, z_masked, steps: int = 20, strength: float = 0.99,
            spacing: str = "leading", solver: str = "ddim", guidance: float = 2.5, cfg_steps=None, progress=None):
    """src/pipeline.rs:295-345 on the device (mh_unet_denoise) from host arrays:
    z_img, init, z_masked [1,64,64,4], mask_lat [1,64,64,1]; returns the final
    latents [1,64,64,4]. progress(done, total) -> truthy cancels."""
    ctx = net.ctx
    arrs = [None if a is None else DeviceArray.from_numpy(ctx, np.ascontiguousarray(a, np.float32))
            for a in (z_img, init, mask_lat, z_masked)]
    out = DeviceArray(ctx, (1, 64, 64, 4))
    prm = _lib.DenoiseParams(strength=float(strength), guidance=float(guidance), steps=int(steps),
                             spacing=_lib.SPACING[spacing], solver=_lib.SOLVER[solver],
                             cfg_steps=-1 if cfg_steps is None else int(cfg_steps), reserved=0)
    cb = _lib.STEP_FN(lambda _u, done, total: 1 if progress is not None and progress(done, total) else 0)
    check(lib().mh_unet_denoise(net.h, arrs[0].ptr if arrs[0] is not None else None, arrs[1].ptr, arrs[2].ptr,
                                arrs[3].ptr, ctypes.byref(prm), cb, None, out.ptr))
    return out.numpy()
