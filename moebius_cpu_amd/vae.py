"""The device VAE over the C ABI (mh_vae_*), mirroring src/vae/mod.rs
`Vae::{load, encode, decode}`."""
from __future__ import annotations

import ctypes

import numpy as np

from . import _lib
from ._lib import check, lib
from .engine import Context, DeviceArray
from .vae_params import vae_specs


class Vae:
    """Weights copied to HBM at construction; encode / decode run on the device."""

    def __init__(self, ctx: Context, params: dict, f16_gemm: bool = False):
        """params: converter tensors as f32 arrays; f16_gemm stores the conv and
        linear weights as f16, as the converter's --dtype f16 does
        (tools/convert_weights.py:27-30)."""
        self.ctx = ctx
        gemm = {s.name for s in vae_specs() if s.gemm}
        keep = []
        arr = (_lib.NamedTensor * len(params))()
        for i, (name, v) in enumerate(params.items()):
            if f16_gemm and name in gemm:
                a, dt = np.ascontiguousarray(v, dtype=np.float16), _lib.DTYPE_F16
            else:
                a, dt = np.ascontiguousarray(v, dtype=np.float32), _lib.DTYPE_F32
            keep.append(a)
            arr[i].name = name.encode()
            arr[i].data = a.ctypes.data
            arr[i].dtype = dt
            arr[i].numel = a.size
        h = ctypes.c_void_p()
        check(lib().mh_vae_create(ctx.h, arr, len(params), ctypes.byref(h)))
        self.h = h
        ctx.adopt(self)

    @classmethod
    def from_file(cls, ctx: Context, path: str) -> "Vae":
        """Loads a converter safetensors file (mh_vae_create_from_file): format-tag and shape checked."""
        self = cls.__new__(cls)
        self.ctx = ctx
        h = ctypes.c_void_p()
        check(lib().mh_vae_create_from_file(ctx.h, str(path).encode(), ctypes.byref(h)))
        self.h = h
        ctx.adopt(self)
        return self

    def close(self):
        if getattr(self, "h", None):
            lib().mh_vae_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _tracer(self, traced):
        def cb(_user, name, dev, n, h, w, c):
            out = np.empty((n, h, w, c), np.float32)
            check(lib().mh_memcpy_d2h(self.ctx.h, out.ctypes.data, dev, out.nbytes))
            traced[name.decode()] = out

        return _lib.TRACE_FN(cb)

    def encode(self, images_dev: DeviceArray, noise_dev: DeviceArray, z_dev: DeviceArray):
        """Device in / device out, asynchronous: images [b,h,w,3], noise and z [b,h/8,w/8,4]."""
        b, h, w, _ = images_dev.shape
        check(lib().mh_vae_encode(self.h, images_dev.ptr, b, h, w, noise_dev.ptr, z_dev.ptr, None, None))

    def decode(self, latents_dev: DeviceArray, out_dev: DeviceArray):
        """Device in / device out, asynchronous: latents [1,h,w,4] -> out [1,8h,8w,3]."""
        _, h, w, _ = latents_dev.shape
        check(lib().mh_vae_decode(self.h, latents_dev.ptr, h, w, out_dev.ptr, None, None))

    def encode_host(self, images: np.ndarray, noise: np.ndarray) -> np.ndarray:
        images = np.ascontiguousarray(images, dtype=np.float32)
        noise = np.ascontiguousarray(noise, dtype=np.float32)
        b, h, w, _ = images.shape
        z = np.empty((b, h // 8, w // 8, 4), np.float32)
        check(lib().mh_vae_encode_host(self.h, images.ctypes.data, b, h, w, noise.ctypes.data, z.ctypes.data))
        return z

    def decode_host(self, latents: np.ndarray) -> np.ndarray:
        latents = np.ascontiguousarray(latents, dtype=np.float32)
        _, h, w, _ = latents.shape
        out = np.empty((1, 8 * h, 8 * w, 3), np.float32)
        check(lib().mh_vae_decode_host(self.h, latents.ctypes.data, h, w, out.ctypes.data))
        return out

    def encode_traced(self, images: np.ndarray, noise: np.ndarray):
        """(z, {block name: host copy}) with the oracle's trace names."""
        images = np.ascontiguousarray(images, dtype=np.float32)
        b, h, w, _ = images.shape
        xd = DeviceArray.from_numpy(self.ctx, images)
        nd = DeviceArray.from_numpy(self.ctx, np.ascontiguousarray(noise, dtype=np.float32))
        z = DeviceArray(self.ctx, (b, h // 8, w // 8, 4))
        traced = {}
        fn = self._tracer(traced)
        check(lib().mh_vae_encode(self.h, xd.ptr, b, h, w, nd.ptr, z.ptr, fn, None))
        return z.numpy(), traced

    def decode_traced(self, latents: np.ndarray):
        """(image, {block name: host copy}) with the oracle's trace names."""
        latents = np.ascontiguousarray(latents, dtype=np.float32)
        _, h, w, _ = latents.shape
        ld = DeviceArray.from_numpy(self.ctx, latents)
        out = DeviceArray(self.ctx, (1, 8 * h, 8 * w, 3))
        traced = {}
        fn = self._tracer(traced)
        check(lib().mh_vae_decode(self.h, ld.ptr, h, w, out.ptr, fn, None))
        return out.numpy(), traced

    def memory(self):
        w, p = ctypes.c_uint64(), ctypes.c_uint64()
        check(lib().mh_vae_memory(self.h, ctypes.byref(w), ctypes.byref(p)))
        return int(w.value), int(p.value)
