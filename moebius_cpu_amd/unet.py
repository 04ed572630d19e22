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
