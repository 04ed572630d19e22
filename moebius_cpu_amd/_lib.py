"""ctypes declarations of include/moebius_hip.h and include/moebius_engine.h
over libmoebius_hip.so.

Loading fails loudly when the library is missing: there is no CPU fallback.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libmoebius_hip.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "moebius_hip.h")
ENGINE_HEADER = os.path.join(os.path.dirname(HERE), "include", "moebius_engine.h")
HEADERS = (HEADER, ENGINE_HEADER)

OK = 0
ERR_INVALID_ARGUMENT = 1
ERR_WEIGHTS = 2
ERR_UNSUPPORTED_DEVICE = 3
ERR_CANCELLED = 4
ERR_IO = 5
ERR_INTERNAL = 6
ERR_OUT_OF_MEMORY = 7

DTYPE_F32 = 0
DTYPE_F16 = 1
EPILOGUE = {"none": 0, "relu": 1, "glu_silu": 2}
PRECISION_EXACT = 0
PRECISION_FAST = 1


class MoebiusError(RuntimeError):
    """A non-zero status from the C API, with mh_last_error's message."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"[{code}] {msg}")
        self.code = code
        self.msg = msg


_vp = ctypes.c_void_p
_u32 = ctypes.c_uint32
_u64 = ctypes.c_uint64
_i32 = ctypes.c_int32
_f32 = ctypes.c_float
_u32p = ctypes.POINTER(ctypes.c_uint32)

# name -> (restype, argtypes); every function the two headers declare.
SIGNATURES = {
    "mh_abi_version": (_u32, []),
    "mh_last_error": (ctypes.c_char_p, []),
    "mh_context_create": (_i32, [_i32, ctypes.POINTER(_vp)]),
    "mh_context_destroy": (None, [_vp]),
    "mh_context_set_precision": (_i32, [_vp, _u32]),
    "mh_context_set_tuning": (_i32, [_vp, ctypes.c_char_p, ctypes.c_char_p]),
    "mh_device_allocations": (_i32, [ctypes.POINTER(ctypes.c_uint64)]),
    "mh_context_gemm_times": (_i32, [_vp, ctypes.c_char_p, _u64, ctypes.POINTER(_u64)]),
    "mh_context_stream": (_vp, [_vp]),
    "mh_synchronize": (_i32, [_vp]),
    "mh_device_arch": (_i32, [_vp, ctypes.c_char_p, _u32]),
    "mh_malloc": (_i32, [_vp, _u64, ctypes.POINTER(_vp)]),
    "mh_free": (_i32, [_vp, _vp]),
    "mh_memcpy_h2d": (_i32, [_vp, _vp, _vp, _u64]),
    "mh_memcpy_d2h": (_i32, [_vp, _vp, _vp, _u64]),
    "mh_memcpy_d2d": (_i32, [_vp, _vp, _vp, _u64]),
    "mh_event_create": (_i32, [_vp, ctypes.POINTER(_vp)]),
    "mh_event_record": (_i32, [_vp, _vp]),
    "mh_event_elapsed_ms": (_i32, [_vp, _vp, ctypes.POINTER(_f32)]),
    "mh_event_destroy": (None, [_vp]),
    "mh_bias_residual_add": (_i32, [_vp, _vp, _u64, _u32, _vp, _vp, _vp]),
    "mh_conv1x1_forward": (_i32, [_vp, _vp, _u32, _u32, _u32, _u32, _vp, _u32, _u32, _vp, _vp, _vp]),
    "mh_conv1x1_fused": (_i32, [_vp, _vp, _u32, _u32, _u32, _u32, _vp, _u32, _u32, _vp, _vp, _vp, _vp, _u32, _vp,
                                 _vp]),
    "mh_conv1x1_gn_partials": (_i32, [_vp, _vp, _u32, _u32, _u32, _u32, _vp, _u32, _u32, _vp, _vp, _vp, _vp, _u32p]),
    "mh_group_norm_affine_partials": (_i32, [_vp, _vp, _u32, _u32, _u32, _u32, _u32, _u32, _f32, _vp, _vp, _vp, _vp,
                                             _vp]),
    "mh_conv3x3_output_hw": (_i32, [_u32, _u32, _u32, _u32p, _u32, _u32p, _u32p]),
    "mh_conv3x3_forward": (_i32, [_vp, _vp, _u32, _u32, _u32, _u32, _vp, _u32, _u32, _vp, _u32, _u32p, _u32,
                                  _vp, _vp, _u32, _vp]),
    "mh_winograd_weight_transform": (_i32, [_vp, _vp, _u32, _u32, _u32, _vp]),
    "mh_winograd_input_transform": (_i32, [_vp, _vp, _u32, _u32, _u32, _u32, _u32, _vp, _vp, _u32, _vp]),
    "mh_winograd_output_transform": (_i32, [_vp, _vp, _u32, _u32, _u32, _u32, _u32, _vp, _vp]),
    "mh_conv3x3_winograd": (_i32, [_vp, _vp, _u32, _u32, _u32, _u32, _vp, _u32, _vp, _u32, _vp, _vp, _u32, _vp]),
    "mh_im2col_gather": (_i32, [_vp, _vp, _u32, _u32, _u32, _u32, _u32, _u32p, _u32, _u64, _u64, _vp]),
    "mh_depthwise3x3": (_i32, [_vp, _vp, _u32, _u32, _u32, _u32, _vp, _vp, _u32, _vp]),
    "mh_depthwise3x3_fused": (_i32, [_vp, _vp, _u32, _u32, _u32, _u32, _vp, _vp, _u32, _vp, _vp, _u32, _vp]),
    "mh_group_norm_affine": (_i32, [_vp, _vp, _u32, _u32, _u32, _u32, _u32, _f32, _vp, _vp, _vp, _vp, _vp]),
    "mh_group_norm_forward": (_i32, [_vp, _vp, _u32, _u32, _u32, _u32, _u32, _f32, _vp, _vp, _vp, _u32, _vp]),
    "mh_group_norm_forward_noalloc": (_i32, [_vp, _vp, _u32, _u32, _u32, _u32, _u32, _f32, _vp, _vp, _vp, _u32,
                                             _vp]),
    "mh_apply_affine": (_i32, [_vp, _vp, _u32, _u32, _u32, _u32, _vp, _vp, _u32, _vp]),
    "mh_layer_norm": (_i32, [_vp, _vp, _u64, _u32, _vp, _vp, _f32, _vp]),
    "mh_conv1x1_layer_norm": (_i32, [_vp, _vp, _u64, _u32, _vp, _vp, _f32, _vp, _u32, _u32, _vp, _u32, _vp]),
    "mh_conv1x1_layer_norm_stats": (_i32, [_vp, _vp, _u64, _u32, _vp, _vp, _f32, _vp, _u32, _u32, _vp, _u32, _vp,
                                           _u32, _vp]),
    "mh_conv1x1_row_partials": (_i32, [_vp, _vp, _u64, _u32, _vp, _u32, _u32, _vp, _vp, _vp, ctypes.POINTER(_u32)]),
    "mh_silu_inplace": (_i32, [_vp, _vp, _u64]),
    "mh_add_inplace": (_i32, [_vp, _vp, _vp, _u64]),
    "mh_concat_channels": (_i32, [_vp, _vp, _u32, _vp, _u32, _u64, _vp]),
    "mh_to_u8": (_i32, [_vp, _vp, _u64, _vp]),
    "mh_math_eval": (_i32, [_vp, _u32, _vp, _u64, _vp]),
    "mh_selftest_mfma_f32": (_i32, [_vp, _vp, _vp, _vp]),
    "mh_softmax_lambda": (_i32, [_vp, _vp, _vp, _u32, _u32, _u32, _u32, _vp]),
    "mh_tap_filter": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32]),
    "mh_tap_filter_row_sums": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _vp,
                                      ctypes.POINTER(_u32)]),
    "mh_tap_filter_ln": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _vp, _vp, _f32, _vp]),
    "mh_lambda_position_coeffs": (_i32, [_vp, _vp, _vp, _vp, _u32, _u32, _u32, _vp, _vp]),
    "mh_self_lambda_fused": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _vp]),
    "mh_position_term": (_i32, [_vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _vp, _vp, _vp]),
    "mh_cross_lambda": (_i32, [_vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _vp, _vp]),
    "mh_cross_lambda_row_sums": (_i32, [_vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _vp, _vp, _vp]),
    "mh_gemm_nt": (_i32, [_vp, _vp, _u64, _vp, _u32, _u64, _u32, _u32, _u32, _vp, _vp, _vp, _u64, _u32]),
    "mh_unet_create": (_i32, [_vp, _vp, _u32, ctypes.POINTER(_vp)]),
    "mh_unet_destroy": (None, [_vp]),
    "mh_unet_forward": (_i32, [_vp, _vp, _u32, _u32, _vp]),
    "mh_unet_forward_host": (_i32, [_vp, _vp, _u32, _u32, _vp]),
    "mh_unet_forward_traced": (_i32, [_vp, _vp, _u32, _u32, _vp, _vp, _vp]),
    "mh_unet_memory": (_i32, [_vp, ctypes.POINTER(_u64), ctypes.POINTER(_u64)]),
    "mh_weights_validate": (_i32, [ctypes.c_char_p, _u32]),
    "mh_unet_create_from_file": (_i32, [_vp, ctypes.c_char_p, ctypes.POINTER(_vp)]),
    "mh_vae_create_from_file": (_i32, [_vp, ctypes.c_char_p, ctypes.POINTER(_vp)]),
    "mh_mask_bbox": (_i32, [_vp, _u32, _u32, _u32, _u32p, _u32p]),
    "mh_mask_dilate": (_i32, [_vp, _u32, _u32, _u32, _u32, _vp]),
    "mh_crop_plan": (_i32, [_u32p, _u32, _u32, ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(ctypes.c_int64),
                            _u32p]),
    "mh_gaussian_blur": (_i32, [_vp, _u32, _u32, _f32, _vp]),
    "mh_paste": (_i32, [_vp, _u32, _u32, _u32, _u32, _vp, _u32, _vp, ctypes.c_int64, ctypes.c_int64, _u32, _u32,
                        _u32p]),
    "mh_resize_u8": (_i32, [_vp, _vp, _u32, _u32, _u32, _u32, _u32, _vp]),
    "mh_roi_window": (_i32, [_vp, _u32, _u32p, _u32p]),
    "mh_schedule_timesteps": (_i32, [_u32, ctypes.c_double, _u32, _u32p, _u32p, _u32p]),
    "mh_schedule_alphas_cumprod": (_i32, [_vp]),
    "mh_scheduler_create": (_i32, [_vp, _u32, ctypes.c_double, _u32, _u64, ctypes.POINTER(_vp)]),
    "mh_scheduler_destroy": (None, [_vp]),
    "mh_scheduler_add_noise": (_i32, [_vp, _vp, _vp, _u32, _vp]),
    "mh_scheduler_ddim_step": (_i32, [_vp, _vp, _vp, _f32, _u32, _vp]),
    "mh_scheduler_dpm_step": (_i32, [_vp, _vp, _vp, _f32, _u32, _vp]),
    "mh_scheduler_dpm_restart": (_i32, [_vp]),
    "mh_unet_denoise": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "mh_vae_create": (_i32, [_vp, _vp, _u32, _vp]),
    "mh_vae_destroy": (None, [_vp]),
    "mh_vae_encode": (_i32, [_vp, _vp, _u32, _u32, _u32, _vp, _vp, _vp, _vp]),
    "mh_vae_decode": (_i32, [_vp, _vp, _u32, _u32, _vp, _vp, _vp]),
    "mh_vae_encode_host": (_i32, [_vp, _vp, _u32, _u32, _u32, _vp, _vp]),
    "mh_vae_decode_host": (_i32, [_vp, _vp, _u32, _u32, _vp]),
    "mh_vae_memory": (_i32, [_vp, _vp, _vp]),
    "mh_softmax_rows": (_i32, [_vp, _vp, _u64, _u32, _f32]),
    "mh_vae_sample": (_i32, [_vp, _vp, _vp, _u64, _vp]),
    "mh_timestep_sinusoid": (None, [_u32, _vp]),
    "mh_scratch_best_fit": (ctypes.c_int64, [_vp, _vp, _u64, _u64]),
    # include/moebius_engine.h
    "moebius_abi_version": (_u32, []),
    "moebius_last_error": (ctypes.c_char_p, []),
    "moebius_engine_create": (_i32, [ctypes.c_char_p, _u32, ctypes.POINTER(_vp)]),
    "moebius_engine_destroy": (None, [_vp]),
    "moebius_inpaint": (_i32, [_vp, _vp, _u32, _u32, _u32, _u32, _vp, _u32, _vp, _vp, _vp, _vp]),
    "mh_inpaint_params": (_i32, [_vp, _vp]),
    "mh_sample_noise": (_i32, [_u64, _vp]),
    "mh_engine_create": (_i32, [_i32, ctypes.c_char_p, ctypes.POINTER(_vp)]),
    "mh_inpaint_with_noise": (_i32, [_vp, _vp, _u32, _u32, _u32, _u32, _vp, _u32, _vp, _vp, _vp, _vp, _vp, _vp]),
    "mh_engine_memory": (_i32, [_vp, ctypes.POINTER(_u64), ctypes.POINTER(_u64)]),
    "mh_engine_release_scratch": (_i32, [_vp]),
}

GUIDANCE_CFG = 0
GUIDANCE_COND_ONLY = 1


class NamedTensor(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("data", ctypes.c_void_p), ("dtype", ctypes.c_uint32),
                ("reserved", ctypes.c_uint32), ("numel", ctypes.c_uint64)]


class DenoiseParams(ctypes.Structure):
    """include/moebius_hip.h MhDenoiseParams (src/preset.rs InpaintParams' sampling fields)."""
    _fields_ = [("strength", ctypes.c_double), ("guidance", ctypes.c_float), ("steps", ctypes.c_uint32),
                ("spacing", ctypes.c_uint32), ("solver", ctypes.c_uint32), ("cfg_steps", ctypes.c_int32),
                ("reserved", ctypes.c_uint32)]


MODEL_UNET = 0
MODEL_VAE = 1
SPACING = {"leading": 0, "trailing": 1}
SOLVER = {"ddim": 0, "dpm": 1}
STEP_FN = ctypes.CFUNCTYPE(ctypes.c_int32, ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint32)

PRESET = {"exact": 0, "fast": 1}
PASTE = {"default": 0, "none": 1, "feather": 2, "feather_compensate": 3}
PROGRESS_FN = ctypes.CFUNCTYPE(ctypes.c_int32, ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32)
NOISE_FLOATS = 3 * 64 * 64 * 4 + 4


class MoebiusParams(ctypes.Structure):
    """include/moebius_engine.h MoebiusParams (src/ffi.rs:43-53)."""
    _fields_ = [("preset", ctypes.c_uint32), ("steps", ctypes.c_uint32), ("guidance", ctypes.c_float),
                ("seed", ctypes.c_uint64), ("paste", ctypes.c_uint32), ("mask_dilate", ctypes.c_uint32)]


class MoebiusRect(ctypes.Structure):
    _fields_ = [("x", ctypes.c_uint32), ("y", ctypes.c_uint32), ("width", ctypes.c_uint32),
                ("height", ctypes.c_uint32)]


class InpaintParams(ctypes.Structure):
    """include/moebius_engine.h MhInpaintParams (src/preset.rs:34-58 InpaintParams + precision)."""
    _fields_ = [("steps", ctypes.c_uint32), ("spacing", ctypes.c_uint32), ("solver", ctypes.c_uint32),
                ("cfg_steps", ctypes.c_int32), ("strength", ctypes.c_double), ("guidance", ctypes.c_float),
                ("noise_offset", ctypes.c_float), ("seed", ctypes.c_uint64), ("roi_encode", ctypes.c_uint32),
                ("roi_decode", ctypes.c_uint32), ("paste", ctypes.c_uint32), ("mask_dilate", ctypes.c_uint32),
                ("precision", ctypes.c_uint32), ("reserved", ctypes.c_uint32)]


TRACE_FN = ctypes.CFUNCTYPE(None, ctypes.c_void_p, ctypes.c_char_p, ctypes.c_void_p, ctypes.c_uint32,
                            ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32)

_lib = None


def lib():
    """The loaded library (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"HIP library not built: {LIB_PATH} is missing (run __graft_entry__.build() or "
                "`python -m moebius_cpu_amd.build`); there is no CPU fallback")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(status: int) -> None:
    if status != OK:
        msg = lib().mh_last_error().decode("utf-8", "replace")
        raise MoebiusError(int(status), msg)


def u32x4(vals):
    return (ctypes.c_uint32 * 4)(*[int(v) for v in vals])
