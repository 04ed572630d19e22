"""CPU oracle for the moebius-cpu conv/norm path (test infrastructure only).

ctypes bindings over ``liboracle.so`` (built from this directory by
``make``), a C++ restatement of moebius-cpu ``src/engine`` and of the
``src/unet`` / ``src/vae`` block chains. Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg import
this module; the product library never does.

Arrays are numpy float32 NHWC, C-contiguous. Each wrapper names the
reference function it restates.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

_f32p = ctypes.POINTER(ctypes.c_float)
_i64 = ctypes.c_int64
_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"oracle library missing: {LIB_PATH} (run `make -C oracle`)")
        _lib = ctypes.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


def _declare(L):
    vp = ctypes.c_void_p
    L.orc_exp.restype = ctypes.c_float
    L.orc_exp.argtypes = [ctypes.c_float]
    L.orc_silu.restype = ctypes.c_float
    L.orc_silu.argtypes = [ctypes.c_float]
    L.orc_matmul.argtypes = [vp, vp, _i64, _i64, vp, _i64, _i64, _i64, _i64, _i64, ctypes.c_int]
    L.orc_init_output.restype = ctypes.c_int
    L.orc_init_output.argtypes = [vp, _i64, _i64, vp, vp]
    L.orc_conv1x1.argtypes = [vp, _i64, _i64, vp, _i64, vp, vp, vp]
    L.orc_conv3x3_forward.argtypes = [vp, _i64, _i64, _i64, _i64, vp, _i64, vp, ctypes.c_int, vp, ctypes.c_int,
                                      vp, vp, ctypes.c_int, vp]
    L.orc_conv3x3_im2col.argtypes = [vp, _i64, _i64, _i64, _i64, vp, _i64, vp, ctypes.c_int, vp, ctypes.c_int, vp]
    L.orc_wino_kernel_transform_all.argtypes = [vp, _i64, _i64, vp]
    L.orc_wino_input_transform_all.argtypes = [vp, _i64, _i64, _i64, _i64, ctypes.c_int, vp, vp, ctypes.c_int, vp]
    L.orc_wino_output_transform_all.argtypes = [vp, _i64, _i64, _i64, _i64, ctypes.c_int, vp, vp]
    L.orc_im2col_gather_row.argtypes = [vp, _i64, _i64, _i64, _i64, _i64, _i64, ctypes.c_int, ctypes.c_int,
                                        ctypes.c_int, ctypes.c_int, _i64, vp]
    L.orc_depthwise3x3.argtypes = [vp, _i64, _i64, _i64, _i64, vp, vp, ctypes.c_int, vp]
    L.orc_group_norm_affine.argtypes = [vp, _i64, _i64, _i64, _i64, _i64, ctypes.c_float, vp, vp, vp, vp, vp]
    L.orc_group_norm_forward.argtypes = [vp, _i64, _i64, _i64, _i64, _i64, ctypes.c_float, vp, vp, vp,
                                         ctypes.c_int, vp]
    L.orc_apply_affine.argtypes = [vp, _i64, _i64, vp, vp, ctypes.c_int, vp]
    L.orc_layer_norm.argtypes = [vp, _i64, _i64, vp, vp, ctypes.c_float, vp]
    L.orc_silu_inplace.argtypes = [vp, _i64]
    L.orc_add_inplace.argtypes = [vp, vp, _i64]
    L.orc_concat_channels.argtypes = [vp, _i64, vp, _i64, _i64, vp]
    L.orc_to_u8.argtypes = [vp, _i64, vp]
    L.orc_set_threads.argtypes = [ctypes.c_int]
    L.orc_get_threads.restype = ctypes.c_int


def _p(a):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data


def _f32(a):
    if a is None:
        return None
    return np.ascontiguousarray(a, dtype=np.float32)


def set_threads(n: int) -> None:
    lib().orc_set_threads(int(n))


def threads() -> int:
    return int(lib().orc_get_threads())


def exp(x: float) -> float:
    """src/engine/math.rs:17-30"""
    return float(lib().orc_exp(float(x)))


def silu_scalar(x: float) -> float:
    """src/engine/math.rs:33-36"""
    return float(lib().orc_silu(float(x)))


def matmul(a, b, c=None, accumulate=False):
    """src/engine/gemm.rs:63-132 with numpy views: a [m, k], b [k, n] of any strides."""
    a = np.asarray(a, dtype=np.float32)
    b = np.asarray(b, dtype=np.float32)
    m, k = a.shape
    k2, n = b.shape
    assert k == k2, "inner dimensions differ"
    if c is None:
        c = np.zeros((m, n), np.float32)
    es = 4
    lib().orc_matmul(_p(c), a.ctypes.data, a.strides[0] // es, a.strides[1] // es, b.ctypes.data,
                     b.strides[0] // es, b.strides[1] // es, m, k, n, int(bool(accumulate)))
    return c


def conv1x1(x, weight, bias=None, residual=None):
    """src/engine/conv.rs:38-55: x [n,h,w,ci], weight [co, ci]."""
    x, weight, bias, residual = _f32(x), _f32(weight), _f32(bias), _f32(residual)
    n, h, w, ci = x.shape
    co = weight.shape[0]
    assert weight.shape == (co, ci), "Conv1x1 weight size"
    out = np.empty((n, h, w, co), np.float32)
    if residual is not None:
        assert residual.shape == out.shape, "Conv1x1 residual shape"
    lib().orc_conv1x1(_p(x), n * h * w, ci, _p(weight), co, _p(bias), _p(residual), _p(out))
    return out


def conv3x3_output_hw(h, w, stride=1, pad=(1, 1, 1, 1), upsample2x=False):
    """src/engine/conv.rs:77-81"""
    up = 2 if upsample2x else 1
    return ((h * up + pad[0] + pad[2] - 3) // stride + 1, (w * up + pad[1] + pad[3] - 3) // stride + 1)


def conv3x3(x, weight, bias=None, stride=1, pad=(1, 1, 1, 1), upsample2x=False, prologue=None, im2col=False):
    """src/engine/conv.rs:83-102 (forward / forward_prologue) or 106-130 (im2col).

    weight [co, 3, 3, ci]; prologue = (scale [n*ci], shift [n*ci], silu) or None."""
    x, weight, bias = _f32(x), _f32(weight), _f32(bias)
    n, h, w, ci = x.shape
    co = weight.shape[0]
    assert weight.size == 9 * ci * co, "Conv3x3 weight size"
    ho, wo = conv3x3_output_hw(h, w, stride, pad, upsample2x)
    out = np.empty((n, ho, wo, co), np.float32)
    padv = (ctypes.c_int * 4)(*pad)
    if im2col:
        assert prologue is None
        lib().orc_conv3x3_im2col(_p(x), n, h, w, ci, _p(weight), co, _p(bias), stride, padv, int(upsample2x),
                                 _p(out))
    else:
        sc = sh = None
        silu = 0
        if prologue is not None:
            assert stride == 1 and tuple(pad) == (1, 1, 1, 1), \
                "Conv3x3 prologue needs the stride-1 / pad-1 Winograd path"
            sc, sh, silu = _f32(prologue[0]), _f32(prologue[1]), int(prologue[2])
        lib().orc_conv3x3_forward(_p(x), n, h, w, ci, _p(weight), co, _p(bias), stride, padv, int(upsample2x),
                                  _p(sc), _p(sh), silu, _p(out))
    return out


def wino_tiles(n, h, w, upsample2x=False):
    """Tiles of the Winograd F(2x2,3x3) conv (src/engine/winograd.rs:64-69)."""
    up = 2 if upsample2x else 1
    return n * ((h * up + 1) // 2) * ((w * up + 1) // 2)


def wino_kernel_transform(weight):
    """src/engine/winograd.rs:254-297: U = G g G^T; weight [co,3,3,ci] -> u [16,co,ci]."""
    weight = _f32(weight)
    co, ci = weight.shape[0], weight.shape[3]
    u = np.empty((16, co, ci), np.float32)
    lib().orc_wino_kernel_transform_all(_p(weight), co, ci, _p(u))
    return u


def wino_input_transform(x, upsample2x=False, prologue=None):
    """src/engine/winograd.rs:144-160, 210-251, 299-327: V = B^T d B per tile -> v [16, tiles, ci]."""
    x = _f32(x)
    n, h, w, ci = x.shape
    v = np.empty((16, wino_tiles(n, h, w, upsample2x), ci), np.float32)
    sc = sh = None
    silu = 0
    if prologue is not None:
        sc, sh, silu = _f32(prologue[0]), _f32(prologue[1]), int(prologue[2])
    lib().orc_wino_input_transform_all(_p(x), n, h, w, ci, int(upsample2x), _p(sc), _p(sh), silu, _p(v))
    return v


def wino_output_transform(m, n, h, w, upsample2x=False, bias=None):
    """src/engine/winograd.rs:164-202, 329-352: out = A^T m A + bias; m [16, tiles, co]."""
    m, bias = _f32(m), _f32(bias)
    co = m.shape[2]
    up = 2 if upsample2x else 1
    out = np.zeros((n, h * up, w * up, co), np.float32)
    lib().orc_wino_output_transform_all(_p(m), n, h, w, co, int(upsample2x), _p(bias), _p(out))
    return out


def im2col_row(x, p, stride=1, pad=(1, 1, 1, 1), upsample2x=False):
    """src/engine/conv.rs:145-165: patch row of output pixel p."""
    x = _f32(x)
    n, h, w, c = x.shape
    ho, wo = conv3x3_output_hw(h, w, stride, pad, upsample2x)
    row = np.empty(9 * c, np.float32)
    lib().orc_im2col_gather_row(_p(x), n, h, w, c, ho, wo, stride, pad[0], pad[1], int(upsample2x), int(p), _p(row))
    return row


EPILOGUE = {"none": 0, "relu": 1, "glu_silu": 2}


def depthwise3x3(x, weight, bias, epilogue="none"):
    """src/engine/depthwise.rs:31-59; weight [3,3,c], bias [c]."""
    x, weight, bias = _f32(x), _f32(weight), _f32(bias)
    n, h, w, c = x.shape
    assert weight.size == 9 * c, "depthwise weight size"
    assert bias.size == c, "depthwise bias size"
    ep = EPILOGUE[epilogue]
    co = c // 2 if ep == 2 else c
    out = np.empty((n, h, w, co), np.float32)
    lib().orc_depthwise3x3(_p(x), n, h, w, c, _p(weight), _p(bias), ep, _p(out))
    return out


def group_norm_affine(x, groups, eps, gamma, beta, add=None):
    """src/engine/norm.rs:57-105: returns (scale [n*c], shift [n*c])."""
    x, gamma, beta, add = _f32(x), _f32(gamma), _f32(beta), _f32(add)
    n, h, w, c = x.shape
    assert c % groups == 0, "channels not divisible by groups"
    scale = np.empty(n * c, np.float32)
    shift = np.empty(n * c, np.float32)
    lib().orc_group_norm_affine(_p(x), n, h, w, c, groups, float(eps), _p(gamma), _p(beta), _p(add), _p(scale),
                                _p(shift))
    return scale, shift


def group_norm(x, groups, eps, gamma, beta, add=None, silu=False):
    """src/engine/norm.rs:41-53"""
    x, gamma, beta, add = _f32(x), _f32(gamma), _f32(beta), _f32(add)
    n, h, w, c = x.shape
    out = np.empty_like(x)
    lib().orc_group_norm_forward(_p(x), n, h, w, c, groups, float(eps), _p(gamma), _p(beta), _p(add), int(silu),
                                 _p(out))
    return out


def apply_affine(x, scale, shift, silu):
    """src/engine/norm.rs:132-148 for one item: x [pixels, c] (any leading shape), scale/shift [c]."""
    x, scale, shift = _f32(x), _f32(scale), _f32(shift)
    c = x.shape[-1]
    out = np.empty_like(x)
    lib().orc_apply_affine(_p(x), x.size // c, c, _p(scale), _p(shift), int(silu), _p(out))
    return out


def layer_norm(x, gamma, beta, eps):
    """src/engine/norm.rs:151-173, over the last axis."""
    x, gamma, beta = _f32(x), _f32(gamma), _f32(beta)
    c = x.shape[-1]
    out = np.empty_like(x)
    lib().orc_layer_norm(_p(x), x.size // c, c, _p(gamma), _p(beta), float(eps), _p(out))
    return out


def silu(x):
    """src/engine/ops.rs:11-13 (out of place)."""
    y = _f32(x).copy()
    lib().orc_silu_inplace(_p(y), y.size)
    return y


def add(a, b):
    """src/engine/ops.rs:16-19 (out of place)."""
    y = _f32(a).copy()
    b = _f32(b)
    assert y.size == b.size, "add length mismatch"
    lib().orc_add_inplace(_p(y), _p(b), y.size)
    return y


def init_output(rows, cols, bias=None, residual=None):
    """src/engine/conv.rs:170-191: returns (prefilled [rows, cols], accumulate)."""
    bias, residual = _f32(bias), _f32(residual)
    out = np.zeros((rows, cols), np.float32)
    acc = lib().orc_init_output(_p(out), rows, cols, _p(bias), _p(residual))
    return out, bool(acc)


def concat_channels(a, b):
    """src/engine/tensor.rs:59-73"""
    a, b = _f32(a), _f32(b)
    assert a.shape[:3] == b.shape[:3], "concat_channels: spatial shapes differ"
    n, h, w, ca = a.shape
    cb = b.shape[3]
    out = np.empty((n, h, w, ca + cb), np.float32)
    lib().orc_concat_channels(_p(a), ca, _p(b), cb, n * h * w, _p(out))
    return out


def to_u8(x):
    """src/imaging/blend.rs:21-24"""
    x = _f32(x)
    out = np.empty(x.shape, np.uint8)
    lib().orc_to_u8(_p(x), x.size, _p(out))
    return out


# ---- UNet chain (oracle/unet.cpp)
class _Named(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("data", ctypes.c_void_p), ("numel", ctypes.c_int64)]


_TRACE_FN = ctypes.CFUNCTYPE(None, ctypes.c_void_p, ctypes.c_char_p, ctypes.POINTER(ctypes.c_float), ctypes.c_int64,
                             ctypes.c_int64, ctypes.c_int64, ctypes.c_int64)


def _declare_unet(L):
    vp = ctypes.c_void_p
    L.orc_timestep_sinusoid.argtypes = [ctypes.c_int, vp]
    L.orc_unet_create.restype = vp
    L.orc_unet_create.argtypes = [ctypes.POINTER(_Named), ctypes.c_int, ctypes.c_char_p, ctypes.c_int]
    L.orc_unet_destroy.argtypes = [vp]
    L.orc_unet_forward.restype = ctypes.c_int
    L.orc_unet_forward.argtypes = [vp, vp, ctypes.c_int, ctypes.c_int, vp, _TRACE_FN, vp]
    L.orc_softmax_lambda.argtypes = [vp, vp, _i64, _i64, _i64, vp]
    L.orc_tap_filter.argtypes = [vp, vp, vp, _i64, _i64, _i64, _i64, _i64]
    L.orc_dot8.restype = ctypes.c_float
    L.orc_dot8.argtypes = [vp, vp, _i64]
    L.orc_position_term.argtypes = [vp, vp, vp, vp, _i64, _i64]
    L.orc_unet_flops.argtypes = [vp]
    L.orc_unet_flops_reset.argtypes = []
    L.orc_block_forward.restype = ctypes.c_int
    L.orc_block_forward.argtypes = [ctypes.c_int, ctypes.POINTER(_Named), ctypes.c_int, ctypes.c_char_p, vp, _i64,
                                    _i64, _i64, _i64, _i64, vp, vp, vp, ctypes.c_char_p, ctypes.c_int]


def timestep_sinusoid(t: int) -> np.ndarray:
    """src/unet/embed.rs:21-30"""
    L = lib()
    _declare_unet(L)
    out = np.empty(320, np.float32)
    L.orc_timestep_sinusoid(int(t), _p(out))
    return out


def softmax_lambda(keys, v):
    """src/unet/lambda.rs:322-359: keys [rows, k], v [rows, vd] -> lambda [k, vd]."""
    L = lib()
    _declare_unet(L)
    keys = _f32(keys).copy()
    v = _f32(v)
    rows, k = keys.shape
    vd = v.shape[1]
    out = np.empty((k, vd), np.float32)
    L.orc_softmax_lambda(_p(keys), _p(v), rows, k, vd, _p(out))
    return out


def tap_filter(a, v, o, hh, ww):
    """src/unet/lambda.rs:154-185 over a whole item: a [hw, 8, 226], v [hw, k], o [hw, 8*k] (updated)."""
    L = lib()
    _declare_unet(L)
    a, v = _f32(a), _f32(v)
    o = _f32(o).copy()
    L.orc_tap_filter(_p(a), _p(v), _p(o), 0, hh * ww, hh, ww, v.shape[1])
    return o


def position_term(q, e, v, o):
    """src/unet/lambda.rs:279-295: q, o [px, 8k]; e [px, 10, k]; v [10, k]; returns the updated o."""
    L = lib()
    _declare_unet(L)
    q, e, v = _f32(q), _f32(e), _f32(v)
    o = _f32(o).copy()
    L.orc_position_term(_p(q), _p(e), _p(v), _p(o), q.shape[0], v.shape[1])
    return o


def dot8(a, b):
    """src/unet/lambda.rs:297-309"""
    L = lib()
    _declare_unet(L)
    a, b = _f32(a), _f32(b)
    return float(L.orc_dot8(_p(a), _p(b), a.size))


class UNet:
    """src/unet/mod.rs UNet over a dict of converter tensors (f32 arrays)."""

    def __init__(self, params: dict):
        L = lib()
        _declare_unet(L)
        self._keep = {k: np.ascontiguousarray(v, dtype=np.float32) for k, v in params.items()}
        arr = (_Named * len(self._keep))()
        for i, (k, v) in enumerate(self._keep.items()):
            arr[i].name = k.encode()
            arr[i].data = v.ctypes.data
            arr[i].numel = v.size
        err = ctypes.create_string_buffer(512)
        self.h = L.orc_unet_create(arr, len(self._keep), err, 512)
        if not self.h:
            raise RuntimeError("oracle UNet load failed: " + err.value.decode())

    def forward(self, x, timestep: int, cfg: bool = True, trace: bool = False):
        """x [1,64,64,9] -> eps [b,64,64,4] (b = 2 with CFG); with trace, also {name: tensor}."""
        x = _f32(x)
        b = 2 if cfg else 1
        eps = np.empty((b, 64, 64, 4), np.float32)
        traced = {}

        def cb(_user, name, data, n, h, w, c):
            traced[name.decode()] = np.ctypeslib.as_array(data, shape=(n * h * w * c,)).reshape(n, h, w, c).copy()

        fn = _TRACE_FN(cb) if trace else _TRACE_FN()
        st = lib().orc_unet_forward(self.h, _p(x), int(timestep), 0 if cfg else 1, _p(eps), fn, None)
        if st != 0:
            raise RuntimeError("oracle UNet forward failed")
        return (eps, traced) if trace else eps

    FLOP_KINDS = ("1x1", "3x3 dense", "3x3 stride 2", "depthwise", "lambda pos_conv", "matmul")

    @staticmethod
    def flops_reset() -> None:
        lib().orc_unet_flops_reset()

    @staticmethod
    def flops() -> dict:
        """FLOPs of the forwards run since flops_reset(), tallied per layer at the
        shapes it ran, as the upstream model computes them (the unfolded
        lambda's position Conv3d and products), by category."""
        out = (ctypes.c_double * len(UNet.FLOP_KINDS))()
        lib().orc_unet_flops(out)
        return {k: float(v) for k, v in zip(UNet.FLOP_KINDS, out)}

    def __del__(self):
        try:
            lib().orc_unet_destroy(self.h)
        except Exception:
            pass


BLOCK_KINDS = {"dwconv": 0, "resnet": 1, "self_lambda": 2, "cross_lambda": 3, "transformer": 4}


def block_forward(kind: str, params: dict, prefix: str, x, c_out=None, temb=None, branches=None):
    """One UNet block alone (oracle/unet.cpp orc_block_forward)."""
    L = lib()
    _declare_unet(L)
    keep = {k: np.ascontiguousarray(v, dtype=np.float32) for k, v in params.items()}
    arr = (_Named * len(keep))()
    for i, (k, v) in enumerate(keep.items()):
        arr[i].name = k.encode()
        arr[i].data = v.ctypes.data
        arr[i].numel = v.size
    x = _f32(x)
    n, h, w, ci = x.shape
    co = ci if c_out is None else c_out
    out = np.empty((n, h, w, co), np.float32)
    temb = _f32(temb)
    br = None if branches is None else np.ascontiguousarray(branches, dtype=np.int32)
    err = ctypes.create_string_buffer(512)
    st = L.orc_block_forward(BLOCK_KINDS[kind], arr, len(keep), prefix.encode(), _p(x), n, h, w, ci, co, _p(temb),
                             None if br is None else br.ctypes.data, _p(out), err, 512)
    if st != 0:
        raise RuntimeError(err.value.decode())
    return out


# ---- VAE chain (oracle/vae.cpp)
def _declare_vae(L):
    vp, i64, cp, ci = ctypes.c_void_p, _i64, ctypes.c_char_p, ctypes.c_int
    _declare_unet(L)
    L.orc_vae_create.restype = vp
    L.orc_vae_create.argtypes = [ctypes.POINTER(_Named), ci, cp, ci]
    L.orc_vae_destroy.argtypes = [vp]
    L.orc_vae_encode.restype = ci
    L.orc_vae_encode.argtypes = [vp, vp, i64, i64, i64, vp, vp, _TRACE_FN, vp, cp, ci]
    L.orc_vae_decode.restype = ci
    L.orc_vae_decode.argtypes = [vp, vp, i64, i64, vp, _TRACE_FN, vp, cp, ci]
    L.orc_softmax_rows.argtypes = [vp, i64, i64, ctypes.c_float]
    L.orc_vae_sample.argtypes = [vp, vp, i64, vp]
    L.orc_vae_attention.restype = ci
    L.orc_vae_attention.argtypes = [ctypes.POINTER(_Named), ci, cp, vp, i64, i64, i64, i64, vp, cp, ci]
    L.orc_vae_resnet.restype = ci
    L.orc_vae_resnet.argtypes = [ctypes.POINTER(_Named), ci, cp, vp, i64, i64, i64, i64, i64, vp, cp, ci]


def _named_table(params: dict):
    keep = {k: np.ascontiguousarray(v, dtype=np.float32) for k, v in params.items()}
    arr = (_Named * len(keep))()
    for i, (k, v) in enumerate(keep.items()):
        arr[i].name = k.encode()
        arr[i].data = v.ctypes.data
        arr[i].numel = v.size
    return keep, arr


def softmax_rows(rows, scale: float):
    """src/vae/mod.rs:275-294 over rows [nrows, n] (returns a new array)."""
    L = lib()
    _declare_vae(L)
    r = _f32(rows).copy()
    L.orc_softmax_rows(_p(r), r.shape[0], r.shape[1], float(scale))
    return r


def vae_sample(moments, noise):
    """src/vae/encoder.rs:121-133: moments [..., 8], noise [..., 4] -> z [..., 4]."""
    L = lib()
    _declare_vae(L)
    m, nz = _f32(moments), _f32(noise)
    z = np.empty(nz.shape, np.float32)
    L.orc_vae_sample(_p(m), _p(nz), nz.size // 4, _p(z))
    return z


def vae_attention(params: dict, prefix: str, x):
    """src/vae/mod.rs:240-270 with the weights under prefix (attentions.0)."""
    L = lib()
    _declare_vae(L)
    keep, arr = _named_table(params)
    x = _f32(x)
    out = np.empty_like(x)
    err = ctypes.create_string_buffer(512)
    if L.orc_vae_attention(arr, len(keep), prefix.encode(), _p(x), *x.shape, _p(out), err, 512) != 0:
        raise RuntimeError(err.value.decode())
    return out


def vae_resnet(params: dict, prefix: str, x, c_out: int):
    """src/vae/mod.rs:174-211 with the weights under prefix (resnets.j)."""
    L = lib()
    _declare_vae(L)
    keep, arr = _named_table(params)
    x = _f32(x)
    n, h, w, c = x.shape
    out = np.empty((n, h, w, c_out), np.float32)
    err = ctypes.create_string_buffer(512)
    if L.orc_vae_resnet(arr, len(keep), prefix.encode(), _p(x), n, h, w, c, c_out, _p(out), err, 512) != 0:
        raise RuntimeError(err.value.decode())
    return out


class Vae:
    """src/vae/mod.rs Vae over a dict of converter tensors (f32 arrays)."""

    def __init__(self, params: dict):
        L = lib()
        _declare_vae(L)
        self._keep, arr = _named_table(params)
        err = ctypes.create_string_buffer(512)
        self.h = L.orc_vae_create(arr, len(self._keep), err, 512)
        if not self.h:
            raise RuntimeError("oracle VAE load failed: " + err.value.decode())

    @staticmethod
    def _tracer(traced):
        def cb(_user, name, data, n, h, w, c):
            traced[name.decode()] = np.ctypeslib.as_array(data, shape=(n * h * w * c,)).reshape(n, h, w, c).copy()
        return _TRACE_FN(cb)

    def encode(self, images, noise, trace: bool = False):
        """images [b,h,w,3] in [-1,1], noise [b,h/8,w/8,4] -> z [b,h/8,w/8,4]."""
        images, noise = _f32(images), _f32(noise)
        b, h, w, _ = images.shape
        z = np.empty((b, h // 8, w // 8, 4), np.float32)
        traced = {}
        fn = self._tracer(traced) if trace else _TRACE_FN()
        err = ctypes.create_string_buffer(512)
        if lib().orc_vae_encode(self.h, _p(images), b, h, w, _p(noise), _p(z), fn, None, err, 512) != 0:
            raise RuntimeError("oracle VAE encode failed: " + err.value.decode())
        return (z, traced) if trace else z

    def decode(self, latents, trace: bool = False):
        """latents [1,h,w,4] (scaled) -> [1,8h,8w,3] = (dec + 1) / 2."""
        latents = _f32(latents)
        _, h, w, _ = latents.shape
        out = np.empty((1, 8 * h, 8 * w, 3), np.float32)
        traced = {}
        fn = self._tracer(traced) if trace else _TRACE_FN()
        err = ctypes.create_string_buffer(512)
        if lib().orc_vae_decode(self.h, _p(latents), h, w, _p(out), fn, None, err, 512) != 0:
            raise RuntimeError("oracle VAE decode failed: " + err.value.decode())
        return (out, traced) if trace else out

    def __del__(self):
        try:
            lib().orc_vae_destroy(self.h)
        except Exception:
            pass


# ---- samplers and denoise loop (oracle/pipeline.cpp: src/scheduler.rs, src/pipeline.rs)

def _declare_pipeline(L):
    vp, i64, c_int, c_double = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_double
    L.orc_alphas_cumprod.argtypes = [vp]
    L.orc_sched_create.restype = vp
    L.orc_sched_create.argtypes = [c_int, c_double, c_int]
    L.orc_sched_destroy.argtypes = [vp]
    L.orc_sched_timesteps.restype = c_int
    L.orc_sched_timesteps.argtypes = [vp, vp, vp]
    L.orc_sched_add_noise.argtypes = [vp, vp, vp, i64, c_int, vp]
    L.orc_sched_ddim_step.argtypes = [vp, vp, i64, c_int, vp]
    L.orc_sched_dpm_step.argtypes = [vp, vp, i64, c_int, vp]
    L.orc_sched_dpm_restart.argtypes = [vp]
    L.orc_denoise.restype = c_int
    L.orc_denoise.argtypes = [vp, vp, vp, vp, vp, c_int, c_double, c_int, c_int, ctypes.c_float, c_int, vp,
                              ctypes.c_char_p, c_int]


SPACING = {"leading": 0, "trailing": 1}
SOLVER = {"ddim": 0, "dpm": 1}


def alphas_cumprod() -> np.ndarray:
    """src/scheduler.rs:159-172"""
    L = lib()
    _declare_pipeline(L)
    out = np.empty(1000, np.float32)
    L.orc_alphas_cumprod(_p(out))
    return out


class Scheduler:
    """src/scheduler.rs `Ddim` (+ the `Dpm2M` state): timesteps, add_noise, DDIM and DPM-Solver++(2M) steps."""

    def __init__(self, steps: int, strength: float, spacing: str = "leading"):
        L = lib()
        _declare_pipeline(L)
        self.h = L.orc_sched_create(int(steps), float(strength), SPACING[spacing])
        if not self.h:
            raise ValueError(f"steps must be 1..=1000, got {steps}")
        ts = np.empty(1000, np.int32)
        pure = ctypes.c_int()
        n = L.orc_sched_timesteps(self.h, _p(ts), ctypes.byref(pure))
        self.timesteps = [int(t) for t in ts[:n]]
        self.pure_noise_start = bool(pure.value)

    def add_noise(self, x0, noise, t: int) -> np.ndarray:
        x0, noise = _f32(x0), _f32(noise)
        out = np.empty_like(x0)
        lib().orc_sched_add_noise(self.h, _p(x0), _p(noise), x0.size, int(t), _p(out))
        return out

    def ddim_step(self, eps, t: int, x) -> np.ndarray:
        eps, x = _f32(eps), np.array(_f32(x), copy=True)
        lib().orc_sched_ddim_step(self.h, _p(eps), x.size, int(t), _p(x))
        return x

    def dpm_step(self, eps, i: int, x) -> np.ndarray:
        eps, x = _f32(eps), np.array(_f32(x), copy=True)
        lib().orc_sched_dpm_step(self.h, _p(eps), x.size, int(i), _p(x))
        return x

    def dpm_restart(self):
        lib().orc_sched_dpm_restart(self.h)

    def __del__(self):
        try:
            lib().orc_sched_destroy(self.h)
        except Exception:
            pass


def denoise(unet: "UNet", z_img, init, mask_lat, z_masked, steps: int, strength: float, spacing: str = "leading",
            solver: str = "ddim", guidance: float = 2.5, cfg_steps=None) -> np.ndarray:
    """src/pipeline.rs:295-345 (steps 7-8) over the oracle UNet: the final latents [1,64,64,4]."""
    L = lib()
    _declare_pipeline(L)
    z_img, init, z_masked = _f32(z_img), _f32(init), _f32(z_masked)
    mask_lat = _f32(mask_lat)
    out = np.empty((1, 64, 64, 4), np.float32)
    err = ctypes.create_string_buffer(512)
    st = L.orc_denoise(unet.h, _p(z_img), _p(init), _p(mask_lat), _p(z_masked), int(steps), float(strength),
                       SPACING[spacing], SOLVER[solver], float(guidance), -1 if cfg_steps is None else int(cfg_steps),
                       _p(out), err, 512)
    if st != 0:
        raise RuntimeError("oracle denoise failed: " + err.value.decode())
    return out


def resize_u8(img, to_w: int, to_h: int) -> np.ndarray:
    """src/imaging/resize.rs:15-24 (PIL LANCZOS, 22-bit fixed point): [h, w(, c)] uint8 -> [to_h, to_w(, c)]."""
    L = lib()
    L.orc_resize_u8.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                ctypes.c_void_p]
    a = np.ascontiguousarray(img, np.uint8)
    c = 1 if a.ndim == 2 else a.shape[2]
    out = np.empty((to_h, to_w) + (() if a.ndim == 2 else (c,)), np.uint8)
    L.orc_resize_u8(a.ctypes.data, a.shape[1], a.shape[0], int(to_w), int(to_h), c, out.ctypes.data)
    return out
