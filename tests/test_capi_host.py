"""CPU-side checks of the C ABI library: it was built, it loads, it exports
every function include/moebius_hip.h and include/moebius_engine.h declare (and
the binding declares no more), and its host-only paths behave (argument errors, output_hw). No kernel
is launched here."""
from __future__ import annotations

import ctypes
import re

import pytest

import oracle
from moebius_cpu_amd import _lib


def header_functions():
    names = set()
    for h in _lib.HEADERS:
        text = re.sub(r"/\*.*?\*/", "", open(h).read(), flags=re.S)
        names.update(re.findall(r"\b((?:mh|moebius)_[a-z0-9_]+)\s*\(", text))
    return sorted(names)


def test_library_exports_every_declared_symbol():
    L = _lib.lib()
    names = header_functions()
    assert len(names) >= 30
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, f"declared in include/*.h but not exported: {missing}"
    assert sorted(_lib.SIGNATURES) == names, "the ctypes table and the header disagree"


def test_abi_version_and_error_string():
    L = _lib.lib()
    assert L.mh_abi_version() == 1
    assert L.mh_last_error() is not None


def test_null_arguments_are_invalid_argument():
    L = _lib.lib()
    assert L.mh_context_create(0, None) == _lib.ERR_INVALID_ARGUMENT
    assert b"out is NULL" in L.mh_last_error()
    assert L.mh_conv1x1_forward(None, None, 1, 1, 1, 1, None, 0, 1, None, None, None) == _lib.ERR_INVALID_ARGUMENT
    assert b"context is NULL" in L.mh_last_error()
    L.mh_context_destroy(None)  # a no-op, like moebius_engine_destroy(NULL)


@pytest.mark.parametrize("h,w,stride,pad,up", [(9, 11, 1, (1, 1, 1, 1), 0), (9, 11, 2, (1, 1, 1, 1), 0),
                                               (9, 11, 2, (0, 0, 1, 1), 0), (9, 11, 1, (1, 1, 1, 1), 1),
                                               (64, 64, 2, (1, 1, 1, 1), 0), (512, 512, 2, (0, 0, 1, 1), 0)])
def test_conv3x3_output_hw_matches_reference_formula(h, w, stride, pad, up):
    ho, wo = ctypes.c_uint32(), ctypes.c_uint32()
    _lib.check(_lib.lib().mh_conv3x3_output_hw(h, w, stride, _lib.u32x4(pad), up, ctypes.byref(ho),
                                               ctypes.byref(wo)))
    assert (ho.value, wo.value) == oracle.conv3x3_output_hw(h, w, stride, pad, bool(up))


def test_output_hw_rejects_degenerate_input():
    ho, wo = ctypes.c_uint32(), ctypes.c_uint32()
    st = _lib.lib().mh_conv3x3_output_hw(1, 1, 1, _lib.u32x4((0, 0, 0, 0)), 0, ctypes.byref(ho), ctypes.byref(wo))
    assert st == _lib.ERR_INVALID_ARGUMENT


def test_context_without_a_gpu_fails_cleanly():
    """No device here: creation must return a status, never crash or hang."""
    import os

    if os.path.exists("/dev/kfd") and os.access("/dev/kfd", os.R_OK | os.W_OK):
        pytest.skip("a GPU is present")
    h = ctypes.c_void_p()
    st = _lib.lib().mh_context_create(0, ctypes.byref(h))
    assert st != _lib.OK and not h.value
    assert len(_lib.lib().mh_last_error()) > 0
