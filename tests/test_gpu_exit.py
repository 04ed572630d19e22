"""A process may exit with a live context, live tensors and work still queued:
the reference's worker exits when its stdin closes (src/bin/moebius-cli.rs:52-62),
and a native host may never call the destroy functions. Each case runs in a
child process and must end with status 0 and print its last line."""
from __future__ import annotations

import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

PY_WRAPPERS = f"""
import sys
sys.path.insert(0, {ROOT!r})
from moebius_cpu_amd import engine as E
from moebius_cpu_amd import synthetic as S
ctx = E.Context(0)
x = E.Tensor.from_numpy(ctx, S.normal(1, (2, 16, 16, 64)))
conv = E.Conv3x3.same(ctx, 64, 96, E.Param(ctx, S.normal(2, (96, 3, 3, 64), 0.05)), S.normal(3, (96,), 0.02))
y, z = E.Tensor(ctx), E.Tensor(ctx)
conv.forward(x, y)
E.GroupNorm(ctx, 32, 1e-5, S.normal(4, (96,), 0.1, 1.0), S.normal(5, (96,), 0.1)).forward(y, None, True, z)
print("queued, exiting without close()", flush=True)
"""

RAW_ABI = f"""
import ctypes, sys
sys.path.insert(0, {ROOT!r})
from moebius_cpu_amd import _lib
L = _lib.lib()
h = ctypes.c_void_p()
assert L.mh_context_create(0, ctypes.byref(h)) == 0
p = ctypes.c_void_p()
assert L.mh_malloc(h, 1 << 20, ctypes.byref(p)) == 0
print("context and buffer live, exiting", flush=True)
"""


@pytest.mark.parametrize("name,script", [("python-wrappers", PY_WRAPPERS), ("raw-c-abi", RAW_ABI)])
def test_process_exits_cleanly_with_live_context(name, script):
    print(f"exit case {name}", flush=True)
    p = subprocess.run([sys.executable, "-c", script], capture_output=True, text=True, timeout=120)
    assert p.returncode == 0, f"{name}: exit status {p.returncode}\n{p.stdout}\n{p.stderr[-2000:]}"
    assert "exiting" in p.stdout
