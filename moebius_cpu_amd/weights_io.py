"""Writing converter-format weight files (safetensors, `format` = "moebius-cpu/1",
tools/convert_weights.py's layouts) from a named tensor table, e.g. the seeded
random-init weights, so the file loaders (mh_*_create_from_file) can be
exercised without the real checkpoints."""
from __future__ import annotations

import numpy as np

FORMAT = "moebius-cpu/1"
VAE_SCALING = "0.13025"


def write_weights(path: str, params: dict, gemm_names=(), f16: bool = False, metadata=None) -> None:
    """params {name: array}; with f16, the names in gemm_names are stored as f16
    (the converter's --dtype f16, step 4), everything else f32."""
    from safetensors.numpy import save_file

    gemm = set(gemm_names)
    tensors = {}
    for k, v in params.items():
        dt = np.float16 if (f16 and k in gemm) else np.float32
        tensors[k] = np.ascontiguousarray(v, dtype=dt)
    meta = {"format": FORMAT}
    meta.update(metadata or {})
    save_file(tensors, path, metadata=meta)
