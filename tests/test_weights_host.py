"""The safetensors weight reader on the host (mh_weights_validate): files in
the converter's moebius-cpu/1 format written from the model specs pass; a
wrong format tag, a missing or reshaped tensor, an unsupported dtype, a bad
header and a missing file fail with the reference's status codes
(src/weights.rs:40-96, src/vae/mod.rs:88-93). No GPU."""
from __future__ import annotations

import os
import struct

import numpy as np
import pytest

from moebius_cpu_amd import _lib
from moebius_cpu_amd import unet_params as U
from moebius_cpu_amd import vae_params as V
from moebius_cpu_amd.weights_io import write_weights


def zeros(specs):
    return {s.name: np.zeros(s.shape, np.float32) for s in specs}


def validate(path, model):
    st = _lib.lib().mh_weights_validate(str(path).encode(), model)
    return st, _lib.lib().mh_last_error().decode()


@pytest.fixture(scope="module")
def vae_table():
    return zeros(V.vae_specs())


@pytest.fixture(scope="module")
def unet_file(tmp_path_factory):
    p = tmp_path_factory.mktemp("w") / "unet.safetensors"
    specs = U.unet_specs()
    write_weights(str(p), zeros(specs), [s.name for s in specs if s.gemm], f16=True)
    return p


def test_unet_file_in_the_converter_format_is_accepted(unet_file):
    assert validate(unet_file, _lib.MODEL_UNET)[0] == _lib.OK
    # the same file is not a VAE
    st, msg = validate(unet_file, _lib.MODEL_VAE)
    assert st == _lib.ERR_WEIGHTS and "scaling_factor" in msg


def test_f32_members_of_an_f16_file_are_accepted(tmp_path):
    """The converter keeps a GEMM weight f32 when its f16 copy would overflow
    (tools/convert_weights.py:27-30): an f16 file may hold F32 GEMM weights, also
    inside the groups the device fuses (self-lambda q | k | v, the time projections)."""
    specs = U.unet_specs()
    keep32 = {"diff_model.down_blocks.1.resnets.0.time_emb_proj.weight",
              "diff_model.down_blocks.0.attentions.1.transformer_blocks.0.attn1.to_k.weight"}
    p = tmp_path / "unet_mixed.safetensors"
    write_weights(str(p), zeros(specs), [s.name for s in specs if s.gemm and s.name not in keep32], f16=True)
    assert validate(p, _lib.MODEL_UNET)[0] == _lib.OK


def test_vae_file_needs_its_scaling_factor(tmp_path, vae_table):
    p = tmp_path / "vae.safetensors"
    write_weights(str(p), vae_table, metadata={"scaling_factor": "0.13025"})
    assert validate(p, _lib.MODEL_VAE)[0] == _lib.OK
    write_weights(str(p), vae_table, metadata={"scaling_factor": "0.18215"})
    st, msg = validate(p, _lib.MODEL_VAE)
    assert st == _lib.ERR_WEIGHTS and 'expected "0.13025"' in msg
    write_weights(str(p), vae_table)
    assert validate(p, _lib.MODEL_VAE)[0] == _lib.ERR_WEIGHTS


def test_wrong_format_tag(tmp_path, vae_table):
    p = tmp_path / "vae.safetensors"
    write_weights(str(p), vae_table, metadata={"format": "moebius-cpu/0", "scaling_factor": "0.13025"})
    st, msg = validate(p, _lib.MODEL_VAE)
    assert st == _lib.ERR_WEIGHTS and 'expected "moebius-cpu/1"' in msg


def test_missing_and_reshaped_tensors(tmp_path, vae_table):
    p = tmp_path / "vae.safetensors"
    t = dict(vae_table)
    del t["decoder.mid_block.attentions.0.to_q.weight"]
    write_weights(str(p), t, metadata={"scaling_factor": "0.13025"})
    st, msg = validate(p, _lib.MODEL_VAE)
    assert st == _lib.ERR_WEIGHTS and "missing tensor decoder.mid_block.attentions.0.to_q.weight" in msg
    t = dict(vae_table)
    t["encoder.conv_in.weight"] = np.zeros((128, 3, 3, 3), np.float32).reshape(128, 27, 1, 1)
    write_weights(str(p), t, metadata={"scaling_factor": "0.13025"})
    st, msg = validate(p, _lib.MODEL_VAE)
    assert st == _lib.ERR_WEIGHTS and "encoder.conv_in.weight: shape [128, 27, 1, 1], expected [128, 3, 3, 3]" in msg


def _raw_file(path, header: bytes, data: bytes):
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(header)))
        f.write(header)
        f.write(data)


@pytest.mark.parametrize("header,data,needle", [
    (b'{"__metadata__":{"format":"moebius-cpu/1"},"a":{"dtype":"BF16","shape":[2],"data_offsets":[0,4]}}',
     b"\0" * 4, "unsupported dtype BF16"),
    (b'{"__metadata__":{"format":"moebius-cpu/1"},"a":{"dtype":"F32","shape":[2],"data_offsets":[0,12]}}',
     b"\0" * 12, "does not match its shape"),
    (b'{"__metadata__":{"format":"moebius-cpu/1"},"a":{"dtype":"F32","shape":[2],"data_offsets":[0,8]}}',
     b"\0" * 4, "outside the file"),
    (b'{"__metadata__":{"format":"moebius-cpu/1"},"a":{"dtype":"F32","shape":[2],"data_offsets":[0,8]}',
     b"\0" * 8, "safetensors header"),
    (b'{"__metadata__":{"format":"moebius-cpu/1"},"a":{"dtype":"F32","shape":[1.5],"data_offsets":[0,8]}}',
     b"\0" * 8, "non-integer"),
])
def test_malformed_headers_are_weight_errors(tmp_path, header, data, needle):
    p = tmp_path / "bad.safetensors"
    _raw_file(p, header, data)
    st, msg = validate(p, _lib.MODEL_UNET)
    assert st == _lib.ERR_WEIGHTS and needle in msg, msg


def test_header_length_past_the_end(tmp_path):
    p = tmp_path / "bad.safetensors"
    with open(p, "wb") as f:
        f.write(struct.pack("<Q", 1 << 40) + b"{}")
    st, msg = validate(p, _lib.MODEL_UNET)
    assert st == _lib.ERR_WEIGHTS and "header length" in msg


def test_missing_file_is_an_io_error(tmp_path):
    st, msg = validate(tmp_path / "nope.safetensors", _lib.MODEL_UNET)
    assert st == _lib.ERR_IO and "nope.safetensors" in msg
    assert _lib.lib().mh_weights_validate(None, 0) == _lib.ERR_INVALID_ARGUMENT
