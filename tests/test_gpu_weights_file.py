"""Models loaded from the converter's safetensors files
(mh_unet_create_from_file, mh_vae_create_from_file) give the same bits as
models loaded from the same tensors handed over as a table: f16-stored GEMM
weights for the UNet (the converter's --dtype f16), f32 for the VAE."""
from __future__ import annotations

import numpy as np
import pytest

from moebius_cpu_amd import _lib
from moebius_cpu_amd import engine as E
from moebius_cpu_amd import synthetic as S
from moebius_cpu_amd import unet_params as U
from moebius_cpu_amd import vae_params as V
from moebius_cpu_amd.unet import UNet
from moebius_cpu_amd.vae import Vae
from moebius_cpu_amd.weights_io import write_weights

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    c = E.Context(0)
    yield c
    c.synchronize()
    c.close()


def test_unet_from_file_equals_unet_from_table(ctx, tmp_path):
    params = U.random_unet(seed=4000)
    gemm = [s.name for s in U.unet_specs() if s.gemm]
    path = tmp_path / "unet.safetensors"
    write_weights(str(path), params, gemm, f16=True)
    inp = U.unet_input(seed=5011)
    a = UNet.from_file(ctx, str(path))
    got = a.forward_host(inp.x, inp.timestep, cfg=True)
    a.close()
    b = UNet(ctx, params, f16_gemm=True)
    want = b.forward_host(inp.x, inp.timestep, cfg=True)
    b.close()
    assert np.array_equal(got, want)


def test_vae_from_file_equals_vae_from_table(ctx, tmp_path):
    params = V.random_vae()
    path = tmp_path / "vae.safetensors"
    write_weights(str(path), params, metadata={"scaling_factor": "0.13025"})
    lat = S.normal(29, (1, 16, 16, 4))
    a = Vae.from_file(ctx, str(path))
    got = a.decode_host(lat)
    a.close()
    want = Vae(ctx, params).decode_host(lat)
    assert np.array_equal(got, want)


# The converter keeps a GEMM weight f32 when its f16 copy would overflow
# (tools/convert_weights.py:27-30), so an f16 file can hold F32 members inside the
# groups the device fuses into one GEMM: self-lambda q | k | v, the stacked time
# projections, the VAE attention's q | k | v.
UNET_F32_MEMBERS = ("diff_model.down_blocks.1.resnets.0.time_emb_proj.weight",
                    "diff_model.down_blocks.0.attentions.1.transformer_blocks.0.attn1.to_k.weight")
VAE_F32_MEMBERS = ("decoder.mid_block.attentions.0.to_k.weight",)


def _round_f16(params, names):
    return {k: (v.astype(np.float16).astype(np.float32) if k in names else v) for k, v in params.items()}


def test_unet_file_with_f32_members_in_fused_groups(ctx, tmp_path):
    """Loads, and computes what an all-f32 model holding the same values computes
    (EXACT reads f16-stored weights through their exact f32 widening), bit for bit."""
    params = U.random_unet(seed=4000)
    gemm16 = [s.name for s in U.unet_specs() if s.gemm and s.name not in UNET_F32_MEMBERS]
    path = tmp_path / "unet_mixed.safetensors"
    write_weights(str(path), params, gemm16, f16=True)
    inp = U.unet_input(seed=5012)
    a = UNet.from_file(ctx, str(path))
    got = a.forward_host(inp.x, inp.timestep, cfg=True)
    a.close()
    b = UNet(ctx, _round_f16(params, set(gemm16)))
    want = b.forward_host(inp.x, inp.timestep, cfg=True)
    b.close()
    assert np.array_equal(got, want)


def test_vae_file_with_an_f32_member_in_the_attention_group(ctx, tmp_path):
    params = V.random_vae()
    gemm16 = [s.name for s in V.vae_specs() if s.gemm and s.name not in VAE_F32_MEMBERS]
    path = tmp_path / "vae_mixed.safetensors"
    write_weights(str(path), params, gemm16, f16=True, metadata={"scaling_factor": "0.13025"})
    lat = S.normal(31, (1, 16, 16, 4))
    a = Vae.from_file(ctx, str(path))
    got = a.decode_host(lat)
    a.close()
    want = Vae(ctx, _round_f16(params, set(gemm16))).decode_host(lat)
    assert np.max(np.abs(got - want)) <= 1e-5 * np.max(np.abs(want))


def test_bad_file_is_a_weights_error_before_any_upload(ctx, tmp_path):
    path = tmp_path / "vae.safetensors"
    write_weights(str(path), {"x": np.zeros(3, np.float32)}, metadata={"scaling_factor": "0.13025"})
    with pytest.raises(_lib.MoebiusError) as e:
        Vae.from_file(ctx, str(path))
    assert e.value.code == _lib.ERR_WEIGHTS and "missing tensor" in e.value.msg
