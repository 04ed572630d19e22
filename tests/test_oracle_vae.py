"""The oracle's VAE chain (oracle/vae.cpp) pinned without the reference's
weights: the tensor set against the reference's manifest counts and FLOP
totals, the row softmax and the posterior sample by closed forms, and the
resnet, mid attention, encoder and decoder against float64 restatements of
diffusers' AutoencoderKL definitions (tests/ref_f64.py) at small sizes."""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from moebius_cpu_amd import synthetic as S
from moebius_cpu_amd import vae_params as V
from tests import ref_f64 as R
from tests.util import max_abs_rel, rel_l2


@pytest.fixture(scope="module")
def params():
    return V.random_vae()


def test_tensor_set_matches_the_reference_manifest():
    """docs/weights-manifest.txt holds 248 VAE tensors (SURVEY: 1 455 = 1 203 UNet + 248 VAE);
    docs/PLAN.md:58-59 puts encode (B=2) at 2 233 GFLOP and decode at 2 515 GFLOP."""
    specs = V.vae_specs()
    assert len(specs) == 248 and len({s.name for s in specs}) == 248
    assert round(V.encode_flops(2, 512, 512) / 1e9) == 2233
    assert round(V.decode_flops(64, 64) / 1e9) == 2515
    shapes = {s.name: s.shape for s in specs}
    assert shapes["encoder.conv_in.weight"] == (128, 3, 3, 3)
    assert shapes["decoder.up_blocks.1.resnets.0.conv1.weight"] == (512, 3, 3, 512)
    assert shapes["decoder.up_blocks.2.resnets.0.conv_shortcut.weight"] == (256, 512)
    assert shapes["encoder.mid_block.attentions.0.to_out.0.weight"] == (512, 512)
    assert shapes["quant_conv.weight"] == (8, 8) and shapes["post_quant_conv.weight"] == (4, 4)


def test_softmax_rows_closed_forms():
    """src/vae/mod.rs:275-294: equal entries give exactly 1/n; entries whose
    scaled distance to the max is below -40 are flushed to exactly 0, and an
    entry just above the threshold is kept."""
    eq = oracle.softmax_rows(np.full((3, 8), 1.5, np.float32), 0.5)
    assert np.array_equal(eq, np.full((3, 8), 0.125, np.float32))
    row = np.array([[0.0, -100.0, -79.0, -81.0]], np.float32)
    got = oracle.softmax_rows(row, 0.5)  # scaled: 0, -50, -39.5, -40.5
    assert got[0, 1] == 0.0 and got[0, 3] == 0.0 and got[0, 2] > 0.0
    assert got[0, 0] == np.float32(1.0) / (np.float32(1.0) + np.float32(np.exp(-39.5)))


def test_softmax_rows_matches_f64():
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((17, 300)) * 3).astype(np.float32)
    got = oracle.softmax_rows(x, 0.7)
    s = x.astype(np.float64) * 0.7
    e = np.exp(s - s.max(axis=1, keepdims=True))
    want = e / e.sum(axis=1, keepdims=True)
    assert max_abs_rel(got, want) < 1e-6
    assert np.allclose(got.sum(axis=1, dtype=np.float64), 1.0, atol=1e-5)


def test_sample_closed_forms():
    """src/vae/encoder.rs:121-133: logvar 0 gives (mean + noise) * 0.13025; logvar
    is clamped to [-30, 20]; a NaN log-variance stays NaN (f32::clamp)."""
    m = np.zeros((3, 8), np.float32)
    m[:, :4] = [[1.0, 2.0, -1.0, 0.5]] * 3
    m[1, 4:] = 100.0
    m[2, 4:] = np.nan
    nz = np.ones((3, 4), np.float32)
    z = oracle.vae_sample(m, nz)
    sf = np.float32(0.13025)
    assert np.array_equal(z[0], (m[0, :4] + np.float32(1.0)) * sf)
    assert np.allclose(z[1], (m[1, :4] + np.exp(10.0)) * 0.13025, rtol=1e-6)
    assert np.all(np.isnan(z[2]))


@pytest.mark.parametrize("ci,co", [(128, 128), (128, 256)])
def test_resnet_matches_f64(params, ci, co):
    p = "encoder.down_blocks.1.resnets.0" if ci != co else "encoder.down_blocks.0.resnets.1"
    x = S.normal(11, (2, 6, 5, ci))
    got = oracle.vae_resnet(params, p, x, co)
    want = R.vae_resnet(params, p, x.astype(np.float64), ci, co)
    assert rel_l2(got, want) < 1e-5 and max_abs_rel(got, want) < 1e-4


def test_mid_attention_matches_f64(params):
    x = S.normal(12, (2, 7, 9, 512))
    p = "decoder.mid_block.attentions.0"
    got = oracle.vae_attention(params, p, x)
    want = R.vae_attention(params, p, x.astype(np.float64))
    assert rel_l2(got, want) < 1e-5 and max_abs_rel(got, want) < 1e-4


def test_encode_matches_f64(params):
    images = V.vae_images(seed=13, b=2, h=32, w=24)
    noise = S.normal(14, (2, 4, 3, 4))
    got = oracle.Vae(params).encode(images, noise)
    want = R.vae_encode(params, images, noise.astype(np.float64))
    assert got.shape == (2, 4, 3, 4)
    assert rel_l2(got, want) < 1e-4 and max_abs_rel(got, want) < 1e-3


def test_decode_matches_f64(params):
    lat = S.normal(15, (1, 3, 4, 4))
    got = oracle.Vae(params).decode(lat)
    want = R.vae_decode(params, lat.astype(np.float64))
    assert got.shape == (1, 24, 32, 3)
    assert rel_l2(got, want) < 1e-4 and max_abs_rel(got, want) < 1e-3
