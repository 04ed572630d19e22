"""float64 numpy restatements of the UNet blocks from their mathematical
definitions (not from the reference's folded / banded implementation): used
to pin the oracle. The lambda layers are written in the upstream, unfolded
form documented at src/unet/lambda.rs:7-43: the self-lambda position
lambda lambda_p materialised by the 15x15 Conv3d, the cross-lambda position
lambda as E . V per pixel."""
from __future__ import annotations

import numpy as np

HEADS = 8


def silu(x):
    return x / (1.0 + np.exp(-x))


def group_norm(x, groups, eps, gamma, beta):
    n, h, w, c = x.shape
    xs = x.reshape(n, h * w, groups, c // groups)
    mean = xs.mean(axis=(1, 3), keepdims=True)
    var = xs.var(axis=(1, 3), keepdims=True)
    y = ((xs - mean) / np.sqrt(var + np.float64(np.float32(eps)))).reshape(n, h, w, c)
    return y * gamma + beta


def layer_norm(x, gamma, beta, eps):
    mean = x.mean(axis=-1, keepdims=True)
    var = x.var(axis=-1, keepdims=True)
    return (x - mean) / np.sqrt(var + np.float64(np.float32(eps))) * gamma + beta


def linear(x, w, b=None):
    y = x @ w.T
    return y if b is None else y + b


def depthwise(x, w, b):
    n, h, wd, c = x.shape
    xp = np.zeros((n, h + 2, wd + 2, c))
    xp[:, 1:-1, 1:-1] = x
    y = np.broadcast_to(b, x.shape).copy()
    for ky in range(3):
        for kx in range(3):
            y += xp[:, ky:ky + h, kx:kx + wd] * w[ky, kx]
    return y


def P(params, name):
    return params[name].astype(np.float64)


def dwconv2d(params, p, x, ci, co):
    mid = np.maximum(depthwise(x, P(params, p + ".conv_dw.weight"), P(params, p + ".conv_dw.bias")), 0.0)
    y = linear(mid, P(params, p + ".conv_pw.weight"), P(params, p + ".conv_pw.bias"))
    return y + x if ci == co else y


def resnet(params, p, x, temb, ci, co, eps=1e-5):
    a = silu(group_norm(x, 32, eps, P(params, p + ".norm1.weight"), P(params, p + ".norm1.bias")))
    b = dwconv2d(params, p + ".conv1", a, ci, co)
    tp = linear(silu(temb), P(params, p + ".time_emb_proj.weight"), P(params, p + ".time_emb_proj.bias"))
    a = silu(group_norm(b + tp[:, None, None, :], 32, eps, P(params, p + ".norm2.weight"),
                        P(params, p + ".norm2.bias")))
    out = dwconv2d(params, p + ".conv2", a, co, co)
    if ci != co:
        return out + linear(x, P(params, p + ".conv_shortcut.weight"), P(params, p + ".conv_shortcut.bias"))
    return out + x


def self_lambda(params, p, x):
    n, hh, ww, c = x.shape
    k = c // HEADS
    q = linear(x, P(params, p + ".to_q.weight"), P(params, p + ".to_q.bias")).reshape(n, hh * ww, HEADS, k)
    keys = linear(x, P(params, p + ".to_k.weight")).reshape(n, hh * ww, k)
    v = linear(x, P(params, p + ".to_v.weight"), P(params, p + ".to_v.bias")).reshape(n, hh, ww, k)
    sk = np.exp(keys - keys.max(axis=1, keepdims=True))
    sk /= sk.sum(axis=1, keepdims=True)
    lam_c = np.einsum("bnk,bnv->bkv", sk, v.reshape(n, hh * ww, k))
    yc = np.einsum("bnhk,bkv->bnhv", q, lam_c)
    # lambda_p[b, k, v, y, x] = sum_{dy,dx} W[k, dy*15+dx] V[b, y+dy-7, x+dx-7, v] + bias[k]
    wpos = P(params, p + ".pos_conv.weight").reshape(k, 15, 15)
    bpos = P(params, p + ".pos_conv.bias")
    vp = np.zeros((n, hh + 14, ww + 14, k))
    vp[:, 7:7 + hh, 7:7 + ww] = v
    lam_p = np.zeros((n, k, hh, ww, k)) + bpos[None, :, None, None, None]
    for dy in range(15):
        for dx in range(15):
            lam_p += wpos[None, :, dy, dx, None, None, None] * vp[:, None, dy:dy + hh, dx:dx + ww, :]
    lam_p = lam_p.reshape(n, k, hh * ww, k)  # [b, k, n, v]
    yp = np.einsum("bnhk,bknv->bnhv", q, lam_p)
    return (yc + yp).reshape(n, hh, ww, c)


def conditioning(params):
    """src/unet/embed.rs:72-83 semantics: [uncond = ids 10..20, cond = ids 0..10] projected."""
    table = P(params, "embedding_layer.weight")
    w, b = P(params, "diff_model.encoder_hid_proj.weight"), P(params, "diff_model.encoder_hid_proj.bias")
    return [linear(table[10:20], w, b), linear(table[0:10], w, b)]


def cross_lambda(params, p, x, branches):
    n, hh, ww, c = x.shape
    k = c // HEADS
    ehs = conditioning(params)
    q = linear(x, P(params, p + ".to_q.weight"), P(params, p + ".to_q.bias")).reshape(n, hh * ww, HEADS, k)
    e = P(params, p + ".rel_pos_emb")  # [N, 10, k]
    out = np.zeros((n, hh * ww, HEADS, k))
    for i, br in enumerate(branches):
        keys = linear(ehs[br], P(params, p + ".to_k.weight"))                          # [10, k]
        v = linear(ehs[br], P(params, p + ".to_v.weight"), P(params, p + ".to_v.bias"))  # [10, v]
        sk = np.exp(keys - keys.max(axis=0, keepdims=True))
        sk /= sk.sum(axis=0, keepdims=True)
        lam_c = sk.T @ v                                        # [k, v]
        lam_p = np.einsum("nmk,mv->nkv", e, v)                  # per pixel [k, v]
        out[i] = np.einsum("nhk,kv->nhv", q[i], lam_c) + np.einsum("nhk,nkv->nhv", q[i], lam_p)
    return out.reshape(n, hh, ww, c)


def transformer(params, p, x, branches):
    c = x.shape[-1]
    hidden = int(c * 2.5)
    b = p + ".transformer_blocks.0"
    ff = b + ".ff"
    t = group_norm(x, 32, 1e-6, P(params, p + ".norm.weight"), P(params, p + ".norm.bias"))
    h = linear(t, P(params, p + ".proj_in.weight"), P(params, p + ".proj_in.bias"))
    h = h + self_lambda(params, b + ".attn1",
                        layer_norm(h, P(params, b + ".norm1.weight"), P(params, b + ".norm1.bias"), 1e-5))
    h = h + cross_lambda(params, b + ".attn2",
                         layer_norm(h, P(params, b + ".norm2.weight"), P(params, b + ".norm2.bias"), 1e-5), branches)
    t = layer_norm(h, P(params, b + ".norm3.weight"), P(params, b + ".norm3.bias"), 1e-5)
    a = silu(linear(t, P(params, ff + ".inverted_conv.conv.weight"), P(params, ff + ".inverted_conv.conv.bias")))
    d = depthwise(a, P(params, ff + ".depth_conv.conv.weight"), P(params, ff + ".depth_conv.conv.bias"))
    g = d[..., :hidden] * silu(d[..., hidden:])
    u = linear(g, P(params, ff + ".point_conv.conv.weight")) + h
    return linear(u, P(params, p + ".proj_out.weight"), P(params, p + ".proj_out.bias")) + x


def timestep_embedding_sinusoid(t):
    """diffusers Timesteps(320, flip_sin_to_cos=True, downscale_freq_shift=0) in f64."""
    half = 160
    freq = np.exp(-np.log(10000.0) * np.arange(half) / half)
    arg = t * freq
    return np.concatenate([np.cos(arg), np.sin(arg)])


# ---- VAE (diffusers AutoencoderKL definitions, upstream of src/vae)
VAE_CH = (128, 256, 512, 512)


def conv3x3(x, w, b, stride=1, pad=(1, 1, 1, 1), up=False):
    """Direct 3x3 conv in f64: x [n,h,w,ci], w [co,3,3,ci]; pad = top, left, bottom, right."""
    if up:
        x = x.repeat(2, axis=1).repeat(2, axis=2)
    n, h, w_, ci = x.shape
    xp = np.zeros((n, h + pad[0] + pad[2], w_ + pad[1] + pad[3], ci))
    xp[:, pad[0]:pad[0] + h, pad[1]:pad[1] + w_] = x
    ho = (h + pad[0] + pad[2] - 3) // stride + 1
    wo = (w_ + pad[1] + pad[3] - 3) // stride + 1
    out = np.zeros((n, ho, wo, w.shape[0])) + b
    for ky in range(3):
        for kx in range(3):
            patch = xp[:, ky:ky + stride * (ho - 1) + 1:stride, kx:kx + stride * (wo - 1) + 1:stride]
            out += patch @ w[:, ky, kx, :].T
    return out


def vae_resnet(params, p, x, ci, co):
    g = lambda n: P(params, n)  # noqa: E731
    h = silu(group_norm(x, 32, 1e-6, g(p + ".norm1.weight"), g(p + ".norm1.bias")))
    h = conv3x3(h, g(p + ".conv1.weight"), g(p + ".conv1.bias"))
    h = silu(group_norm(h, 32, 1e-6, g(p + ".norm2.weight"), g(p + ".norm2.bias")))
    h = conv3x3(h, g(p + ".conv2.weight"), g(p + ".conv2.bias"))
    sc = linear(x, g(p + ".conv_shortcut.weight"), g(p + ".conv_shortcut.bias")) if ci != co else x
    return sc + h


def vae_attention(params, p, x):
    g = lambda n: P(params, n)  # noqa: E731
    n, h, w, c = x.shape
    t = group_norm(x, 32, 1e-6, g(p + ".group_norm.weight"), g(p + ".group_norm.bias")).reshape(n, h * w, c)
    q = linear(t, g(p + ".to_q.weight"), g(p + ".to_q.bias"))
    k = linear(t, g(p + ".to_k.weight"), g(p + ".to_k.bias"))
    v = linear(t, g(p + ".to_v.weight"), g(p + ".to_v.bias"))
    s = q @ k.transpose(0, 2, 1) / np.sqrt(c)
    s = np.exp(s - s.max(axis=-1, keepdims=True))
    a = (s / s.sum(axis=-1, keepdims=True)) @ v
    return linear(a, g(p + ".to_out.0.weight"), g(p + ".to_out.0.bias")).reshape(n, h, w, c) + x


def vae_mid(params, p, x):
    c = x.shape[-1]
    x = vae_resnet(params, p + ".resnets.0", x, c, c)
    x = vae_attention(params, p + ".attentions.0", x)
    return vae_resnet(params, p + ".resnets.1", x, c, c)


def vae_encode(params, images, noise):
    """AutoencoderKL.encode(x).latent_dist.sample() * 0.13025 with the given noise."""
    g = lambda n: P(params, n)  # noqa: E731
    e = "encoder"
    x = conv3x3(images.astype(np.float64), g(e + ".conv_in.weight"), g(e + ".conv_in.bias"))
    c_prev = VAE_CH[0]
    for i, c in enumerate(VAE_CH):
        for j in range(2):
            x = vae_resnet(params, f"{e}.down_blocks.{i}.resnets.{j}", x, c_prev if j == 0 else c, c)
        if i + 1 < len(VAE_CH):
            x = conv3x3(x, g(f"{e}.down_blocks.{i}.downsamplers.0.conv.weight"),
                        g(f"{e}.down_blocks.{i}.downsamplers.0.conv.bias"), stride=2, pad=(0, 0, 1, 1))
        c_prev = c
    x = vae_mid(params, e + ".mid_block", x)
    x = silu(group_norm(x, 32, 1e-6, g(e + ".conv_norm_out.weight"), g(e + ".conv_norm_out.bias")))
    x = conv3x3(x, g(e + ".conv_out.weight"), g(e + ".conv_out.bias"))
    m = linear(x, g("quant_conv.weight"), g("quant_conv.bias"))
    mean, logvar = m[..., :4], np.clip(m[..., 4:], -30.0, 20.0)
    return (mean + np.exp(0.5 * logvar) * noise) * 0.13025


def vae_decode(params, latents):
    """(AutoencoderKL.decode(z / 0.13025) + 1) / 2."""
    g = lambda n: P(params, n)  # noqa: E731
    d = "decoder"
    z = linear(latents.astype(np.float64) / np.float64(np.float32(0.13025)), g("post_quant_conv.weight"),
               g("post_quant_conv.bias"))
    x = conv3x3(z, g(d + ".conv_in.weight"), g(d + ".conv_in.bias"))
    x = vae_mid(params, d + ".mid_block", x)
    c_prev = VAE_CH[-1]
    for i, c in enumerate(reversed(VAE_CH)):
        for j in range(3):
            x = vae_resnet(params, f"{d}.up_blocks.{i}.resnets.{j}", x, c_prev if j == 0 else c, c)
        if i + 1 < len(VAE_CH):
            x = conv3x3(x, g(f"{d}.up_blocks.{i}.upsamplers.0.conv.weight"),
                        g(f"{d}.up_blocks.{i}.upsamplers.0.conv.bias"), up=True)
        c_prev = c
    x = silu(group_norm(x, 32, 1e-6, g(d + ".conv_norm_out.weight"), g(d + ".conv_norm_out.bias")))
    x = conv3x3(x, g(d + ".conv_out.weight"), g(d + ".conv_out.bias"))
    return (x + 1.0) / 2.0
