"""float64 numpy restatements of the UNet blocks from their mathematical
definitions (not from the reference's folded / banded implementation): used
to pin the oracle. The lambda layers are written in the upstream, unfolded
form documented at src/unet/lambda.rs:131-172: the self-lambda position
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
