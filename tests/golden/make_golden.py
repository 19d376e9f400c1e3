#!/usr/bin/env python3
"""Writes tests/golden/dit_small.npz: the expected outputs of a small DiT velocity evaluation,
computed by an independent float64 NumPy restatement of the block graph (not the C++ oracle, not
the GPU library).

Graph, following src/dit_fwd.cpp:104-304 op order with the configured two-stream variant:
  t -> 256-d sinusoid (cos half, sin half; fr_k = 1e4/t_max * 1e4^(-2k/D), src/dit_fwd.cpp:111-119)
    -> Linear + SiLU -> Linear, + pooled = g, gs = silu(g)                   (:122-140)
  audio rows = z W_in^T + b; text rows = text features                      (:142-149)
  joint block: per stream adaLN (chunks 0,1) -> QKV + b -> per-head RMS(q), RMS(k) -> RoPE on audio
    rows -> joint softmax attention -> out-proj + b, gate chunk 2 -> adaLN (chunks 3,4) ->
    FFN (audio: conv k3 pad 1, SiLU, conv k3; text: linear, SiLU, linear), gate chunk 5
  fused block: one weight set over all rows, RoPE on the audio rows, linear FFN  (:267-279)
  final layer: adaLN (2 chunks) on audio rows -> Linear + b                    (:287-303)

Weights and inputs come from the library's specified counter-based generator (BF16 weights, seed
below), so the fixture holds only seeds and expected outputs. Run from the repository root:
    python3 tests/golden/make_golden.py
"""
import importlib
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

SPEC = dict(B=2, La=12, Lt=5, H=256, NH=4, HD=64, F=512, latent=64, temb_dim=256, n_joint=1, n_fused=1,
            audio_ffn_conv=1, rope_theta=10000.0, t_max_period=1.0, ln_eps=1e-5, rms_eps=1e-6)
WEIGHT_SEED, INPUT_SEED, NORM_MEAN = 77, 78, 1.0


def silu(x):
    return x / (1.0 + np.exp(-x))


def layer_norm(x, eps):
    mu = x.mean(-1, keepdims=True)
    return (x - mu) / np.sqrt(((x - mu) ** 2).mean(-1, keepdims=True) + eps)


def rms_heads(x, w, nh, eps):
    h = x.reshape(x.shape[0], nh, -1)
    return (h / np.sqrt((h ** 2).mean(-1, keepdims=True) + eps) * w).reshape(x.shape)


def rope(x, nh, theta, npos):
    """rotate pairs (2j, 2j+1) of each head by pos * theta^(-2j/64) for the first npos rows"""
    L = x.shape[0]
    h = x.reshape(L, nh, -1).copy()
    hd = h.shape[-1]
    j = np.arange(hd // 2)
    ang = np.arange(L)[:, None] * theta ** (-2.0 * j / hd)[None, :]
    ang[npos:] = 0.0
    c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
    e, o = h[..., 0::2].copy(), h[..., 1::2].copy()
    h[..., 0::2] = e * c - o * s
    h[..., 1::2] = e * s + o * c
    return h.reshape(L, -1)


def attention(q, k, v, nh, scale):
    L = q.shape[0]
    out = np.empty_like(q)
    hd = q.shape[1] // nh
    for h in range(nh):
        sl = slice(h * hd, (h + 1) * hd)
        s = q[:, sl] @ k[:, sl].T * scale
        p = np.exp(s - s.max(1, keepdims=True))
        out[:, sl] = (p / p.sum(1, keepdims=True)) @ v[:, sl]
    return out


def conv3(x, w):
    """x [T, IC], w [OC, IC, 3]: y[t] = sum_k w[:, :, k] x[t - 1 + k], zero padded"""
    xp = np.pad(x, ((1, 1), (0, 0)))
    return sum(xp[k:k + x.shape[0]] @ w[:, :, k].T for k in range(3))


def forward(spec, get, z, t, text, pooled):
    B, La, Lt, H, NH, F = spec["B"], spec["La"], spec["Lt"], spec["H"], spec["NH"], spec["F"]
    D = spec["temb_dim"]
    k = np.arange(D // 2)
    fr = (1e4 / spec["t_max_period"]) * 1e4 ** (-2.0 * k / D)
    taps = []
    v = np.empty((B, La, spec["latent"]))
    for b in range(B):
        emb = np.concatenate([np.cos(t[b] * fr), np.sin(t[b] * fr)])
        h1 = silu(get("t_embed.mlp.0.weight", (H, D)) @ emb + get("t_embed.mlp.0.bias"))
        g = get("t_embed.mlp.2.weight", (H, H)) @ h1 + get("t_embed.mlp.2.bias") + pooled[b]
        gs = silu(g)
        X = np.concatenate([z[b] @ get("audio_input_proj.weight", (H, spec["latent"])).T + get("audio_input_proj.bias"),
                            text[b]], 0)
        btaps = []
        for i in range(spec["n_joint"]):
            streams = [("joint_blocks.%d.latent_block" % i, 0, La, True, True),
                       ("joint_blocks.%d.text_block" % i, La, Lt, False, False)]
            X = block(spec, get, X, gs, streams)
            btaps.append(X.copy())
        for i in range(spec["n_fused"]):
            X = block(spec, get, X, gs, [("fused_blocks.%d" % i, 0, La + Lt, La, False)])
            btaps.append(X.copy())
        mod = get("final_layer.adaLN_modulation.1.weight", (2 * H, H)) @ gs + get("final_layer.adaLN_modulation.1.bias")
        xn = layer_norm(X[:La], spec["ln_eps"]) * (1 + mod[H:]) + mod[:H]
        v[b] = xn @ get("final_layer.linear.weight", (spec["latent"], H)).T + get("final_layer.linear.bias")
        taps.append(btaps)
    return v, np.array(taps).transpose(1, 0, 2, 3)


def block(spec, get, X, gs, streams):
    """streams: (prefix, first row, rows, rope rows (True = all, int = first n, False = none), conv FFN)"""
    H, NH, F, eps, reps = spec["H"], spec["NH"], spec["F"], spec["ln_eps"], spec["rms_eps"]
    X = X.copy()
    mods, qs, ks, vs = [], [], [], []
    for (p, lo, L, rp, conv) in streams:
        mod = get(p + ".adaLN_modulation.1.weight", (6 * H, H)) @ gs + get(p + ".adaLN_modulation.1.bias")
        xn = layer_norm(X[lo:lo + L], eps) * (1 + mod[H:2 * H]) + mod[:H]
        qkv = xn @ get(p + ".attn.qkv.weight", (3 * H, H)).T + get(p + ".attn.qkv.bias")
        q = rms_heads(qkv[:, :H], get(p + ".attn.q_norm.weight"), NH, reps)
        kk = rms_heads(qkv[:, H:2 * H], get(p + ".attn.k_norm.weight"), NH, reps)
        npos = L if rp is True else (0 if rp is False else rp)
        q, kk = rope(q, NH, spec["rope_theta"], npos), rope(kk, NH, spec["rope_theta"], npos)
        mods.append(mod); qs.append(q); ks.append(kk); vs.append(qkv[:, 2 * H:])
    A = attention(np.concatenate(qs), np.concatenate(ks), np.concatenate(vs), NH, 1.0 / 8.0)
    row = 0
    for (p, lo, L, rp, conv), mod in zip(streams, mods):
        x = X[lo:lo + L] + (A[row:row + L] @ get(p + ".linear1.weight", (H, H)).T + get(p + ".linear1.bias")) * mod[2 * H:3 * H]
        row += L
        xn = layer_norm(x, eps) * (1 + mod[4 * H:5 * H]) + mod[3 * H:4 * H]
        if conv:
            f = conv3(silu(conv3(xn, get(p + ".ffn.w1.weight", (F, H, 3)))), get(p + ".ffn.w2.weight", (H, F, 3)))
        else:
            f = silu(xn @ get(p + ".ffn.w1.weight", (F, H)).T) @ get(p + ".ffn.w2.weight", (H, F)).T
        X[lo:lo + L] = x + f * mod[5 * H:6 * H]
    return X


def main():
    tsn = importlib.import_module("thinksound-native_amd")
    spec = tsn.DitSpec(**SPEC)
    w = tsn.bf16_to_f32(tsn.synth_weights(spec, WEIGHT_SEED, NORM_MEAN)).astype(np.float64)
    idx = {name: (off, n) for name, n, off in tsn.manifest(spec)}

    def get(name, shape=None):
        off, n = idx[name]
        a = w[off:off + n]
        return a.reshape(shape) if shape else a

    inp = tsn.synth_inputs(spec, INPUT_SEED, cfg_pairs=False)
    v, taps = forward(SPEC, get, *(inp[k].astype(np.float64) for k in ("z", "t", "text", "pooled")))
    out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "dit_small.npz")
    np.savez_compressed(out, spec_keys=np.array(list(SPEC)), spec_vals=np.array([float(SPEC[k]) for k in SPEC]),
                        seeds=np.array([WEIGHT_SEED, INPUT_SEED]), norm_mean=np.array(NORM_MEAN),
                        v=v.astype(np.float32), taps=taps.astype(np.float32),
                        z_checksum=np.array(inp["z"].astype(np.float64).sum()),
                        w_checksum=np.array(w.sum()))
    print("wrote", out, v.shape, taps.shape, "v std %.4f" % v.std())


if __name__ == "__main__":
    main()
