#!/usr/bin/env python3
"""Precision study of the reference checkpoint's graph (src/dit_fwd.cpp:104-304) at 8 s, one
sample: a float32 NumPy emulation of the forward in which chosen operand sites are rounded to f16,
one site set per command-line argument, reporting the velocity rel-L2 against the all-f32
emulation and the latent stream's rel-L2 after every block. This regenerates the per-site table
that decided which GEMM operands the GPU graph keeps as f32-accurate hi|lo pairs.

Site tags (a trailing L restricts a tag to the latent stream, CT to the clip and text streams):
  extc  silu(extended_c), the per-row modulation operand   in    input projection hidden
  xn1   LN1 output -> QKV        qk / v  q, k / v inside attention    ao   attention output -> out-proj
  xn2   LN2 output -> FFN1       hf      SwiGLU hidden -> FFN2        mod  modulation rows
  xn    both LN outputs          all     every site
Sites combine with '+'. Example (about 20 s per site set on 8 cores):
    python3 tests/precision_sites.py extc xn2L hfL aoL in xn1 qk v xn2CT+hfCT+aoCT
With PREP=1 the clip/text/sync/gcmlp inputs come from the conditioning-prep oracle instead of
N(0, 1) draws. Run from anywhere; weights are the seeded synthetic BF16 set (seed 4242, q/k norm
weights 1 + N(0, 0.02)).
"""
import importlib
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
tsn = importlib.import_module('thinksound-native_amd')


def h16(a): return a.astype(np.float16).astype(np.float32)
def silu(x): return x / (1 + np.exp(-x))
def ln(x, eps):
    mu = x.mean(-1, keepdims=True); d = x - mu
    return d / np.sqrt((d * d).mean(-1, keepdims=True) + eps)

spec = tsn.ref_spec_for_duration(8, 2); d = spec.as_dict()
T, L = d['T'], d['latent']
H, NH, F, L, T, C, TS = d["H"], d["NH"], d["F"], d["latent"], d["T"], d["C"], d["TS"]
w16 = tsn.ref_synth_weights(spec, 4242, 1.0)
man = {n: (o, k) for n, k, o in tsn.ref_manifest(spec)}
cache = {}
def get(n, shape=None, conv=False):
    key = (n, conv)
    if key not in cache:
        o, k = man[n]; a = tsn.bf16_to_f32(w16[o:o + k])
        if shape: a = a.reshape(shape)
        if conv: a = np.ascontiguousarray(a.transpose(2, 1, 0))   # [K][IC][OC]
        elif a.ndim == 2: a = np.ascontiguousarray(a.T)           # [IC][OC]
        cache[key] = a
    return cache[key]
def conv(x, wk, b, pad):   # wk [K][IC][OC]
    K = wk.shape[0]; xp = np.pad(x, ((pad, K - 1 - pad), (0, 0)))
    y = xp[0:len(x)] @ wk[0]
    for k in range(1, K): y += xp[k:k + len(x)] @ wk[k]
    return y + b if b is not None else y
def rope(x, fscale):
    Lr = x.shape[0]; h = x.reshape(Lr, NH, 64).copy()
    inv = (10000.0 ** (-2.0 * np.arange(32) / 64)).astype(np.float32)
    ang = (np.arange(Lr, dtype=np.float32) * np.float32(fscale))[:, None] * inv[None, :]
    c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
    e, o = h[..., 0::2].copy(), h[..., 1::2].copy()
    h[..., 0::2] = e * c - o * s; h[..., 1::2] = e * s + o * c
    return h.reshape(Lr, -1)
def attn(q, k, v):
    out = np.empty_like(q)
    for h in range(NH):
        sl = slice(h * 64, (h + 1) * 64)
        s = q[:, sl] @ k[:, sl].T / 8.0
        p = np.exp(s - s.max(1, keepdims=True)); out[:, sl] = (p / p.sum(1, keepdims=True)) @ v[:, sl]
    return out

def fwd(flags, x, t, clip_pp, text_pp, gcmlp, sync_gather):
    r = lambda tag, a: h16(a) if (tag in flags or 'all' in flags) else a
    def ffn(p, xn, cv):
        st = 'L' if ('latent' in p or 'fused' in p or 'input' in p) else 'CT'
        xn = r('xn2' + st, r('xn2', r('xn', xn)))
        if cv:
            h = silu(conv(xn, get(p + ".w1.weight", (F, H, 3), True), None, 1)) * conv(xn, get(p + ".w3.weight", (F, H, 3), True), None, 1)
            return conv(r('hf' + st, r('hf', h)), get(p + ".w2.weight", (H, F, 3), True), None, 1)
        h = silu(xn @ get(p + ".w1.weight", (F, H))) * (xn @ get(p + ".w3.weight", (F, H)))
        return r('hf' + st, r('hf', h)) @ get(p + ".w2.weight", (H, F))
    def pre(p, xs, mod, fscale):
        st = 'L' if ('latent' in p or 'fused' in p) else 'CT'
        xn = r('xn1' + st, r('xn1', r('xn', ln(xs, 1e-5) * (1 + mod[..., H:2 * H]) + mod[..., :H])))
        qkv = xn @ get(p + ".attn.qkv.weight", (3 * H, H)) + get(p + ".attn.qkv.bias")
        qkv = np.concatenate([qkv[:, 0::3], qkv[:, 1::3], qkv[:, 2::3]], 1)
        out = []
        for c, nm in ((0, "q_norm"), (H, "k_norm")):
            hh = qkv[:, c:c + H].reshape(len(xs), NH, -1)
            hh = (hh / np.sqrt((hh ** 2).mean(-1, keepdims=True) + 1e-6) * get(p + ".attn." + nm + ".weight")).reshape(len(xs), H)
            out.append(r('qk' + st, r('qk', rope(hh, fscale) if fscale else hh)))
        return out[0], out[1], r('v' + st, r('v', qkv[:, 2 * H:]))
    def post(p, xs, a, mod, cv):
        st = 'L' if ('latent' in p or 'fused' in p) else 'CT'
        a = r('ao' + st, r('ao', a))
        o = conv(a, get(p + ".linear1.weight", (H, H, 3), True), get(p + ".linear1.bias"), 1) if cv else \
            a @ get(p + ".linear1.weight", (H, H)) + get(p + ".linear1.bias")
        xs = xs + o * mod[..., 2 * H:3 * H]
        xn = ln(xs, 1e-5) * (1 + mod[..., 4 * H:5 * H]) + mod[..., 3 * H:4 * H]
        return xs + ffn(p + ".ffn", xn, cv) * mod[..., 5 * H:6 * H]
    fr = (1e4 * 1e4 ** (-2.0 * np.arange(H // 2) / H)).astype(np.float32)
    b = 0
    emb = np.concatenate([np.cos(t[b] * fr), np.sin(t[b] * fr)])
    te = silu(emb @ get("t_embed.mlp.0.weight", (H, H)) + get("t_embed.mlp.0.bias")) @ get("t_embed.mlp.2.weight", (H, H)) + get("t_embed.mlp.2.bias")
    gc = gcmlp[b] + te
    extc = r('extc', silu(sync_gather[b] + gc)); gs = silu(gc)
    xin = r('in', silu(conv(x[b], get("audio_input_proj.0.weight", (H, L, 3), True), get("audio_input_proj.0.bias"), 1)))
    h = silu(conv(xin, get("audio_input_proj.2.w1.weight", (F, H, 3), True), None, 1)) * conv(xin, get("audio_input_proj.2.w3.weight", (F, H, 3), True), None, 1)
    lat = conv(r('in', h), get("audio_input_proj.2.w2.weight", (H, F, 3), True), None, 1)
    clip, text = clip_pp[b].copy(), text_pp[b].copy()
    taps = []
    for i in range(d["n_joint"]):
        pre_only = i == d["n_joint"] - 1; cc = 2 if pre_only else 6; p = "joint_blocks.%d" % i
        ml = r('mod', extc @ get(p + ".latent_block.adaLN_modulation.1.weight", (6 * H, H)) + get(p + ".latent_block.adaLN_modulation.1.bias"))
        mc = gs @ get(p + ".clip_block.adaLN_modulation.1.weight", (cc * H, H)) + get(p + ".clip_block.adaLN_modulation.1.bias")
        mt = gs @ get(p + ".text_block.adaLN_modulation.1.weight", (cc * H, H)) + get(p + ".text_block.adaLN_modulation.1.bias")
        parts = [pre(p + ".latent_block", lat, ml, 1.0), pre(p + ".clip_block", clip, mc, T / C), pre(p + ".text_block", text, mt, 0.0)]
        A = attn(*(np.concatenate([pp[j] for pp in parts]) for j in range(3)))
        lat = post(p + ".latent_block", lat, A[:T], ml, True)
        if not pre_only:
            clip = post(p + ".clip_block", clip, A[T:T + C], mc, True)
            text = post(p + ".text_block", text, A[T + C:], mt, False)
        taps.append(lat.copy())
    for i in range(d["n_fused"]):
        p = "fused_blocks.%d" % i
        ml = r('mod', extc @ get(p + ".adaLN_modulation.1.weight", (6 * H, H)) + get(p + ".adaLN_modulation.1.bias"))
        q, k, vv = pre(p, lat, ml, 1.0)
        lat = post(p, lat, attn(q, k, vv), ml, True)
        taps.append(lat.copy())
    mf = extc @ get("final_layer.adaLN_modulation.1.weight", (2 * H, H)) + get("final_layer.adaLN_modulation.1.bias")
    xn = ln(lat, 1e-5) * (1 + mf[:, H:]) + mf[:, :H]
    return conv(xn, get("final_layer.conv.weight", (L, H, 7), True), get("final_layer.conv.bias"), 3), taps

inp = tsn.ref_synth_inputs(spec, 4242)
inp1 = {k: v[:1] for k, v in inp.items()}
if os.environ.get("PREP"):
    sys.path.insert(0, os.path.join(ROOT, 'oracle')); sys.path.insert(0, os.path.join(ROOT, 'tests'))
    import pyoracle as orc
    from conftest import rng as _rng
    cs = tsn.cond_spec_for_duration(8)
    cw = tsn.bf16_to_f32(tsn.cond_synth_weights(cs, 99))
    rr = _rng(8)
    f = lambda *sh: rr.standard_normal(sh).astype(np.float32)
    clip_f, sync_f, text_c = f(cs.C, cs.clip_dim), f(cs.sync_S, cs.sync_dim), f(cs.TS, cs.text_dim)
    f(cs.TS, cs.text_dim)
    gtext = f(cs.gtext_dim)
    cpp, sg, cfc = orc.ref_prep_conditioning(cs.as_dict(), cw, clip_f, sync_f)
    tp, gc = orc.ref_prep_text_arm(cs.as_dict(), cw, text_c, gtext, cfc)
    inp1 = dict(x=_rng(9).standard_normal((1, T, L)).astype(np.float32), t=np.array([0.7], np.float32),
                clip_pp=cpp[None], text_pp=tp[None], gcmlp=gc[None], sync_gather=sg[None])
    print('prep-derived inputs: std clip %.3g text %.3g gcmlp %.3g sync %.3g' % (cpp.std(), tp.std(), gc.std(), sg.std()))
rl = lambda a, b: float(np.linalg.norm((a - b).astype(np.float64)) / np.linalg.norm(b.astype(np.float64)))
a = time.time(); v0, t0 = fwd(set(), **inp1); print('base %.1fs' % (time.time() - a), flush=True)
for fl in sys.argv[1:]:
    f = set(fl.split('+'))
    v1, t1 = fwd(f, **inp1)
    print('%-20s v %.3g  taps %s' % (fl, rl(v1, v0), ' '.join('%.2g' % rl(x, y) for x, y in zip(t1, t0))), flush=True)
