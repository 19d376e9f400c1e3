"""Pinning of the oracle's reference-graph restatement (oracle/oracle_ref.cpp) and conditioning
prep (oracle/oracle_cond.cpp) — CPU only.

Checked against:
  * a float64 NumPy restatement of the three-stream graph written here from the reference forward
    (per-row adaLN from extended_c, element-interleaved qkv rows, SwiGLU conv-MLPs, conv-k3 out-proj,
    clip RoPE scaled by T/C, pre-only last joint block, conv-k7 final layer);
  * structure: the pre-only block leaves the clip and text rows untouched, fused blocks never touch
    them, samples do not mix;
  * closed form: a zero final conv makes the velocity its bias and the sampler moves x by -bias;
  * conditioning prep (src/dit.cpp:55-191) against a float64 NumPy restatement, with the sync
    gather's row choice as a known answer.
"""
import numpy as np
import pytest

from conftest import rel_l2, rng


def tiny_ref_spec(B=2):
    return dict(B=B, T=6, C=3, TS=4, H=128, NH=2, HD=64, F=192, latent=8, n_joint=2, n_fused=1,
                rope_theta=10000.0, t_max_period=1.0, ln_eps=1e-5, rms_eps=1e-6)


def ref_weights(orc, spec, seed=0):
    man = orc.ref_manifest(spec)
    r = rng(seed)
    w = np.empty(sum(n for _, n, _ in man), np.float32)
    for name, n, off in man:
        mean = 1.0 if "norm.weight" in name else 0.0
        w[off:off + n] = (mean + 0.05 * r.standard_normal(n)).astype(np.float32)
    return w, {name: (off, n) for name, n, off in man}


def ref_inputs(spec, seed=1):
    r = rng(seed)
    B, T, C, TS, H = spec["B"], spec["T"], spec["C"], spec["TS"], spec["H"]
    f = lambda *sh: r.standard_normal(sh).astype(np.float32)
    return dict(x=f(B, T, spec["latent"]), t=np.array([0.3, 0.8][:B] + [0.5] * max(0, B - 2), np.float32),
                clip_pp=f(B, C, H), text_pp=f(B, TS, H), gcmlp=f(B, H), sync_gather=f(B, T, H))


# ---------------- float64 restatement ----------------
def _silu(x):
    return x / (1 + np.exp(-x))


def _ln(x, eps):
    mu = x.mean(-1, keepdims=True)
    return (x - mu) / np.sqrt(((x - mu) ** 2).mean(-1, keepdims=True) + eps)


def _conv(x, w, b, pad):
    """x [T, IC], w [OC, IC, K]: y[t] = sum_k w[:, :, k] x[t - pad + k] (+ b)"""
    K = w.shape[2]
    xp = np.pad(x, ((pad, K - 1 - pad), (0, 0)))
    y = sum(xp[k:k + x.shape[0]] @ w[:, :, k].T for k in range(K))
    return y + b if b is not None else y


def _rope(x, nh, theta, fscale):
    L = x.shape[0]
    h = x.reshape(L, nh, -1).copy()
    hd = h.shape[-1]
    ang = (np.arange(L) * fscale)[:, None] * theta ** (-2.0 * np.arange(hd // 2) / hd)[None, :]
    c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
    e, o = h[..., 0::2].copy(), h[..., 1::2].copy()
    h[..., 0::2] = e * c - o * s
    h[..., 1::2] = e * s + o * c
    return h.reshape(L, -1)


def _attn(q, k, v, nh):
    out = np.empty_like(q)
    hd = q.shape[1] // nh
    for h in range(nh):
        sl = slice(h * hd, (h + 1) * hd)
        s = q[:, sl] @ k[:, sl].T / np.sqrt(hd)
        p = np.exp(s - s.max(1, keepdims=True))
        out[:, sl] = (p / p.sum(1, keepdims=True)) @ v[:, sl]
    return out


def np_ref_forward(spec, w, idx, x, t, clip_pp, text_pp, gcmlp, sync_gather):
    H, NH, F, L, T, C, TS = spec["H"], spec["NH"], spec["F"], spec["latent"], spec["T"], spec["C"], spec["TS"]
    eps, reps, theta = spec["ln_eps"], spec["rms_eps"], spec["rope_theta"]

    def get(n, shape=None):
        o, k = idx[n]
        a = w[o:o + k].astype(np.float64)
        return a.reshape(shape) if shape else a

    def ffn(p, xn, conv):
        if conv:
            h = _silu(_conv(xn, get(p + ".w1.weight", (F, H, 3)), None, 1)) * _conv(xn, get(p + ".w3.weight", (F, H, 3)), None, 1)
            return _conv(h, get(p + ".w2.weight", (H, F, 3)), None, 1)
        h = _silu(xn @ get(p + ".w1.weight", (F, H)).T) * (xn @ get(p + ".w3.weight", (F, H)).T)
        return h @ get(p + ".w2.weight", (H, F)).T

    def pre(p, xs, mod, fscale):
        xn = _ln(xs, eps) * (1 + mod[..., H:2 * H]) + mod[..., :H]
        qkv = xn @ get(p + ".attn.qkv.weight", (3 * H, H)).T + get(p + ".attn.qkv.bias")
        qkv = np.concatenate([qkv[:, 0::3], qkv[:, 1::3], qkv[:, 2::3]], 1)   # interleaved rows 3c + j
        out = []
        for c, nm in ((0, "q_norm"), (H, "k_norm")):
            hh = qkv[:, c:c + H].reshape(len(xs), NH, -1)
            hh = (hh / np.sqrt((hh ** 2).mean(-1, keepdims=True) + reps) * get(p + ".attn." + nm + ".weight")).reshape(len(xs), H)
            out.append(_rope(hh, NH, theta, fscale) if fscale else hh)
        return out[0], out[1], qkv[:, 2 * H:]

    def post(p, xs, a, mod, conv):
        o = _conv(a, get(p + ".linear1.weight", (H, H, 3)), get(p + ".linear1.bias"), 1) if conv else \
            a @ get(p + ".linear1.weight", (H, H)).T + get(p + ".linear1.bias")
        xs = xs + o * mod[..., 2 * H:3 * H]
        xn = _ln(xs, eps) * (1 + mod[..., 4 * H:5 * H]) + mod[..., 3 * H:4 * H]
        return xs + ffn(p + ".ffn", xn, conv) * mod[..., 5 * H:6 * H]

    B = x.shape[0]
    v = np.empty((B, T, L))
    taps = []
    D = H
    fr = (1e4 / spec["t_max_period"]) * 1e4 ** (-2.0 * np.arange(D // 2) / D)
    for b in range(B):
        emb = np.concatenate([np.cos(t[b] * fr), np.sin(t[b] * fr)])
        te = get("t_embed.mlp.2.weight", (H, H)) @ _silu(get("t_embed.mlp.0.weight", (H, H)) @ emb + get("t_embed.mlp.0.bias")) + get("t_embed.mlp.2.bias")
        gc = gcmlp[b] + te
        extc = _silu(sync_gather[b] + gc)
        gs = _silu(gc)
        xin = _silu(_conv(x[b], get("audio_input_proj.0.weight", (H, L, 3)), get("audio_input_proj.0.bias"), 1))
        lat, clip, text = ffn("audio_input_proj.2", xin, True), clip_pp[b].astype(np.float64), text_pp[b].astype(np.float64)
        bt = []
        for i in range(spec["n_joint"]):
            pre_only = i == spec["n_joint"] - 1
            cc = 2 if pre_only else 6
            p = "joint_blocks.%d" % i
            ml = extc @ get(p + ".latent_block.adaLN_modulation.1.weight", (6 * H, H)).T + get(p + ".latent_block.adaLN_modulation.1.bias")
            mc = get(p + ".clip_block.adaLN_modulation.1.weight", (cc * H, H)) @ gs + get(p + ".clip_block.adaLN_modulation.1.bias")
            mt = get(p + ".text_block.adaLN_modulation.1.weight", (cc * H, H)) @ gs + get(p + ".text_block.adaLN_modulation.1.bias")
            parts = [pre(p + ".latent_block", lat, ml, 1.0), pre(p + ".clip_block", clip, mc, T / C),
                     pre(p + ".text_block", text, mt, 0.0)]
            A = _attn(*(np.concatenate([pp[j] for pp in parts]) for j in range(3)), NH)
            lat = post(p + ".latent_block", lat, A[:T], ml, True)
            if not pre_only:
                clip = post(p + ".clip_block", clip, A[T:T + C], mc, True)
                text = post(p + ".text_block", text, A[T + C:], mt, False)
            bt.append(np.concatenate([lat, clip, text]))
        for i in range(spec["n_fused"]):
            p = "fused_blocks.%d" % i
            ml = extc @ get(p + ".adaLN_modulation.1.weight", (6 * H, H)).T + get(p + ".adaLN_modulation.1.bias")
            q, k, vv = pre(p, lat, ml, 1.0)
            lat = post(p, lat, _attn(q, k, vv, NH), ml, True)
            bt.append(np.concatenate([lat, clip, text]))
        mf = extc @ get("final_layer.adaLN_modulation.1.weight", (2 * H, H)).T + get("final_layer.adaLN_modulation.1.bias")
        xn = _ln(lat, eps) * (1 + mf[:, H:]) + mf[:, :H]
        v[b] = _conv(xn, get("final_layer.conv.weight", (L, H, 7)), get("final_layer.conv.bias"), 3)
        taps.append(bt)
    return v, np.array(taps).transpose(1, 0, 2, 3)


# ---------------- tests ----------------
def test_ref_forward_vs_numpy(orc):
    spec = tiny_ref_spec()
    w, idx = ref_weights(orc, spec)
    inp = ref_inputs(spec)
    v, taps = orc.ref_dit_forward(spec, w, taps=True, **inp)
    vr, tr = np_ref_forward(spec, w, idx, **inp)
    # f32 against float64: about 1e-5 after the conv SwiGLU input projection and three blocks
    assert rel_l2(v, vr) < 3e-5
    for i in range(taps.shape[0]):
        assert rel_l2(taps[i], tr[i]) < 3e-5


def test_ref_structure(orc):
    spec = tiny_ref_spec()
    w, _ = ref_weights(orc, spec)
    inp = ref_inputs(spec)
    _, taps = orc.ref_dit_forward(spec, w, taps=True, **inp)
    T = spec["T"]
    # the last joint block (pre-only) and the fused block leave clip and text rows unchanged
    nj = spec["n_joint"]
    assert np.array_equal(taps[nj - 1][:, T:], taps[nj - 2][:, T:])
    assert np.array_equal(taps[nj][:, T:], taps[nj - 1][:, T:])
    # earlier joint blocks do update them
    assert not np.array_equal(taps[0][:, T:], np.concatenate([inp["clip_pp"], inp["text_pp"]], 1))
    # samples do not mix
    s1 = dict(spec, B=1)
    one = {k: np.ascontiguousarray(a[1:]) for k, a in inp.items()}
    v1 = orc.ref_dit_forward(s1, w, **one)
    v2 = orc.ref_dit_forward(spec, w, **inp)
    assert np.array_equal(v1[0], v2[1])


def test_ref_sampler_closed_form(orc):
    spec = tiny_ref_spec()
    w, idx = ref_weights(orc, spec)
    o, n = idx["final_layer.conv.weight"]
    w[o:o + n] = 0.0
    ob, nb = idx["final_layer.conv.bias"]
    bias = np.linspace(-1, 1, nb).astype(np.float32)
    w[ob:ob + nb] = bias
    inp = ref_inputs(spec)
    x0 = inp["x"][:1]
    x = orc.ref_dit_sample(spec, w, x0, inp["clip_pp"], inp["text_pp"], inp["gcmlp"], inp["sync_gather"], 4, 5.0)
    assert np.allclose(x, x0 - bias, atol=1e-6)


# ---------------- conditioning prep (oracle/oracle_cond.cpp) ----------------
def tiny_cond_spec():
    return dict(H=128, F=64, T=10, C=4, sync_S=12, TS=5, sync_dim=64, clip_dim=96, text_dim=160, gtext_dim=32)


def cond_weights(orc, spec, seed=3):
    man = orc.cond_manifest(spec)
    r = rng(seed)
    w = (0.05 * r.standard_normal(sum(n for _, n, _ in man))).astype(np.float32)
    return w, {name: (off, n) for name, n, off in man}


def np_prep(spec, w, idx, clip_f, sync_f, text_cat, gtext):
    """float64 restatement of src/dit.cpp:55-191 written from the reference's steps"""
    H, F = spec["H"], spec["F"]

    def get(n, shape):
        o, k = idx[n]
        return w[o:o + k].astype(np.float64).reshape(shape)

    def convmlp(p, x):
        h = _silu(_conv(x, get(p + ".w1.weight", (F, H, 3)), None, 1)) * _conv(x, get(p + ".w3.weight", (F, H, 3)), None, 1)
        return _conv(h, get(p + ".w2.weight", (H, F, 3)), None, 1)

    def mlp(p, x):
        h = _silu(x @ get(p + ".w1.weight", (F, H)).T) * (x @ get(p + ".w3.weight", (F, H)).T)
        return h @ get(p + ".w2.weight", (H, F)).T

    SS, T = spec["sync_S"], spec["T"]
    pe = get("sync_pos_emb", (8, spec["sync_dim"]))
    sb = sync_f.astype(np.float64) + pe[np.arange(SS) % 8]
    smid = convmlp("sync_input_proj.2", _silu(_conv(sb, get("sync_input_proj.0.weight", (H, spec["sync_dim"], 7)),
                                                    get("sync_input_proj.0.bias", (H,)), 3)))
    f = np.float32   # the row index is computed in f32: floorf(((float)i + 0.5f) * (float)S / (float)T)
    rows = [int(np.floor((f(i) + f(0.5)) * f(SS) / f(T))) for i in range(T)]
    sync_gather = smid[rows]
    clip = _silu(clip_f.astype(np.float64) @ get("clip_input_proj.0.weight", (H, spec["clip_dim"])).T
                 + get("clip_input_proj.0.bias", (H,)))
    clip_pp = convmlp("clip_input_proj.2", clip)
    clip_fc = get("clip_cond_proj.weight", (H, H)) @ clip_pp.mean(0) + get("clip_cond_proj.bias", (H,))
    text = _silu(text_cat.astype(np.float64) @ get("text_input_proj.0.weight", (H, spec["text_dim"])).T
                 + get("text_input_proj.0.bias", (H,)))
    text_pp = mlp("text_input_proj.2", text)
    fc = get("text_cond_proj.weight", (H, spec["gtext_dim"])) @ gtext.astype(np.float64) + \
        get("text_cond_proj.bias", (H,)) + clip_fc
    gcmlp = mlp("global_cond_mlp", fc[None, :])[0]
    return clip_pp, sync_gather, clip_fc, text_pp, gcmlp, rows


def test_cond_prep_vs_numpy(orc):
    spec = tiny_cond_spec()
    w, idx = cond_weights(orc, spec)
    r = rng(4)
    clip_f = r.standard_normal((spec["C"], spec["clip_dim"])).astype(np.float32)
    sync_f = r.standard_normal((spec["sync_S"], spec["sync_dim"])).astype(np.float32)
    text_cat = r.standard_normal((spec["TS"], spec["text_dim"])).astype(np.float32)
    gtext = r.standard_normal(spec["gtext_dim"]).astype(np.float32)
    clip_pp, sg, clip_fc = orc.ref_prep_conditioning(spec, w, clip_f, sync_f)
    text_pp, gcmlp = orc.ref_prep_text_arm(spec, w, text_cat, gtext, clip_fc)
    e = np_prep(spec, w, idx, clip_f, sync_f, text_cat, gtext)
    for got, ref in zip((clip_pp, sg, clip_fc, text_pp, gcmlp), e[:5]):
        assert rel_l2(got, ref) < 1e-5
    # the gather picks rows floor((i + 0.5) * sync_S / T): for 12 -> 10 rows that is row 0, 1, 3, ...
    assert e[5] == [0, 1, 3, 4, 5, 6, 7, 9, 10, 11]
    # upsampling (sync_S < T) repeats rows: 12 -> 20 takes each sync row for 5/3 latent rows
    up = dict(spec, T=20)
    _, sg_up, _ = orc.ref_prep_conditioning(up, w, clip_f, sync_f)
    assert np.array_equal(sg_up[0], sg_up[1]) and not np.array_equal(sg_up[1], sg_up[2])
