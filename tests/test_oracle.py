"""Pinning of the CPU oracle (oracle/) — CPU only.

Each oracle function is checked against something other than its own formula:
  * brute force in float64 with numpy primitives (matmul, explicit conv loops, softmax),
  * closed forms and special cases (q = 0 attention is the mean of V, pos 0 RoPE is the identity,
    t = 0 timestep embedding is [1.., 0..]),
  * invariants (LayerNorm rows have mean 0 / variance var/(var+eps); RMS of a unit-weight head is
    ~1; RoPE preserves pair norms and makes <R(m)q, R(n)k> depend on m - n only),
  * structural identities of the block graph (zero gates make a block the identity; a model whose
    output layer is zero has a constant velocity, which the sampler integrates in closed form).
A plausible slip — a transposed operand, a shifted conv tap, a wrong chunk index, a missing
residual — fails at least one of them.
"""
import numpy as np
import pytest

from conftest import rel_l2, rng


def test_gemm_brute_force(orc):
    r = rng(1)
    for (M, N, K) in [(1, 1, 1), (3, 5, 7), (65, 130, 257), (128, 64, 1024)]:
        X = r.standard_normal((M, K)).astype(np.float32)
        W = r.standard_normal((N, K)).astype(np.float32)
        b = r.standard_normal(N).astype(np.float32)
        ref = X.astype(np.float64) @ W.T.astype(np.float64) + b
        assert rel_l2(orc.gemm(W, X, b), ref) < 1e-6
        assert rel_l2(orc.gemm(W, X), X.astype(np.float64) @ W.T.astype(np.float64)) < 1e-6


def test_gemm_not_transposed(orc):
    # Y = X W^T, not X W: a rectangular W only fits one way round
    X = np.eye(2, 3, dtype=np.float32)
    W = np.arange(12, dtype=np.float32).reshape(4, 3)
    Y = orc.gemm(W, X)
    assert Y.shape == (2, 4)
    assert np.array_equal(Y, X @ W.T)


def test_gemv(orc):
    r = rng(2)
    W = r.standard_normal((300, 200)).astype(np.float32)
    x = r.standard_normal(200).astype(np.float32)
    b = r.standard_normal(300).astype(np.float32)
    assert rel_l2(orc.gemv(W, x, b), W.astype(np.float64) @ x + b) < 1e-6


def _conv_brute(W, b, x, stride, pad, dil):
    OC, IC, K = W.shape
    T = x.shape[0]
    OL = (T + 2 * pad - dil * (K - 1) - 1) // stride + 1
    y = np.zeros((OL, OC))
    for t in range(OL):
        for k in range(K):
            ti = t * stride - pad + k * dil
            if 0 <= ti < T:
                y[t] += W[:, :, k].astype(np.float64) @ x[ti].astype(np.float64)
    return y + (b if b is not None else 0)


@pytest.mark.parametrize("K,pad,stride,dil", [(3, 1, 1, 1), (7, 3, 1, 1), (1, 0, 1, 1), (3, 1, 2, 1), (3, 2, 1, 2), (3, 0, 1, 1)])
def test_conv1d(orc, K, pad, stride, dil):
    r = rng(3 + K)
    W = r.standard_normal((6, 5, K)).astype(np.float32)
    x = r.standard_normal((11, 5)).astype(np.float32)
    b = r.standard_normal(6).astype(np.float32)
    ref = _conv_brute(W, b, x, stride, pad, dil)
    assert rel_l2(orc.conv1d(W, b, x, pad, stride, dil), ref) < 1e-6
    assert rel_l2(orc.conv1d(W, b, x, pad, stride, dil, direct=True), ref) < 1e-6


def test_conv1d_taps_are_causal_order(orc):
    # impulse response: x = delta at t0 -> y[t, oc] = W[oc, ic, t0 - t + pad] (tap k reads row t - pad + k)
    W = np.arange(2 * 1 * 3, dtype=np.float32).reshape(2, 1, 3) + 1
    x = np.zeros((5, 1), np.float32)
    x[2, 0] = 1.0
    y = orc.conv1d(W, None, x, 1)
    for t in range(5):
        for oc in range(2):
            k = 2 - t + 1
            assert y[t, oc] == (W[oc, 0, k] if 0 <= k < 3 else 0.0)


@pytest.mark.parametrize("per_row,chunks,base", [(0, 6, 0), (0, 6, 3 * 64), (1, 2, 0)])
def test_adaln_ln(orc, per_row, chunks, base):
    r = rng(4)
    rows, H, eps = 9, 64, 1e-5
    x = (r.standard_normal((rows, H)) * 3 + 2).astype(np.float32)
    mod = r.standard_normal((rows if per_row else 1, chunks * H)).astype(np.float32)
    y = orc.adaln_ln(x, mod, per_row, chunks, base, eps)
    x64 = x.astype(np.float64)
    mu = x64.mean(1, keepdims=True)
    var = x64.var(1, keepdims=True)          # biased
    ln = (x64 - mu) / np.sqrt(var + eps)
    m = mod if per_row else np.repeat(mod, rows, 0)
    ref = ln * (1 + m[:, base + H:base + 2 * H]) + m[:, base:base + H]
    assert rel_l2(y, ref) < 1e-6
    # invariant: with zero modulation each row has mean 0 and variance var/(var+eps)
    y0 = orc.adaln_ln(x, np.zeros_like(mod), per_row, chunks, base, eps).astype(np.float64)
    assert np.abs(y0.mean(1)).max() < 1e-6
    assert np.allclose(y0.var(1), (var / (var + eps)).ravel(), rtol=1e-5)


def test_gate_add(orc):
    r = rng(5)
    x, f = r.standard_normal((4, 8)).astype(np.float32), r.standard_normal((4, 8)).astype(np.float32)
    mod = r.standard_normal((4, 48)).astype(np.float32)
    assert np.allclose(orc.gate_add(x, f, mod, 1, 6, 2), x + f * mod[:, 16:24], rtol=1e-6)
    assert np.allclose(orc.gate_add(x, f, mod[:1], 0, 6, 5), x + f * mod[0, 40:48], rtol=1e-6)


def test_rms_head(orc):
    r = rng(6)
    rows, nh, hd, ld = 5, 3, 64, 3 * 3 * 64
    x = r.standard_normal((rows + 2, ld)).astype(np.float32)
    w = np.ones(hd, np.float32)
    y = orc.rms_head(x, w, rows, nh, ld, hd, 64 * 3, 1)
    sl = y[1:1 + rows, 192:192 + nh * hd].reshape(rows, nh, hd)
    ms = (x[1:1 + rows, 192:192 + nh * hd].reshape(rows, nh, hd).astype(np.float64) ** 2).mean(-1)
    assert np.allclose((sl.astype(np.float64) ** 2).mean(-1), ms / (ms + 1e-6), rtol=1e-5)   # RMS ~ 1
    # untouched outside the slice
    assert np.array_equal(y[0], x[0]) and np.array_equal(y[1:1 + rows, :192], x[1:1 + rows, :192])
    w2 = r.standard_normal(hd).astype(np.float32)
    y2 = orc.rms_head(x, w2, rows, nh, ld, hd, 192, 1)
    src = x[1:1 + rows, 192:192 + nh * hd].reshape(rows, nh, hd).astype(np.float64)
    ref = src / np.sqrt((src ** 2).mean(-1, keepdims=True) + 1e-6) * w2
    assert rel_l2(y2[1:1 + rows, 192:192 + nh * hd].reshape(rows, nh, hd), ref) < 1e-6


def test_rope_pairs(orc):
    r = rng(7)
    rows, nh, hd, ld = 16, 2, 64, 128
    x = r.standard_normal((rows, ld)).astype(np.float32)
    y = orc.rope_pairs(x, None, rows, nh, ld, hd, 0, 0)
    # pos 0 is the identity; pair norms are preserved
    assert np.allclose(y[0], x[0], atol=1e-7)
    n_in = x.reshape(rows, -1, 2) ** 2
    n_out = y.reshape(rows, -1, 2) ** 2
    assert np.allclose(n_in.sum(-1), n_out.sum(-1), rtol=1e-5)
    # complex-number form: (x0 + i x1) * exp(i * pos * base^(-2j/hd))
    j = np.arange(hd // 2)
    inv = 10000.0 ** (-2.0 * j / hd)
    z = x.reshape(rows, nh, hd // 2, 2)
    zc = z[..., 0] + 1j * z[..., 1]
    ang = np.arange(rows)[:, None, None] * inv[None, None, :]
    ref = zc * np.exp(1j * ang)
    out = y.reshape(rows, nh, hd // 2, 2)
    assert rel_l2(out[..., 0] + 1j * out[..., 1], ref) < 2e-6
    # relative position: <R(m)q, R(n)k> depends on m - n only
    q, k = r.standard_normal(hd).astype(np.float32), r.standard_normal(hd).astype(np.float32)
    def rot(v, pos):
        buf = np.zeros((pos + 1, hd), np.float32)
        buf[pos] = v
        return orc.rope_pairs(buf, None, pos + 1, 1, hd, hd, 0, 0)[pos].astype(np.float64)
    assert abs(rot(q, 5) @ rot(k, 2) - rot(q, 9) @ rot(k, 6)) < 1e-4
    # explicit positions and fscale: pos p with fscale s equals pos p*s when p*s is an integer
    pos = np.array([3, 1, 4], np.int32)
    ya = orc.rope_pairs(x[:3], pos, 3, nh, ld, hd, 0, 0, fscale=2.0)
    yb = orc.rope_pairs(np.stack([x[0]] * 7)[:7], None, 7, nh, ld, hd, 0, 0)
    assert np.allclose(ya[0], yb[6], atol=2e-6)


def _attn_ref(qkv, S, nh, hd, H, scale):
    q = qkv[:, :H].reshape(S, nh, hd).astype(np.float64)
    k = qkv[:, H:2 * H].reshape(S, nh, hd).astype(np.float64)
    v = qkv[:, 2 * H:].reshape(S, nh, hd).astype(np.float64)
    s = np.einsum("qhd,khd->hqk", q, k) * scale
    s -= s.max(-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(-1, keepdims=True)
    return np.einsum("hqk,khd->qhd", p, v).reshape(S, H)


def test_attention(orc):
    r = rng(8)
    S, nh, hd = 37, 2, 64
    H = nh * hd
    qkv = r.standard_normal((S, 3 * H)).astype(np.float32)
    out = orc.attention(qkv, S, nh, hd, 3 * H, H, 0, H, 2 * H, 0, 0.125)
    assert rel_l2(out, _attn_ref(qkv, S, nh, hd, H, 0.125)) < 1e-5
    # q = 0: uniform weights -> every row is the mean of V
    z = qkv.copy()
    z[:, :H] = 0
    out0 = orc.attention(z, S, nh, hd, 3 * H, H, 0, H, 2 * H, 0, 0.125)
    assert np.allclose(out0, np.broadcast_to(qkv[:, 2 * H:].mean(0), (S, H)), atol=1e-5)
    # one key with a huge logit selects its V row
    q1 = np.zeros_like(qkv)
    q1[:, :H] = 1.0
    q1[7, H:2 * H] = 50.0
    q1[:, 2 * H:] = qkv[:, 2 * H:]
    out1 = orc.attention(q1, S, nh, hd, 3 * H, H, 0, H, 2 * H, 0, 0.125)
    assert np.allclose(out1, np.broadcast_to(qkv[7, 2 * H:], (S, H)), atol=1e-5)


def test_elementwise(orc):
    r = rng(9)
    a, b, c = (r.standard_normal(1000).astype(np.float32) for _ in range(3))
    a64 = a.astype(np.float64)
    assert np.allclose(orc.silu(a), a64 / (1 + np.exp(-a64)), rtol=1e-6, atol=1e-7)
    assert np.allclose(orc.swiglu(a, b), a64 / (1 + np.exp(-a64)) * b, rtol=1e-6, atol=1e-7)
    assert np.array_equal(orc.add(a, b), a + b)
    assert np.allclose(orc.cfg_euler(a, b, c, 5.0, -0.25), c - 0.25 * (b + 5.0 * (a - b)), rtol=1e-6, atol=1e-6)
    X = r.standard_normal((10, 16)).astype(np.float32)
    v = r.standard_normal(16).astype(np.float32)
    assert np.array_equal(orc.add_bcast_col(X, v), X + v)


def test_timestep_embedding(orc):
    e0 = orc.timestep_embedding(0.0, 256)
    assert np.array_equal(e0[:128], np.ones(128, np.float32)) and np.array_equal(e0[128:], np.zeros(128, np.float32))
    t = 0.37
    k = np.arange(128)
    fr = 10000.0 * 10000.0 ** (-2.0 * k / 256)
    ref = np.concatenate([np.cos(t * fr), np.sin(t * fr)])
    # f32 argument t*fr reaches 3.7e3 rad: compare at the f32 argument rounding level
    assert np.abs(orc.timestep_embedding(t, 256) - ref).max() < 2e-3


# ---------------- block graph ----------------
def tiny_spec(B=2, La=12, Lt=5, n_joint=1, n_fused=1):
    return dict(B=B, La=La, Lt=Lt, H=128, NH=2, HD=64, F=256, latent=8, temb_dim=16, n_joint=n_joint,
                n_fused=n_fused, audio_ffn_conv=1, rope_theta=10000.0, t_max_period=1.0, ln_eps=1e-5, rms_eps=1e-6)


def tiny_weights(orc, spec, seed=0, norm_mean=1.0):
    man = orc.manifest(spec)
    r = rng(seed)
    w = np.empty(sum(n for _, n, _ in man), np.float32)
    for name, n, off in man:
        mean = norm_mean if "norm.weight" in name else 0.0
        w[off:off + n] = (mean + 0.05 * r.standard_normal(n)).astype(np.float32)
    return w, {name: (off, n) for name, n, off in man}


def _silu(x):
    return x / (1 + np.exp(-x))


def _np_block(spec, w, idx, prefix_streams, X, g, fused):
    """float64 numpy restatement of one block, written from the reference dit_fwd.cpp op order."""
    H, NH, HD, F, La, Lt = spec["H"], spec["NH"], spec["HD"], spec["F"], spec["La"], spec["Lt"]
    S = La + Lt
    get = lambda n: w[idx[n][0]:idx[n][0] + idx[n][1]].astype(np.float64)
    gs = _silu(g.astype(np.float64))
    out = X.astype(np.float64).copy()
    for b in range(spec["B"]):
        qkv_rows, mods, segs = [], [], []
        for (p, lo, L, rope, conv) in prefix_streams:
            mod = get(p + ".adaLN_modulation.1.weight").reshape(6 * H, H) @ gs[b] + get(p + ".adaLN_modulation.1.bias")
            x = out[b, lo:lo + L]
            ln = (x - x.mean(1, keepdims=True)) / np.sqrt(x.var(1, keepdims=True) + 1e-5)
            xn = ln * (1 + mod[H:2 * H]) + mod[:H]
            qkv = xn @ get(p + ".attn.qkv.weight").reshape(3 * H, H).T + get(p + ".attn.qkv.bias")
            for c, nm in ((0, "q_norm"), (H, "k_norm")):
                hh = qkv[:, c:c + H].reshape(L, NH, HD)
                hh = hh / np.sqrt((hh ** 2).mean(-1, keepdims=True) + 1e-6) * get(p + ".attn." + nm + ".weight")
                if rope:
                    j = np.arange(HD // 2)
                    ang = np.arange(L)[:, None, None] * (10000.0 ** (-2.0 * j / HD))[None, None, :]
                    zc = (hh[..., 0::2] + 1j * hh[..., 1::2]) * np.exp(1j * ang)
                    hh = np.stack([zc.real, zc.imag], -1).reshape(L, NH, HD)
                qkv[:, c:c + H] = hh.reshape(L, H)
            qkv_rows.append(qkv)
            mods.append(mod)
            segs.append((p, lo, L, conv))
        J = np.concatenate(qkv_rows, 0)
        A = _attn_ref(J, J.shape[0], NH, HD, H, 1 / 8)
        row = 0
        for (p, lo, L, conv), mod in zip(segs, mods):
            x = out[b, lo:lo + L]
            o = A[row:row + L] @ get(p + ".linear1.weight").reshape(H, H).T + get(p + ".linear1.bias")
            row += L
            x = x + o * mod[2 * H:3 * H]
            ln = (x - x.mean(1, keepdims=True)) / np.sqrt(x.var(1, keepdims=True) + 1e-5)
            xn = ln * (1 + mod[4 * H:5 * H]) + mod[3 * H:4 * H]
            if conv:
                h = _silu(_conv_brute(get(p + ".ffn.w1.weight").reshape(F, H, 3), None, xn, 1, 1, 1))
                f = _conv_brute(get(p + ".ffn.w2.weight").reshape(H, F, 3), None, h, 1, 1, 1)
            else:
                h = _silu(xn @ get(p + ".ffn.w1.weight").reshape(F, H).T)
                f = h @ get(p + ".ffn.w2.weight").reshape(H, F).T
            out[b, lo:lo + L] = x + f * mod[5 * H:6 * H]
    return out


def test_joint_and_fused_block_vs_numpy(orc):
    spec = tiny_spec()
    w, idx = tiny_weights(orc, spec)
    r = rng(10)
    S = spec["La"] + spec["Lt"]
    X = r.standard_normal((2, S, 128)).astype(np.float32)
    g = r.standard_normal((2, 128)).astype(np.float32)
    ref = _np_block(spec, w, idx, [("joint_blocks.0.latent_block", 0, spec["La"], True, True),
                                   ("joint_blocks.0.text_block", spec["La"], spec["Lt"], False, False)], X, g, False)
    assert rel_l2(orc.joint_block(spec, w, 0, X, g), ref) < 1e-5
    # fused: one weight set over all S rows, RoPE on the audio rows only
    fused = _np_block_fused(spec, w, idx, X, g)
    assert rel_l2(orc.fused_block(spec, w, 0, X, g), fused) < 1e-5


def _np_block_fused(spec, w, idx, X, g):
    # RoPE on the first La rows only: run the generic block with one stream over S rows, then undo
    # RoPE on the text rows by building q/k with rope only for rows < La. Implemented directly:
    H, NH, HD, F, La, Lt = spec["H"], spec["NH"], spec["HD"], spec["F"], spec["La"], spec["Lt"]
    S = La + Lt
    p = "fused_blocks.0"
    get = lambda n: w[idx[n][0]:idx[n][0] + idx[n][1]].astype(np.float64)
    out = X.astype(np.float64).copy()
    gs = _silu(g.astype(np.float64))
    for b in range(spec["B"]):
        mod = get(p + ".adaLN_modulation.1.weight").reshape(6 * H, H) @ gs[b] + get(p + ".adaLN_modulation.1.bias")
        x = out[b]
        ln = (x - x.mean(1, keepdims=True)) / np.sqrt(x.var(1, keepdims=True) + 1e-5)
        qkv = (ln * (1 + mod[H:2 * H]) + mod[:H]) @ get(p + ".attn.qkv.weight").reshape(3 * H, H).T + get(p + ".attn.qkv.bias")
        for c, nm in ((0, "q_norm"), (H, "k_norm")):
            hh = qkv[:, c:c + H].reshape(S, NH, HD)
            hh = hh / np.sqrt((hh ** 2).mean(-1, keepdims=True) + 1e-6) * get(p + ".attn." + nm + ".weight")
            j = np.arange(HD // 2)
            ang = np.arange(S)[:, None, None] * (10000.0 ** (-2.0 * j / HD))[None, None, :]
            ang[La:] = 0.0
            zc = (hh[..., 0::2] + 1j * hh[..., 1::2]) * np.exp(1j * ang)
            qkv[:, c:c + H] = np.stack([zc.real, zc.imag], -1).reshape(S, H)
        A = _attn_ref(qkv, S, NH, HD, H, 1 / 8)
        x = x + (A @ get(p + ".linear1.weight").reshape(H, H).T + get(p + ".linear1.bias")) * mod[2 * H:3 * H]
        ln = (x - x.mean(1, keepdims=True)) / np.sqrt(x.var(1, keepdims=True) + 1e-5)
        h = _silu((ln * (1 + mod[4 * H:5 * H]) + mod[3 * H:4 * H]) @ get(p + ".ffn.w1.weight").reshape(F, H).T)
        out[b] = x + (h @ get(p + ".ffn.w2.weight").reshape(H, F).T) * mod[5 * H:6 * H]
    return out


def test_zero_gates_make_blocks_identity(orc):
    spec = tiny_spec()
    w, idx = tiny_weights(orc, spec)
    H = spec["H"]
    for p in ("joint_blocks.0.latent_block", "joint_blocks.0.text_block", "fused_blocks.0"):
        ow, _ = idx[p + ".adaLN_modulation.1.weight"]
        ob, _ = idx[p + ".adaLN_modulation.1.bias"]
        for gate in (2, 5):
            w[ow + gate * H * H: ow + (gate + 1) * H * H] = 0.0
            w[ob + gate * H: ob + (gate + 1) * H] = 0.0
    r = rng(11)
    X = r.standard_normal((2, spec["La"] + spec["Lt"], H)).astype(np.float32)
    g = r.standard_normal((2, H)).astype(np.float32)
    assert np.array_equal(orc.joint_block(spec, w, 0, X, g), X)
    assert np.array_equal(orc.fused_block(spec, w, 0, X, g), X)


def test_forward_and_sampler_closed_form(orc):
    spec = tiny_spec(B=2, n_joint=1, n_fused=1)
    w, idx = tiny_weights(orc, spec)
    lat = spec["latent"]
    ow, n = idx["final_layer.linear.weight"]
    w[ow:ow + n] = 0.0
    ob, nb = idx["final_layer.linear.bias"]
    bias = np.linspace(-1, 1, nb).astype(np.float32)
    w[ob:ob + nb] = bias
    r = rng(12)
    z = r.standard_normal((2, spec["La"], lat)).astype(np.float32)
    text = r.standard_normal((2, spec["Lt"], 128)).astype(np.float32)
    pooled = r.standard_normal((2, 128)).astype(np.float32)
    v = orc.dit_forward(spec, w, z, np.array([0.3, 0.3], np.float32), text, pooled)
    assert np.array_equal(v, np.broadcast_to(bias, v.shape))          # zero output layer: v = bias
    x0 = z[:1]
    x = orc.dit_sample(spec, w, x0, text, pooled, 4, 5.0)
    # constant velocity b in both arms: x_T = x0 + sum(dt) * b = x0 - b
    assert np.allclose(x, x0 - bias, atol=1e-6)


def test_forward_taps_and_batch_independence(orc):
    spec = tiny_spec(B=2)
    w, _ = tiny_weights(orc, spec)
    r = rng(13)
    S = spec["La"] + spec["Lt"]
    z = r.standard_normal((2, spec["La"], 8)).astype(np.float32)
    text = r.standard_normal((2, spec["Lt"], 128)).astype(np.float32)
    pooled = r.standard_normal((2, 128)).astype(np.float32)
    t = np.array([0.2, 0.9], np.float32)
    v, taps, gs = orc.dit_forward(spec, w, z, t, text, pooled, taps=True)
    assert taps.shape == (2, 2, S, 128)
    # sample 1 computed alone equals sample 1 of the batch (no cross-sample mixing)
    s1 = dict(spec, B=1)
    v1 = orc.dit_forward(s1, w, z[1:], t[1:], text[1:], pooled[1:])
    assert rel_l2(v1, v[1:]) < 1e-6
    # the last tap feeds the final layer: re-running the final layer on it reproduces v
    H = 128
    wf, idx = tiny_weights(orc, spec)
    def get(n):
        o, k = idx[n]
        return wf[o:o + k].astype(np.float64)
    for b in range(2):
        mod = get("final_layer.adaLN_modulation.1.weight").reshape(2 * H, H) @ gs[b] + get("final_layer.adaLN_modulation.1.bias")
        x = taps[-1, b, :spec["La"]].astype(np.float64)
        ln = (x - x.mean(1, keepdims=True)) / np.sqrt(x.var(1, keepdims=True) + 1e-5)
        ref = (ln * (1 + mod[H:]) + mod[:H]) @ get("final_layer.linear.weight").reshape(8, H).T + get("final_layer.linear.bias")
        assert rel_l2(v[b], ref) < 1e-5


def test_launcher_surface_ops(orc):
    """The rest of the net.h surface, each against an independent library routine or a known answer:
    geglu against torch's tanh-GELU (the clamp at |arg| = 10 changes tanh by < 5e-9), gelu_quick
    against x·sigmoid(1.702 x), ln_plain against torch's layer_norm without affine (biased variance),
    mean_cols against a float64 mean, and qkv_split3 on values that encode their own (row, channel,
    part): a swapped part or a shifted channel is visible element by element."""
    import torch
    r = rng(41)
    a = (3.0 * r.standard_normal(4099)).astype(np.float32)
    a[:3] = [30.0, -30.0, 0.0]                               # deep in the clamp, and zero
    b = r.standard_normal(4099).astype(np.float32)
    ta = torch.from_numpy(a.astype(np.float64))
    ref = torch.nn.functional.gelu(ta, approximate="tanh").numpy() * b
    assert rel_l2(orc.geglu(a, b), ref) < 1e-6
    assert rel_l2(orc.gelu_quick(a), (ta * torch.sigmoid(1.702 * ta)).numpy()) < 1e-6
    x = (2.0 + r.standard_normal((37, 1000))).astype(np.float32)
    ln = torch.nn.functional.layer_norm(torch.from_numpy(x.astype(np.float64)), (1000,), eps=1e-5).numpy()
    assert rel_l2(orc.ln_plain(x, 1e-5), ln) < 1e-6
    assert rel_l2(orc.mean_cols(x), x.astype(np.float64).mean(axis=0)) < 1e-6
    rows, H, off = 5, 6, 2
    src = np.zeros((rows, 3 * H), np.float32)
    for rr in range(rows):
        for c in range(H):
            for j in range(3):
                src[rr, 3 * c + j] = 1000 * rr + 10 * c + j
    out = orc.qkv_split3(src, np.full((rows + 4, 3 * H), -1.0, np.float32), off)
    assert (out[:off] == -1).all() and (out[off + rows:] == -1).all()
    for j in range(3):
        assert np.array_equal(out[off:off + rows, j * H:(j + 1) * H],
                              1000 * np.arange(rows)[:, None] + 10 * np.arange(H)[None, :] + j)
