"""Pinning of the oracle's VAE decoder restatement (oracle/oracle_vae.cpp) — CPU only.

Checked against:
  * snake (shaders/ops_conv.metal:204-213) through its invariants: |y - x| <= exp(-beta) with
    equality where x*exp(alpha) = pi/2, y = x where x*exp(alpha) is a multiple of pi, and y - x
    periodic in x with period pi*exp(-alpha) — a wrong sign on beta, a missing exp on alpha or sin
    instead of sin^2 fails one of them;
  * the transposed conv in the reference's gather form (src/net.mm:36-48) against PyTorch's
    conv_transpose1d in float64, with the reference's kernel being the flipped, transposed
    PyTorch weight and pad = K - 1 - padding (a library routine of the textbook scatter
    definition y[i*s - p + k] += x[i] W[k]), and against that scatter written out in NumPy;
  * dilated convs (the residual units' k7, dilation 1/3/9, pad 3*dil) against PyTorch conv1d;
  * the whole decode (src/vae.cpp:17-86) on small widths against a float64 composition of PyTorch's
    conv1d / conv_transpose1d and NumPy, following the reference's layer order;
  * the output length T * prod(stride) and the manifest's structure.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as Fn

from conftest import rel_l2, rng


def small_spec(T=3):
    return dict(T=T, latent=64, width=[128, 64, 64, 64, 64, 64], stride=[2, 4, 2, 2, 2], kt=[4, 8, 4, 4, 4],
                out_ch=2)


def vae_weights(orc, spec, seed=0):
    """conv weights N(0, 1/fan_in) (residual-branch k1 convs at half gain), biases N(0, 0.02), snake
    alpha/beta N(0, 0.1)"""
    man = orc.vae_manifest(spec)
    r = rng(seed)
    w = np.empty(sum(n for _, n, _ in man), np.float32)
    for name, n, off in man:
        if name.endswith(".alpha") or name.endswith(".beta"):
            std = 0.1
        elif name.endswith(".bias"):
            std = 0.02
        else:
            layer = int(name.split(".")[2])
            oc = spec["width"][0] if layer == 0 else spec["out_ch"] if layer == 7 else spec["width"][layer]
            std = 1.0 / np.sqrt(n / oc) * (0.5 if name.endswith(".layers.3.weight") else 1.0)
        w[off:off + n] = (std * r.standard_normal(n)).astype(np.float32)
    return w, {name: (off, n) for name, n, off in man}


def test_snake_invariants(orc):
    C = 5
    r = rng(3)
    alpha = (0.5 * r.standard_normal(C)).astype(np.float32)
    beta = (0.5 * r.standard_normal(C)).astype(np.float32)
    ea, eb = np.exp(alpha.astype(np.float64)), np.exp(-beta.astype(np.float64))
    # bound, and equality at x*exp(alpha) = pi/2 + k*pi
    x = (4 * r.standard_normal((200, C))).astype(np.float32)
    y = orc.snake(x, alpha, beta)
    assert np.all(np.abs(y.astype(np.float64) - x) <= eb * (1 + 1e-5) + 1e-6)
    k = np.arange(-3, 4)[:, None]
    xq = ((np.pi / 2 + k * np.pi) / ea).astype(np.float32)
    yq = orc.snake(xq, alpha, beta)
    np.testing.assert_allclose(yq - xq, np.broadcast_to(eb, yq.shape), rtol=1e-5, atol=1e-6)
    # zeros of the sine: y = x
    xz = ((k * np.pi) / ea).astype(np.float32)
    np.testing.assert_allclose(orc.snake(xz, alpha, beta), xz, rtol=0, atol=1e-6)
    # period pi*exp(-alpha) of y - x
    x0 = (0.3 * r.standard_normal((50, C))).astype(np.float32)
    x1 = (x0 + np.pi / ea).astype(np.float32)
    d0 = orc.snake(x0, alpha, beta) - x0
    d1 = orc.snake(x1, alpha, beta).astype(np.float64) - x1
    np.testing.assert_allclose(d1, d0, rtol=0, atol=1e-5)


@pytest.mark.parametrize("s,K", [(8, 16), (4, 8), (2, 4), (3, 6)])
def test_conv_t_matches_library_transposed_conv(orc, s, K):
    T, IC, OC = 9, 6, 5
    r = rng(s * 10 + K)
    W = r.standard_normal((OC, IC, K)).astype(np.float32)
    b = r.standard_normal(OC).astype(np.float32)
    x = r.standard_normal((T, IC)).astype(np.float32)
    pad = K - 1 - s // 2
    y = orc.conv1d_t(W, b, x, s, pad)
    assert y.shape == (T * s, OC)
    # PyTorch: weight [IC][OC][K] flipped, padding p = K - 1 - pad; its output length (T-1)s - 2p + K is
    # T*s for even s (one more row for odd s, which the reference's OL = T*s leaves out)
    p = K - 1 - pad
    Wt = torch.from_numpy(W.astype(np.float64)).permute(1, 0, 2).flip(2)
    yt = Fn.conv_transpose1d(torch.from_numpy(x.astype(np.float64)).T[None], Wt,
                             torch.from_numpy(b.astype(np.float64)), stride=s, padding=p)[0].T.numpy()
    assert yt.shape[0] == T * s + (s % 2)
    yt = yt[:T * s]
    assert rel_l2(y, yt) < 1e-6
    # the scatter definition written out
    ys = np.zeros((T * s + 2 * K, OC))
    Wf = W.astype(np.float64)[:, :, ::-1]
    for i in range(T):
        for kk in range(K):
            ys[i * s + kk] += Wf[:, :, kk] @ x[i].astype(np.float64)
    ys = ys[p:p + T * s] + b
    assert rel_l2(y, ys) < 1e-6


@pytest.mark.parametrize("dil", [1, 3, 9])
def test_dilated_conv_matches_library(orc, dil):
    T, IC, OC = 40, 8, 6
    r = rng(dil)
    W = r.standard_normal((OC, IC, 7)).astype(np.float32)
    b = r.standard_normal(OC).astype(np.float32)
    x = r.standard_normal((T, IC)).astype(np.float32)
    y = orc.conv1d(W, b, x, pad=3 * dil, dil=dil)
    yt = Fn.conv1d(torch.from_numpy(x.astype(np.float64)).T[None], torch.from_numpy(W.astype(np.float64)),
                   torch.from_numpy(b.astype(np.float64)), padding=3 * dil, dilation=dil)[0].T.numpy()
    assert y.shape == (T, OC)
    assert rel_l2(y, yt) < 1e-6


def _decode64(spec, w, idx, latent):
    """float64 restatement of src/vae.cpp:17-86 from PyTorch's conv routines"""
    t = lambda a: torch.from_numpy(np.asarray(a, np.float64))
    get = lambda n: w[idx[n][0]:idx[n][0] + idx[n][1]].astype(np.float64)

    def conv(x, name, IC, OC, K, pad, dil=1, bias=True):
        W = t(get(name + ".weight").reshape(OC, IC, K))
        b = t(get(name + ".bias")) if bias else None
        return Fn.conv1d(x, W, b, padding=pad, dilation=dil)

    def snake(x, name):
        a = t(np.exp(get(name + ".alpha")))[None, :, None]
        e = t(np.exp(-get(name + ".beta")))[None, :, None]
        return x + torch.sin(x * a) ** 2 * e

    x = t(latent).T[None]   # [1, C, T]
    C = spec["width"][0]
    x = conv(x, "decoder.layers.0", spec["latent"], C, 7, 3)
    for n in range(5):
        bp = "decoder.layers.%d" % (n + 1)
        s, K, co = spec["stride"][n], spec["kt"][n], spec["width"][n + 1]
        h = snake(x, bp + ".layers.0")
        Wg = t(get(bp + ".layers.1.weight").reshape(co, C, K)).permute(1, 0, 2).flip(2)
        x = Fn.conv_transpose1d(h, Wg, t(get(bp + ".layers.1.bias")), stride=s, padding=s // 2)
        C = co
        for r, d in enumerate((1, 3, 9)):
            rp = bp + ".layers.%d" % (r + 2)
            g = conv(snake(x, rp + ".layers.0"), rp + ".layers.1", C, C, 7, 3 * d, d)
            g = conv(snake(g, rp + ".layers.2"), rp + ".layers.3", C, C, 1, 0)
            x = x + g
    x = conv(snake(x, "decoder.layers.6"), "decoder.layers.7", C, spec["out_ch"], 7, 3, bias=False)
    return x[0].T.numpy()


@pytest.mark.parametrize("T", [1, 3])
def test_decode_matches_float64_composition(orc, T):
    spec = small_spec(T)
    w, idx = vae_weights(orc, spec, seed=T)
    latent = rng(10 + T).standard_normal((T, 64)).astype(np.float32)
    a = orc.vae_decode(spec, w, latent)
    assert a.shape == (T * 2 * 4 * 2 * 2 * 2, 2) == (orc.vae_audio_len(spec), 2)
    ref = _decode64(spec, w, idx, latent)
    assert ref.shape == a.shape
    assert rel_l2(a, ref) < 2e-5


def test_manifest_structure(orc):
    spec = dict(T=4, latent=64, width=[2048, 1024, 512, 256, 128, 128], stride=[8, 8, 4, 4, 2],
                kt=[16, 16, 8, 8, 4], out_ch=2)
    man = orc.vae_manifest(spec)
    assert len(man) == 2 + 5 * (2 + 2 + 3 * 8) + 2 + 1
    d = {n: c for n, c, _ in man}
    assert d["decoder.layers.1.layers.1.weight"] == 1024 * 2048 * 16
    assert d["decoder.layers.5.layers.4.layers.1.weight"] == 128 * 128 * 7
    assert d["decoder.layers.7.weight"] == 2 * 128 * 7
    assert "decoder.layers.7.bias" not in d
    assert orc.vae_audio_len(spec) == 4 * 2048
