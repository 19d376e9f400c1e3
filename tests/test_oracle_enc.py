"""Pinning of the oracle's text encoders (oracle/oracle_enc.cpp) and tokenizer restatement
(oracle/pyoracle.py) — CPU only.

Checked against:
  * T5 relative buckets: 0 at distance 0, the exact range |rel| < 8 (+16 for keys after the query),
    the log-spaced thresholds 8*2^(j/2) of the closed form away from its exact powers, saturation
    at 15 / 31 from distance 128, and monotonicity;
  * attention: a CLIP row 0 is V's row 0 (one visible key), a T5 row with one unpadded key is that
    key's V row, and random cases against a float64 NumPy softmax with the mask / bias applied;
  * LayerNorm (zero mean, variance var/(var + eps) before the affine) and RMSNorm (unit RMS);
  * whole encoders on small widths against a float64 composition of PyTorch primitives written
    from src/clip.cpp and src/t5.cpp (LayerNorm / RMSNorm, masked softmax, quick GELU, tanh GELU);
  * the unigram segmentation against brute force over every segmentation of short strings (random
    continuous scores, so the optimum is unique), and BPE merges against hand-worked answers.
"""
import itertools
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as Fn

from conftest import rel_l2, rng


def clip_small(ctx=9):
    return dict(H=128, NL=2, NH=2, ctx=ctx, vocab=50, eps=1e-5)


def t5_small(ctx=9):
    return dict(d=128, d_ff=192, NL=2, NH=2, ctx=ctx, vocab=40, n_bucket=32, max_dist=128, eps=1e-6)


def enc_weights(man, seed, fan):
    """embeddings N(0, 1), norm weights 1 + N(0, 0.1), biases N(0, 0.02), linears N(0, 1/fan_in)"""
    r = rng(seed)
    w = np.empty(sum(n for _, n, _ in man), np.float32)
    for name, n, off in man:
        if name in ("tok_emb", "pos_emb"):
            std, mean = 1.0, 0.0
        elif name == "rel_bias":
            std, mean = 0.5, 0.0
        elif name.endswith("norm") or name.endswith("ln1.w") or name.endswith("ln2.w") or name == "out_ln.w":
            std, mean = 0.1, 1.0
        elif name.endswith(".b"):
            std, mean = 0.02, 0.0
        else:
            std, mean = 1.0 / math.sqrt(fan(name)), 0.0
        w[off:off + n] = (mean + std * r.standard_normal(n)).astype(np.float32)
    return w, {name: (off, n) for name, n, off in man}


def test_t5_bucket_closed_form(orc):
    assert orc.t5_bucket(0) == 0
    for n in range(1, 8):
        assert orc.t5_bucket(-n) == n and orc.t5_bucket(n) == 16 + n
    # bucket 8 + j from distance 8 * 2^(j/2) on (checked away from the exact powers of two)
    known = {9: 8, 11: 8, 12: 9, 15: 9, 17: 10, 22: 10, 23: 11, 31: 11, 33: 12, 45: 12, 46: 13, 63: 13, 65: 14,
             90: 14, 91: 15, 127: 15, 129: 15, 1000: 15}
    for n, b in known.items():
        assert orc.t5_bucket(-n) == b, n
        assert orc.t5_bucket(n) == 16 + b, n
    seq = [orc.t5_bucket(-n) for n in range(0, 300)]
    assert all(a <= b for a, b in zip(seq, seq[1:]))


def _softmax_attn64(qkv, nh, scale, mask_bias):
    S = qkv.shape[0]
    H = nh * 64
    q, k, v = (qkv[:, j * H:(j + 1) * H].astype(np.float64).reshape(S, nh, 64) for j in range(3))
    out = np.zeros((S, H))
    for h in range(nh):
        s = q[:, h] @ k[:, h].T * scale + mask_bias(h)
        s = s - s.max(1, keepdims=True)
        p = np.exp(s)
        p /= p.sum(1, keepdims=True)
        out[:, h * 64:(h + 1) * 64] = p @ v[:, h]
    return out


def test_attention_modes(orc):
    r = rng(4)
    S, nh = 11, 3
    qkv = r.standard_normal((S, 3 * nh * 64)).astype(np.float32)
    H = nh * 64
    # CLIP: causal and nothing past eot
    eot = 7
    o = orc.enc_attention(qkv, nh, 0.125, 2, eot=eot)
    np.testing.assert_allclose(o[0], qkv[0, 2 * H:], rtol=1e-6, atol=1e-6)
    qi, ki = np.meshgrid(np.arange(S), np.arange(S), indexing="ij")
    m = np.where((ki <= qi) & (ki <= eot), 0.0, -np.inf)
    assert rel_l2(o, _softmax_attn64(qkv, nh, 0.125, lambda h: m)) < 1e-6
    # T5: bucket bias per head, padded keys masked
    bucket = np.array([[orc.t5_bucket(k - q) for k in range(S)] for q in range(S)], np.int32)
    rel = r.standard_normal((32, nh)).astype(np.float32)
    pad = np.ones(S, np.int32)
    pad[[2, 9]] = 0
    o = orc.enc_attention(qkv, nh, 1.0, 1, bucket=bucket, rel=rel, pad=pad)
    mb = lambda h: np.where(pad[None, :] == 0, -np.inf, rel[bucket, h].astype(np.float64))
    assert rel_l2(o, _softmax_attn64(qkv, nh, 1.0, mb)) < 1e-6
    only = np.zeros(S, np.int32)
    only[5] = 1
    o = orc.enc_attention(qkv, nh, 1.0, 1, bucket=bucket, rel=rel, pad=only)
    np.testing.assert_allclose(o, np.repeat(qkv[5:6, 2 * H:], S, 0), rtol=1e-6, atol=1e-6)


def test_norms(orc):
    x = (3 + 2 * rng(5).standard_normal((6, 256))).astype(np.float32)
    y = orc.ln_wb(x, np.ones(256), np.zeros(256), 1e-5)
    var = x.astype(np.float64).var(1)
    np.testing.assert_allclose(y.mean(1), 0, atol=1e-5)
    np.testing.assert_allclose(y.astype(np.float64).var(1), var / (var + 1e-5), rtol=1e-5)
    z = orc.rms_w(x, np.ones(256), 1e-6)
    np.testing.assert_allclose(np.sqrt((z.astype(np.float64) ** 2).mean(1)), 1.0, rtol=1e-5)


def _t(a):
    return torch.from_numpy(np.asarray(a, np.float64))


def _clip64(spec, w, idx, ids):
    get = lambda n: _t(w[idx[n][0]:idx[n][0] + idx[n][1]])
    H, n, nh = spec["H"], spec["ctx"], spec["NH"]
    lin = lambda x, name, N, K, bias=True: x @ get(name + ".w").reshape(N, K).T + (get(name + ".b") if bias else 0)
    x = get("tok_emb").reshape(-1, H)[torch.from_numpy(np.asarray(ids, np.int64))] + get("pos_emb").reshape(n, H)
    eos = int(np.argmax(ids))
    qi, ki = np.meshgrid(np.arange(n), np.arange(n), indexing="ij")
    mask = _t(np.where((ki <= qi) & (ki <= eos), 0.0, -np.inf))
    for l in range(spec["NL"]):
        b = "blk.%d" % l
        r = Fn.layer_norm(x, (H,), get(b + ".ln1.w"), get(b + ".ln1.b"), spec["eps"])
        q, k, v = (lin(r, b + t, H, H).reshape(n, nh, 64).transpose(0, 1) for t in (".q", ".k", ".v"))
        p = torch.softmax(q @ k.transpose(1, 2) / 8.0 + mask, -1)
        a = (p @ v).transpose(0, 1).reshape(n, H)
        x = x + lin(a, b + ".out", H, H)
        r = Fn.layer_norm(x, (H,), get(b + ".ln2.w"), get(b + ".ln2.b"), spec["eps"])
        f = lin(r, b + ".fc1", 4 * H, H)
        f = f * torch.sigmoid(1.702 * f)
        x = x + lin(f, b + ".fc2", H, 4 * H)
    pt = Fn.layer_norm(x, (H,), get("out_ln.w"), get("out_ln.b"), spec["eps"])
    return pt.numpy(), (get("text_proj").reshape(H, H) @ pt[eos]).numpy()


def _t564(spec, w, idx, ids, orc):
    get = lambda n: _t(w[idx[n][0]:idx[n][0] + idx[n][1]])
    d, F, n, nh = spec["d"], spec["d_ff"], spec["ctx"], spec["NH"]
    rms = lambda x, g: x / torch.sqrt((x * x).mean(-1, keepdim=True) + spec["eps"]) * g
    x = get("tok_emb").reshape(-1, d)[torch.from_numpy(np.asarray(ids, np.int64))]
    bucket = np.array([[orc.t5_bucket(k - q) for k in range(n)] for q in range(n)])
    rel = get("rel_bias").reshape(spec["n_bucket"], nh)
    bias = rel[torch.from_numpy(bucket)].permute(2, 0, 1)   # [nh, q, k]
    padm = _t(np.where(np.asarray(ids) == 0, -np.inf, 0.0))[None, None, :]
    bias = torch.where(torch.isinf(padm), padm, bias)
    for l in range(spec["NL"]):
        b = "blk.%d" % l
        r = rms(x, get(b + ".attn_norm"))
        q, k, v = (r @ get(b + t).reshape(d, d).T for t in (".q", ".k", ".v"))
        q, k, v = (t.reshape(n, nh, 64).transpose(0, 1) for t in (q, k, v))
        p = torch.softmax(q @ k.transpose(1, 2) + bias, -1)
        x = x + (p @ v).transpose(0, 1).reshape(n, d) @ get(b + ".o").reshape(d, d).T
        r = rms(x, get(b + ".ffn_norm"))
        u = r @ get(b + ".wi_0").reshape(F, d).T
        g = 0.5 * u * (1 + torch.tanh(torch.clamp(0.7978845608 * (u + 0.044715 * u ** 3), -10, 10)))
        x = x + (g * (r @ get(b + ".wi_1").reshape(F, d).T)) @ get(b + ".wo").reshape(d, F).T
    return rms(x, get("out_norm")).numpy()


def test_clip_encode_matches_float64(orc):
    spec = clip_small()
    man = orc.clip_manifest(spec)
    w, idx = enc_weights(man, 1, lambda n: 4 * spec["H"] if n.endswith("fc2.w") else spec["H"])
    ids = np.array([spec["vocab"] - 2, 3, 17, 5, spec["vocab"] - 1, spec["vocab"] - 1, spec["vocab"] - 1, 2, 9],
                   np.int32)   # eos (the largest id) first at 4; ids after it are not seen by earlier rows
    pt, g = orc.clip_encode(spec, w, ids)
    rpt, rg = _clip64(spec, w, idx, ids)
    assert rel_l2(pt, rpt) < 1e-5 and rel_l2(g, rg) < 1e-5


def test_t5_encode_matches_float64(orc):
    spec = t5_small()
    man = orc.t5_manifest(spec)
    w, idx = enc_weights(man, 2, lambda n: spec["d_ff"] if n.endswith(".wo") else spec["d"])
    ids = np.array([7, 31, 4, 1, 0, 0, 0, 0, 0], np.int32)   # eos 1, then padding
    out = orc.t5_encode(spec, w, ids)
    assert rel_l2(out, _t564(spec, w, idx, ids, orc)) < 1e-5


def _segmentations(chars):
    if not chars:
        yield []
        return
    for j in range(1, len(chars) + 1):
        for rest in _segmentations(chars[j:]):
            yield ["".join(chars[:j])] + rest


def test_unigram_against_brute_force(orc):
    r = rng(6)
    alphabet = ["▁", "a", "b", "c", "é"]
    pieces = ["<pad>", "</s>", "<unk>"] + sorted({"".join(r.choice(alphabet, size=k)) for k in (1, 2, 3) for _ in range(12)})
    scores = [0.0, 0.0, 0.0] + list(-r.uniform(1, 8, size=len(pieces) - 3))
    unk = min([0.0] + scores) - 10.0
    pid = {p: i for i, p in enumerate(pieces)}
    for _ in range(40):
        text = "".join(r.choice(["a", "b", "c", " ", "é", "d"], size=r.integers(1, 7)))
        ids = orc.t5_unigram_encode(pieces, scores, text, 64, False)
        chars = list("▁" + text.strip(" ").replace(" ", "▁"))
        best, best_ids = -1e30, None
        for seg in _segmentations(chars):
            if any(s not in pid and len(s) > 1 for s in seg):
                continue
            sc = sum(scores[pid[s]] if s in pid else unk for s in seg)
            if sc > best + 1e-9:
                best, best_ids = sc, [pid.get(s, 2) for s in seg]
        assert ids == best_ids + [1], text


def test_bpe_known_answers(orc):
    vocab = ["a", "b", "c", "a</w>", "b</w>", "c</w>", "ab", "abc</w>", "aa", "!", "!</w>"]
    merges = ["a b", "ab c</w>", "a a"]
    enc = lambda t, ctx=8: orc.clip_bpe_encode(vocab, merges, t, ctx, bos=100, eos=101)
    assert enc("ABC") == [100, 7, 101, 101, 101, 101, 101, 101]                 # a b c</w> -> ab c</w> -> abc</w>
    assert enc("abab") == [100, 6, 0, 4, 101, 101, 101, 101]                    # ab a b</w>
    assert enc("aaa\tc") == [100, 8, 3, 5, 101, 101, 101, 101]                  # aa a</w> | c</w>
    assert enc("a! zz") == [100, 0, 10, 101, 101, 101, 101, 101]                # unknown symbols dropped
    assert enc("abc " * 10, ctx=5) == [100, 7, 7, 7, 101]                       # cut: last id eos
