"""GPU parity of the reference's text encoders (tsn_clip_*, tsn_t5_*: ClipModel::encode, src/clip.cpp:34-92,
and T5Model::encode, src/t5.cpp:88-131) against the oracle (oracle/oracle_enc.cpp), f32 weights from the
specified synthetic generator:

  * CLIP at the reference's full size (24 layers, H = 1024, 16 heads, 77 tokens, vocabulary 49408):
    per-token features and the pooled vector within rel-L2 1e-4;
  * T5 at the reference's widths (d = 2048, d_ff = 5120, 32 heads, 77 tokens, vocabulary 32128),
    padded ids: with 4 of its 24 layers within 1e-4; at the full 24 layers (1.2 G f32 weights,
    about 30 s of host work) within 2e-3. Random-init T5 amplifies rounding-level differences with
    depth: perturbing every weight by 6e-8 relative (half an f32 ulp) moves the f32 oracle's own
    output by 5.4e-6 at 4 layers, 5.6e-5 at 12 and 4.2e-4 at 24 (measured), so at full depth two
    correct f32 implementations that only sum in different orders differ by that much;
  * small widths for both, with an end-of-text token in the middle of the context (CLIP) and
    padding (T5);
  * bit-identical reruns; a GGUF load (F32 tensors) encodes bit-identically to the flat upload.
"""
import numpy as np
import pytest

from conftest import rel_l2, rng

pytestmark = pytest.mark.gpu

TOL = 1e-4


def _clip_ids(spec, seed):
    r = rng(seed)
    n = int(r.integers(5, spec.ctx - 2))
    ids = [spec.vocab - 2] + list(r.integers(0, spec.vocab - 2, size=n)) + [spec.vocab - 1]
    return np.array(ids + [spec.vocab - 1] * (spec.ctx - len(ids)), np.int32)


def _t5_ids(spec, seed):
    r = rng(seed)
    n = int(r.integers(5, spec.ctx - 2))
    ids = list(r.integers(2, spec.vocab, size=n)) + [1]
    return np.array(ids + [0] * (spec.ctx - len(ids)), np.int32)


@pytest.mark.parametrize("size", ["full", "small"])
def test_clip_parity(tsn, rt, orc, size):
    spec = tsn.clip_spec_default()
    if size == "small":
        spec = spec.copy(H=256, NL=3, NH=4, ctx=21, vocab=300)
    w = tsn.clip_synth_weights(spec, 21)
    m = tsn.ClipModel(rt, spec)
    try:
        m.upload_weights(w)
        ids = _clip_ids(spec, 3)
        pt, g = rt.empty((spec.ctx, spec.H)), rt.empty((spec.H,))
        m.encode(ids, pt, g)
        rt.sync()
        rpt, rg = orc.clip_encode(spec.as_dict(), w, ids)
        e1, e2 = rel_l2(pt.numpy(), rpt), rel_l2(g.numpy(), rg)
        print("clip %s: per-token rel-L2 %.3g, pooled %.3g" % (size, e1, e2))
        assert e1 <= TOL and e2 <= TOL
        pt2, g2 = rt.empty((spec.ctx, spec.H)), rt.empty((spec.H,))
        m.encode(ids, pt2, g2)
        rt.sync()
        assert np.array_equal(pt2.numpy().view(np.uint32), pt.numpy().view(np.uint32))
        assert np.array_equal(g2.numpy().view(np.uint32), g.numpy().view(np.uint32))
    finally:
        m.close()


@pytest.mark.parametrize("size", ["full", "full_width_4_layers", "small"])
def test_t5_parity(tsn, rt, orc, size):
    spec = tsn.t5_spec_default()
    tol = 2e-3 if size == "full" else TOL
    if size == "full_width_4_layers":
        spec = spec.copy(NL=4)
    if size == "small":
        spec = spec.copy(d=256, d_ff=320, NL=3, NH=4, ctx=19, vocab=200)
    print("t5 %s: synthesising %d layers of weights" % (size, spec.NL), flush=True)
    w = tsn.t5_synth_weights(spec, 22)
    m = tsn.T5Model(rt, spec)
    try:
        m.upload_weights(w)
        ids = _t5_ids(spec, 4)
        out = rt.empty((spec.ctx, spec.d))
        m.encode(ids, out)
        rt.sync()
        print("t5 %s: oracle" % size, flush=True)
        ref = orc.t5_encode(spec.as_dict(), w, ids)
        e = rel_l2(out.numpy(), ref)
        print("t5 %s: rel-L2 %.3g, max |ref| %.3g" % (size, e, np.abs(ref).max()))
        assert e <= tol
        out2 = rt.empty((spec.ctx, spec.d))
        m.encode(ids, out2)
        rt.sync()
        assert np.array_equal(out2.numpy().view(np.uint32), out.numpy().view(np.uint32))
    finally:
        m.close()


def test_encoders_gguf_load(tsn, rt, tmp_path):
    from gguf_writer import F32, KV_F32, KV_U32, write
    cspec = tsn.clip_spec_default().copy(H=128, NL=2, NH=2, ctx=9, vocab=64)
    tspec = tsn.t5_spec_default().copy(d=128, d_ff=160, NL=2, NH=2, ctx=9, vocab=48)
    cw, tw = tsn.clip_synth_weights(cspec, 5), tsn.t5_synth_weights(tspec, 6)
    cpath, tpath = str(tmp_path / "clip.gguf"), str(tmp_path / "t5.gguf")
    ct = [(n, (k,), F32, cw[o:o + k]) for n, k, o in tsn.clip_manifest(cspec)]
    ct[0] = ("tok_emb", (128, 64), F32, cw[:128 * 64])
    write(cpath, ct, [("clip.hidden", KV_U32, 128), ("clip.layers", KV_U32, 2), ("clip.heads", KV_U32, 2),
                      ("clip.ctx", KV_U32, 9)])
    tt = [(n, (k,), F32, tw[o:o + k]) for n, k, o in tsn.t5_manifest(tspec)]
    tt[0] = ("tok_emb", (128, 48), F32, tw[:128 * 48])
    write(tpath, tt, [("t5.d_model", KV_U32, 128), ("t5.d_ff", KV_U32, 160), ("t5.n_layers", KV_U32, 2),
                      ("t5.n_heads", KV_U32, 2), ("t5.eps", KV_F32, 1e-6)])
    cs = tsn.clip_spec_from_gguf(cpath)
    assert (cs.H, cs.NL, cs.NH, cs.ctx, cs.vocab) == (128, 2, 2, 9, 64)
    ts = tsn.t5_spec_from_gguf(tpath)
    assert (ts.d, ts.d_ff, ts.NL, ts.NH, ts.vocab, ts.ctx) == (128, 160, 2, 2, 48, 77)
    ts = ts.copy(ctx=9)   # the context is the reference's constant (T5_TOKEN_CTX), not checkpoint metadata
    models = []
    try:
        a, b = tsn.ClipModel(rt, cspec), tsn.ClipModel(rt, cs)
        models += [a, b]
        a.upload_weights(cw)
        b.load_gguf(cpath)
        ids = _clip_ids(cspec, 7)
        outs = []
        for m in (a, b):
            pt, g = rt.empty((9, 128)), rt.empty((128,))
            m.encode(ids, pt, g)
            rt.sync()
            outs.append(pt.numpy())
        assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
        c, d = tsn.T5Model(rt, tspec), tsn.T5Model(rt, ts)
        models += [c, d]
        c.upload_weights(tw)
        d.load_gguf(tpath)
        ids = _t5_ids(tspec, 8)
        outs = []
        for m in (c, d):
            o = rt.empty((9, 128))
            m.encode(ids, o)
            rt.sync()
            outs.append(o.numpy())
        assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    finally:
        for m in models:
            m.close()
