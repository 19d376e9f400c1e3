"""GPU parity of the reference's conditioning prep (tsn_refcond_*: DitModel::prep_conditioning and
prep_text_arm, src/dit.cpp:55-191) against the oracle (oracle/oracle_cond.cpp) at the 8 s geometry
(T = 172, C = 64, sync_S = 192, TS = 154, H = 1024, F = 2816) with random BF16 weights:

  * every output (clip_pp, sync_gather, clip_fc, text_pp, gcmlp) within rel-L2 1e-3;
  * the whole reference chain: prep (once) + two text arms + the reference graph's forward on the
    prepared tensors, CFG arms batched, velocity within 1e-3 of the oracle's chain;
  * bit-identical reruns.
"""
import numpy as np
import pytest

from conftest import rel_l2, rng

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def cond(tsn, rt):
    spec = tsn.cond_spec_for_duration(8)
    w16 = tsn.cond_synth_weights(spec, 99)
    m = tsn.RefCondModel(rt, spec)
    m.upload_weights(w16)
    yield spec, m, tsn.bf16_to_f32(w16)
    m.close()


def _inputs(spec, seed=7):
    r = rng(seed)
    f = lambda *sh: r.standard_normal(sh).astype(np.float32)
    return dict(clip_f=f(spec.C, spec.clip_dim), sync_f=f(spec.sync_S, spec.sync_dim),
                text_c=f(spec.TS, spec.text_dim), text_u=f(spec.TS, spec.text_dim),
                gtext_c=f(spec.gtext_dim), gtext_u=np.zeros(spec.gtext_dim, np.float32))


def _prep(rt, spec, m, inp):
    H = spec.H
    d = {k: rt.array(v) for k, v in inp.items()}
    clip_pp, sg, cfc = rt.empty((spec.C, H)), rt.empty((spec.T, H)), rt.empty((H,))
    m.prep_conditioning(d["clip_f"], d["sync_f"], clip_pp, sg, cfc)
    arms = []
    for a in ("c", "u"):
        tp, gc = rt.empty((spec.TS, H)), rt.empty((H,))
        m.prep_text_arm(d["text_" + a], d["gtext_" + a], cfc, tp, gc)
        arms.append((tp, gc))
    rt.sync()
    return clip_pp.numpy(), sg.numpy(), cfc.numpy(), [(tp.numpy(), gc.numpy()) for tp, gc in arms]


def test_cond_prep_parity(tsn, rt, orc, cond):
    spec, m, w32 = cond
    inp = _inputs(spec)
    clip_pp, sg, cfc, arms = _prep(rt, spec, m, inp)
    rc, rs, rf = orc.ref_prep_conditioning(spec.as_dict(), w32, inp["clip_f"], inp["sync_f"])
    errs = {"clip_pp": rel_l2(clip_pp, rc), "sync_gather": rel_l2(sg, rs), "clip_fc": rel_l2(cfc, rf)}
    for a, (tp, gc) in zip(("c", "u"), arms):
        rtp, rgc = orc.ref_prep_text_arm(spec.as_dict(), w32, inp["text_" + a], inp["gtext_" + a], rf)
        errs["text_pp_" + a] = rel_l2(tp, rtp)
        errs["gcmlp_" + a] = rel_l2(gc, rgc)
    print("conditioning prep rel-L2: " + ", ".join("%s %.3g" % kv for kv in errs.items()))
    assert max(errs.values()) <= 1e-3
    # reruns are bit-identical
    again = _prep(rt, spec, m, inp)
    assert np.array_equal(again[0].view(np.uint32), clip_pp.view(np.uint32))
    assert np.array_equal(again[3][0][1].view(np.uint32), arms[0][1].view(np.uint32))


def test_cond_prep_feeds_forward(tsn, rt, orc, cond):
    """prep -> reference graph forward (CFG arms batched) against the oracle's prep -> forward"""
    spec, m, w32 = cond
    inp = _inputs(spec, seed=8)
    clip_pp, sg, cfc, arms = _prep(rt, spec, m, inp)
    dspec = tsn.ref_spec_for_duration(8, 2)
    dw16 = tsn.ref_synth_weights(dspec, 4242, 1.0)
    dit = tsn.RefDitModel(rt, dspec)
    try:
        dit.upload_weights(dw16)
        x = rng(9).standard_normal((1, dspec.T, dspec.latent)).astype(np.float32)
        batch = dict(x=np.repeat(x, 2, 0), t=np.full(2, 0.7, np.float32), clip_pp=np.stack([clip_pp] * 2),
                     text_pp=np.stack([arms[0][0], arms[1][0]]), gcmlp=np.stack([arms[0][1], arms[1][1]]),
                     sync_gather=np.stack([sg] * 2))
        dev = {k: rt.array(v) for k, v in batch.items()}
        v = rt.empty((2, dspec.T, dspec.latent))
        dit.forward_ex(dev["x"], dev["t"], dev["clip_pp"], dev["text_pp"], dev["gcmlp"], dev["sync_gather"], v)
        rt.sync()
        # the oracle's chain end to end
        rc, rs, rf = orc.ref_prep_conditioning(spec.as_dict(), w32, inp["clip_f"], inp["sync_f"])
        ra = [orc.ref_prep_text_arm(spec.as_dict(), w32, inp["text_" + a], inp["gtext_" + a], rf) for a in "cu"]
        ref = dict(batch, clip_pp=np.stack([rc] * 2), text_pp=np.stack([ra[0][0], ra[1][0]]),
                   gcmlp=np.stack([ra[0][1], ra[1][1]]), sync_gather=np.stack([rs] * 2))
        vr = orc.ref_dit_forward(dspec.as_dict(), tsn.bf16_to_f32(dw16), **ref)
        err = rel_l2(v.numpy(), vr)
        print("prep -> forward velocity rel-L2 %.3g" % err)
        assert err <= 1e-3
    finally:
        dit.close()
