"""GPU parity of the reference checkpoint's DiT graph (libtsn tsn_refdit_*) against the oracle's
restatement of src/dit_fwd.cpp:104-304 (oracle/oracle_ref.cpp) on identical seeded weights and
inputs, at the reference's own 8 s geometry (B = 2 CFG arms, T = 172 latent, C = 64 clip,
TS = 154 text rows, H = 1024, SwiGLU F = 2816, 7 joint + 14 fused blocks):

  * one evaluation: velocity rel-L2 <= 1e-3, the three streams after every block <= 2e-3;
  * structure, bit-exact: the pre-only last joint block and the fused blocks leave the clip and
    text rows untouched; samples do not mix;
  * bit-identical reruns, eager and hipGraph replay (with eager work between replays);
  * the CFG Euler sampler (2 steps): displacement x - x0 rel-L2 <= 2e-3, graph replay bit-identical;
  * real-weight mode: a small GGUF checkpoint with F32, F16, BF16 and Q8_0 tensors loads by name
    and its velocity matches the oracle on the decoded weights (rel-L2 <= 1e-3).

Tolerances: velocity rel-L2 <= 1e-3 per evaluation and <= 2e-3 per block output (f16 MFMA operands,
f32 accumulation and residual streams).
"""
import numpy as np
import pytest

from conftest import rel_l2

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ref(tsn, rt):
    spec = tsn.ref_spec_for_duration(8, 2)
    w16 = tsn.ref_synth_weights(spec, 4242, 1.0)     # q/k norm weights 1 + N(0, 0.02)
    m = tsn.RefDitModel(rt, spec)
    m.upload_weights(w16)
    yield spec, m, tsn.bf16_to_f32(w16)
    m.close()


def _io(tsn, rt, spec, seed=4242, cfg_pairs=False):
    inp = tsn.ref_synth_inputs(spec, seed, cfg_pairs=cfg_pairs)
    return inp, {k: rt.array(v) for k, v in inp.items()}


def _fwd(m, rt, spec, dev, taps=None):
    v = rt.empty((spec.B, spec.T, spec.latent))
    m.forward_ex(dev["x"], dev["t"], dev["clip_pp"], dev["text_pp"], dev["gcmlp"], dev["sync_gather"], v, taps)
    rt.sync()
    return v


def test_ref_forward_parity_and_taps(tsn, rt, orc, ref):
    spec, m, w32 = ref
    inp, dev = _io(tsn, rt, spec)
    nblk = spec.n_joint + spec.n_fused
    S, T, C = spec.T + spec.C + spec.TS, spec.T, spec.C
    taps = rt.empty((nblk, spec.B, S, spec.H))
    v = _fwd(m, rt, spec, dev, taps).numpy()
    vr, tr = orc.ref_dit_forward(spec.as_dict(), w32, taps=True, **inp)
    tg = taps.numpy()
    err = rel_l2(v, vr)
    blk = [rel_l2(tg[i], tr[i]) for i in range(nblk)]
    lat = [rel_l2(tg[i][:, :T], tr[i][:, :T]) for i in range(nblk)]
    clip = [rel_l2(tg[i][:, T:T + C], tr[i][:, T:T + C]) for i in range(nblk)]
    text = [rel_l2(tg[i][:, T + C:], tr[i][:, T + C:]) for i in range(nblk)]
    print("velocity rel-L2 %.3g; worst block %.3g (latent %.3g, clip %.3g, text %.3g)"
          % (err, max(blk), max(lat), max(clip), max(text)))
    assert err <= 1e-3
    assert max(blk) <= 2e-3 and max(lat) <= 2e-3 and max(clip) <= 2e-3 and max(text) <= 2e-3
    # pre-only last joint block and fused blocks leave clip and text rows as they were
    nj = spec.n_joint
    for i in range(nj - 1, nblk):
        assert np.array_equal(tg[i][:, T:].view(np.uint32), tg[nj - 2][:, T:].view(np.uint32))


def test_ref_samples_do_not_mix(tsn, rt, ref):
    spec, m, _ = ref
    inp, dev = _io(tsn, rt, spec, seed=91)
    a = _fwd(m, rt, spec, dev).numpy()
    for k in ("x", "clip_pp", "text_pp", "gcmlp", "sync_gather"):
        b = inp[k].copy()
        b[0] = b[0][::-1] if b.ndim > 2 else -b[0]
        d = dict(dev, **{k: rt.array(b)})
        out = _fwd(m, rt, spec, d).numpy()
        assert np.array_equal(out[1].view(np.uint32), a[1].view(np.uint32)), k
        assert not np.array_equal(out[0], a[0]), k


def test_ref_bit_identical_and_graph(tsn, rt, ref):
    spec, m, _ = ref
    inp, dev = _io(tsn, rt, spec, seed=77)
    a = _fwd(m, rt, spec, dev).numpy()
    b = _fwd(m, rt, spec, dev).numpy()
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    v3 = rt.empty((spec.B, spec.T, spec.latent))
    m.capture_forward(dev["x"], dev["t"], dev["clip_pp"], dev["text_pp"], dev["gcmlp"], dev["sync_gather"], v3)
    for _ in range(3):
        m.replay()
        rt.sync()
        assert np.array_equal(a.view(np.uint32), v3.numpy().view(np.uint32))
        _fwd(m, rt, spec, dev)   # eager work on the same buffers between replays
    # scalar-t entry point (DitModel::forward signature) matches the device-t one
    v4 = rt.empty((spec.B, spec.T, spec.latent))
    m.forward(dev["x"], float(inp["t"][0]), dev["clip_pp"], dev["text_pp"], dev["gcmlp"], dev["sync_gather"], v4)
    rt.sync()
    assert np.array_equal(a.view(np.uint32), v4.numpy().view(np.uint32))


def test_ref_sampler_two_steps(tsn, rt, orc, ref):
    spec, m, w32 = ref
    inp, dev = _io(tsn, rt, spec, cfg_pairs=True)
    x0 = inp["x"][0::2].copy()
    x = rt.array(x0)
    args = (dev["clip_pp"], dev["text_pp"], dev["gcmlp"], dev["sync_gather"])
    m.sample(x, *args, 2, 5.0)
    rt.sync()
    out = x.numpy()
    r = orc.ref_dit_sample(spec.as_dict(), w32, x0, inp["clip_pp"], inp["text_pp"], inp["gcmlp"],
                           inp["sync_gather"], 2, 5.0)
    err = rel_l2(out - x0, r - x0)
    print("reference-graph sampler displacement rel-L2 %.3g" % err)
    assert out.shape == (spec.B // 2, spec.T, spec.latent)
    assert err <= 2e-3
    x2 = rt.array(x0)
    m.capture_sample(x2, *args, 2, 5.0)
    m.replay()
    rt.sync()
    assert np.array_equal(out.view(np.uint32), x2.numpy().view(np.uint32))


def test_ref_gguf_checkpoint(tsn, rt, orc, tmp_path):
    """A small checkpoint written as GGUF with every tensor type the reader takes (F32 vectors, F16,
    BF16 and Q8_0 matrices, conv weights as (K, IC, OC) dims) goes through tsn_refdit_spec_from_gguf
    and tsn_refdit_load_gguf; the velocity matches the oracle run on the reader's own decoded
    weights (rel-L2 <= 1e-3), so names, shapes, dequantization and every upload-time layout agree."""
    import gguf_writer as gw
    from conftest import rng
    geo = dict(B=2, T=20, C=8, TS=12)
    spec_d = dict(geo, H=256, NH=4, HD=64, F=128, latent=64, n_joint=2, n_fused=1, rope_theta=10000.0,
                  t_max_period=1.0, ln_eps=1e-5, rms_eps=1e-6)
    man = orc.ref_manifest(spec_d)
    r = rng(11)
    tensors = []
    for i, (name, n, _) in enumerate(man):
        ne = gw.ref_ne(name, n, spec_d)
        vals = ((1.0 if "norm.weight" in name else 0.0) + 0.05 * r.standard_normal(n)).astype(np.float32)
        if len(ne) == 1:
            ty = gw.F32
        elif ne[0] % 32 == 0 and i % 3 == 0:
            ty = gw.Q8_0
        else:
            ty = (gw.F16, gw.BF16)[i % 2]
        tensors.append((name, ne, ty, vals))
    meta = [("dit.hidden_dim", gw.KV_U32, 256), ("dit.num_heads", gw.KV_U32, 4), ("dit.depth", gw.KV_U32, 3),
            ("dit.fused_depth", gw.KV_U32, 1), ("dit.latent_dim", gw.KV_U32, 64)]
    path = str(tmp_path / "tiny.gguf")
    dec = gw.write(path, tensors, meta)
    assert {t for _, _, t, _ in tensors} == {gw.F32, gw.F16, gw.BF16, gw.Q8_0}
    spec = tsn.ref_spec_from_gguf(path, **geo)
    assert spec.as_dict() == pytest.approx(spec_d)
    m = tsn.RefDitModel(rt, spec)
    try:
        m.load_gguf(path)
        w32 = np.concatenate([dec[name] for name, _, _ in man])
        inp = tsn.ref_synth_inputs(spec, 4242)
        dev = {k: rt.array(v) for k, v in inp.items()}
        v = rt.empty((spec.B, spec.T, spec.latent))
        m.forward_ex(dev["x"], dev["t"], dev["clip_pp"], dev["text_pp"], dev["gcmlp"], dev["sync_gather"], v)
        rt.sync()
        vr = orc.ref_dit_forward(spec_d, w32, **inp)
        err = rel_l2(v.numpy(), vr)
        print("gguf checkpoint velocity rel-L2 %.3g" % err)
        assert err <= 1e-3
    finally:
        m.close()


def test_ref_gguf_bf16_reference_size(tsn, rt, ref, tmp_path):
    """The reference-size checkpoint (every tensor of the 8 s graph, 1.2 G BF16 parameters) written
    as a BF16 GGUF from the same bits the module's model was uploaded from: tsn_refdit_load_gguf
    moves the raw payloads to HBM and converts them there, and the evaluation is bit-identical to
    the model uploaded from the flat BF16 buffer."""
    import os
    import gguf_writer as gw
    spec, m, _ = ref
    sd = spec.as_dict()
    w16 = tsn.ref_synth_weights(spec, 4242, 1.0)
    man = tsn.ref_manifest(spec)
    path = str(tmp_path / "ref8s.gguf")
    meta = [("dit.hidden_dim", gw.KV_U32, spec.H), ("dit.num_heads", gw.KV_U32, spec.NH),
            ("dit.depth", gw.KV_U32, spec.n_joint + spec.n_fused), ("dit.fused_depth", gw.KV_U32, spec.n_fused),
            ("dit.latent_dim", gw.KV_U32, spec.latent)]
    size = gw.write_bf16(path, [(n, gw.ref_ne(n, k, sd), w16[o:o + k]) for n, k, o in man], meta)
    assert size > 2 * int(w16.size)
    del w16
    m2 = tsn.RefDitModel(rt, tsn.ref_spec_from_gguf(path, spec.B, spec.T, spec.C, spec.TS))
    try:
        m2.load_gguf(path)
        os.remove(path)
        inp, dev = _io(tsn, rt, spec, seed=12)
        a = _fwd(m, rt, spec, dev).numpy()
        b = _fwd(m2, rt, spec, dev).numpy()
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    finally:
        m2.close()


def test_ref_replay_refused_after_sampler_reallocation(tsn, rt, ref):
    """as for the configured graph: a sampler run with another step count reallocates what the
    captured sampler addresses; the old graph refuses to replay, a new capture matches eager"""
    spec, m, _ = ref
    inp, dev = _io(tsn, rt, spec, seed=6, cfg_pairs=True)
    args = (dev["clip_pp"], dev["text_pp"], dev["gcmlp"], dev["sync_gather"])
    x0 = inp["x"][0::2].copy()
    m.capture_sample(rt.array(x0), *args, 2, 5.0)
    xb = rt.array(x0)
    m.sample(xb, *args, 3, 5.0)
    rt.sync()
    with pytest.raises(tsn.TsnError) as e:
        m.replay()
    assert e.value.code == 5
    eager3 = xb.numpy()
    xc = rt.array(x0)
    m.capture_sample(xc, *args, 3, 5.0)
    m.replay()
    rt.sync()
    assert np.array_equal(xc.numpy().view(np.uint32), eager3.view(np.uint32))
