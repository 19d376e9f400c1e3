"""GPU parity of the DiT velocity path (libtsn) against the CPU oracle on identical seeded weights
and inputs — the benchmark workloads at full size:

  * one joint block and one fused block (the single-block workload, B=2, La=256, Lt=141):
    rel-L2 <= 2e-3 per block output;
  * one full 21-block evaluation (8 s, B=2): velocity rel-L2 <= 1e-3, every block tap <= 2e-3;
  * bit-identical reruns (eager and hipGraph replay);
  * the CFG Euler sampler (2 steps at full size): displacement x - z0 rel-L2 <= 2e-3.

Tolerances: velocity rel-L2 <= 1e-3 per evaluation and <= 2e-3 per block output (f16 MFMA operands,
f32 accumulation and residual stream).
"""
import numpy as np
import pytest

from conftest import rel_l2

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def model(tsn, rt, orc):
    spec = tsn.default_spec(1)
    w16 = tsn.synth_weights(spec, 4242, 1.0)        # q/k norm weights 1 + N(0, 0.02): sharp attention
    w32 = tsn.bf16_to_f32(w16)
    m = tsn.DitModel(rt, spec)
    m.upload_weights(w16)
    yield spec, m, w32
    m.close()


def _io(tsn, rt, spec, seed=4242, cfg_pairs=False):
    inp = tsn.synth_inputs(spec, seed, cfg_pairs=cfg_pairs)
    dev = {k: rt.array(v) for k, v in inp.items()}
    return inp, dev


def test_joint_block(tsn, rt, orc, model):
    spec, m, w32 = model
    S = spec.La + spec.Lt
    X = tsn.synth_normal_f32(4242, tsn.IDX_X, 0.0, 1.0, (spec.B, S, spec.H))
    g = tsn.synth_normal_f32(4242, tsn.IDX_G, 0.0, 1.0, (spec.B, spec.H))
    Xd, gd = rt.array(X), rt.array(g)
    m.joint_block(0, Xd, gd)
    rt.sync()
    out = Xd.numpy()
    ref = orc.joint_block(spec, w32, 0, X, g)
    err = rel_l2(out, ref)
    print("joint block rel-L2 %.3g" % err)
    assert err <= 2e-3
    # both streams individually
    assert rel_l2(out[:, :spec.La], ref[:, :spec.La]) <= 2e-3
    assert rel_l2(out[:, spec.La:], ref[:, spec.La:]) <= 2e-3


def test_fused_block(tsn, rt, orc, model):
    spec, m, w32 = model
    S = spec.La + spec.Lt
    X = tsn.synth_normal_f32(4243, tsn.IDX_X, 0.0, 1.0, (spec.B, S, spec.H))
    g = tsn.synth_normal_f32(4243, tsn.IDX_G, 0.0, 1.0, (spec.B, spec.H))
    Xd, gd = rt.array(X), rt.array(g)
    m.fused_block(3, Xd, gd)
    rt.sync()
    err = rel_l2(Xd.numpy(), orc.fused_block(spec, w32, 3, X, g))
    print("fused block rel-L2 %.3g" % err)
    assert err <= 2e-3


def test_forward_parity_and_taps(tsn, rt, orc, model):
    spec, m, w32 = model
    inp, dev = _io(tsn, rt, spec)
    nblk = spec.n_joint + spec.n_fused
    S = spec.La + spec.Lt
    v = rt.empty((spec.B, spec.La, spec.latent))
    taps = rt.empty((nblk, spec.B, S, spec.H))
    m.forward_ex(dev["z"], dev["t"], dev["text"], dev["pooled"], v, taps)
    rt.sync()
    vr, tr, _ = orc.dit_forward(spec, w32, inp["z"], inp["t"], inp["text"], inp["pooled"], taps=True)
    err = rel_l2(v.numpy(), vr)
    tg = taps.numpy()
    blk = [rel_l2(tg[i], tr[i]) for i in range(nblk)]
    print("velocity rel-L2 %.3g; worst block %.3g" % (err, max(blk)))
    assert err <= 1e-3
    assert max(blk) <= 2e-3


@pytest.mark.parametrize("B,H,latent,La,Lt", [(2, 512, 32, 100, 37), (2, 2048, 64, 64, 20), (16, 512, 32, 40, 9)])
def test_forward_other_widths(tsn, rt, orc, B, H, latent, La, Lt):
    """The evaluation at hidden widths other than the benchmark's, one joint and one fused block,
    row counts that are not multiples of 16: H = 512 (8 heads, 32 latent channels) and H = 2048
    (32 heads), so the one-launch final layer runs with 2 and 8 float4 column groups per lane (its
    8-group build batches two rows per load instead of four); at B = 16 the conditioning GEMVs run
    on MFMA with K = 256 and K = 512. Velocity rel-L2 <= 1e-3, every block tap <= 2e-3."""
    spec = tsn.default_spec(1).copy(B=B, H=H, NH=H // 64, F=2 * H, latent=latent, La=La, Lt=Lt, n_joint=1,
                                    n_fused=1)
    w16 = tsn.synth_weights(spec, 91, 1.0)
    w32 = tsn.bf16_to_f32(w16)
    m = tsn.DitModel(rt, spec)
    try:
        m.upload_weights(w16)
        inp, dev = _io(tsn, rt, spec, seed=92)
        S = spec.La + spec.Lt
        v = rt.empty((spec.B, spec.La, spec.latent))
        taps = rt.empty((2, spec.B, S, spec.H))
        m.forward_ex(dev["z"], dev["t"], dev["text"], dev["pooled"], v, taps)
        rt.sync()
        vr, tr, _ = orc.dit_forward(spec, w32, inp["z"], inp["t"], inp["text"], inp["pooled"], taps=True)
        err = rel_l2(v.numpy(), vr)
        tg = taps.numpy()
        blk = [rel_l2(tg[i], tr[i]) for i in range(2)]
        print("B=%d H=%d: velocity rel-L2 %.3g; worst block %.3g" % (B, H, err, max(blk)))
        assert err <= 1e-3
        assert max(blk) <= 2e-3
    finally:
        m.close()


def test_forward_bit_identical_and_graph(tsn, rt, orc, model):
    spec, m, w32 = model
    inp, dev = _io(tsn, rt, spec, seed=77)
    v1, v2, v3 = (rt.empty((spec.B, spec.La, spec.latent)) for _ in range(3))
    m.forward_ex(dev["z"], dev["t"], dev["text"], dev["pooled"], v1)
    m.forward_ex(dev["z"], dev["t"], dev["text"], dev["pooled"], v2)
    rt.sync()
    a, b = v1.numpy(), v2.numpy()
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    m.capture_forward(dev["z"], dev["t"], dev["text"], dev["pooled"], v3)
    for _ in range(3):
        m.replay()
        rt.sync()
        c = v3.numpy()
        assert np.array_equal(a.view(np.uint32), c.view(np.uint32))
        # eager work on the same buffers between replays
        m.forward_ex(dev["z"], dev["t"], dev["text"], dev["pooled"], v2)
        rt.sync()
    # scalar-t entry point (DitModel::forward signature) matches the device-t one
    m.forward(dev["z"], float(inp["t"][0]), dev["text"], dev["pooled"], v2)
    rt.sync()
    assert np.array_equal(a.view(np.uint32), v2.numpy().view(np.uint32))


def test_sampler_two_steps(tsn, rt, orc, model):
    spec, m, w32 = model
    inp, dev = _io(tsn, rt, spec, cfg_pairs=True)
    P = spec.B // 2
    x0 = inp["z"][0::2].copy()
    x = rt.array(x0)
    m.sample(x, dev["text"], dev["pooled"], 2, 5.0)
    rt.sync()
    out = x.numpy()
    ref = orc.dit_sample(spec, w32, x0, inp["text"], inp["pooled"], 2, 5.0)
    err = rel_l2(out - x0, ref - x0)
    print("sampler displacement rel-L2 %.3g" % err)
    assert out.shape == (P, spec.La, spec.latent)
    assert err <= 2e-3
    # graph-captured sampler reproduces the eager one bit for bit
    x2 = rt.array(x0)
    m.capture_sample(x2, dev["text"], dev["pooled"], 2, 5.0)
    m.replay()
    rt.sync()
    assert np.array_equal(out.view(np.uint32), x2.numpy().view(np.uint32))


@pytest.fixture(scope="module")
def bench_model(tsn, rt):
    """the weights the benchmark times: every weight N(0, 0.02) from seed 4242, q/k norm weights too"""
    spec = tsn.default_spec(2)
    w16 = tsn.synth_weights(spec, 4242, 0.0)
    m = tsn.DitModel(rt, spec)
    m.upload_weights(w16)
    yield spec, m, w16
    m.close()


def test_forward_on_bench_weights(tsn, rt, orc, bench_model):
    """one evaluation on exactly the weights and inputs of the benchmark (cond/uncond pair, seed 4242)"""
    spec, m, w16 = bench_model
    inp, dev = _io(tsn, rt, spec, cfg_pairs=True)
    nblk = spec.n_joint + spec.n_fused
    v = rt.empty((spec.B, spec.La, spec.latent))
    taps = rt.empty((nblk, spec.B, spec.La + spec.Lt, spec.H))
    m.forward_ex(dev["z"], dev["t"], dev["text"], dev["pooled"], v, taps)
    rt.sync()
    vr, tr, _ = orc.dit_forward(spec, tsn.bf16_to_f32(w16), inp["z"], inp["t"], inp["text"], inp["pooled"], taps=True)
    err = rel_l2(v.numpy(), vr)
    tg = taps.numpy()
    blk = max(rel_l2(tg[i], tr[i]) for i in range(nblk))
    print("bench weights: velocity rel-L2 %.3g, worst block %.3g" % (err, blk))
    assert err <= 1e-3 and blk <= 2e-3


def test_sampler_24_steps_against_fixture(tsn, rt, bench_model):
    """The whole 24-step CFG sampler at 8 s on the benchmark's weights and inputs against the oracle's
    final latent (tests/golden/sampler_8s_24steps.npz, written by make_sampler_golden.py): the
    displacement x - z0 within rel-L2 2e-3, eager and graph-captured runs bit-identical."""
    import os
    spec, m, w16 = bench_model
    g = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "sampler_8s_24steps.npz"))
    inp, dev = _io(tsn, rt, spec, cfg_pairs=True)
    assert int(g["seeds"][0]) == 4242 and int(g["seeds"][1]) == 24 and float(g["norm_mean"]) == 0.0
    assert np.isclose(tsn.bf16_to_f32(w16).astype(np.float64).sum(), float(g["w_checksum"]), rtol=0, atol=1e-6)
    x0 = inp["z"][0::2].copy()
    assert np.array_equal(x0, g["x0"])
    x = rt.array(x0)
    m.sample(x, dev["text"], dev["pooled"], 24, float(g["cfg"]))
    rt.sync()
    out = x.numpy()
    err = rel_l2(out - x0, g["x"] - x0)
    print("24-step sampler: displacement rel-L2 %.3g, final latent rel-L2 %.3g" % (err, rel_l2(out, g["x"])))
    assert err <= 2e-3
    x2 = rt.array(x0)
    m.capture_sample(x2, dev["text"], dev["pooled"], 24, float(g["cfg"]))
    m.replay()
    rt.sync()
    assert np.array_equal(out.view(np.uint32), x2.numpy().view(np.uint32))


def test_replay_refused_after_sampler_reallocation(tsn, rt, model):
    """A captured sampler addresses the step schedule and conditioning buffers. An eager sampler run
    with another step count reallocates them, so the old graph must refuse to replay (state error)
    instead of writing into freed memory; a new capture then matches the eager run bit for bit."""
    spec, m, _ = model
    inp, dev = _io(tsn, rt, spec, seed=5, cfg_pairs=True)
    x0 = inp["z"][0::2].copy()
    xa = rt.array(x0)
    m.capture_sample(xa, dev["text"], dev["pooled"], 2, 5.0)
    xb = rt.array(x0)
    m.sample(xb, dev["text"], dev["pooled"], 3, 5.0)
    rt.sync()
    with pytest.raises(tsn.TsnError) as e:
        m.replay()
    assert e.value.code == 5
    eager3 = xb.numpy()
    xc = rt.array(x0)
    m.capture_sample(xc, dev["text"], dev["pooled"], 3, 5.0)
    m.replay()
    rt.sync()
    assert np.array_equal(xc.numpy().view(np.uint32), eager3.view(np.uint32))
