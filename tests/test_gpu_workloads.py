"""GPU parity at the two other full-size workloads, against the CPU oracle on identical seeded
weights and inputs:

  * 30 s audio: La=960, Lt=141 (S=1101 joint tokens), B=2 — long attention and long convs;
  * batch 16: 8 prompts x CFG at 8 s (La=256, Lt=141) — large-M GEMMs, 16-row GEMVs.

Bars as for the 8 s evaluation: velocity rel-L2 <= 1e-3, every block output <= 2e-3; the batch-16
sampler step (8 cond/uncond pairs), and the whole 24-step samplers of the 30 s clip and of the
batch-16 workload (eight prompts from seeds 1..8, against committed oracle fixtures) <= 2e-3 on the
displacement, for every prompt.
"""
import numpy as np
import pytest

from conftest import rel_l2

pytestmark = pytest.mark.gpu


def _model(tsn, rt, workload):
    spec = tsn.default_spec(workload)
    w16 = tsn.synth_weights(spec, 4242, 1.0)
    m = tsn.DitModel(rt, spec)
    m.upload_weights(w16)
    return spec, m, tsn.bf16_to_f32(w16)


@pytest.mark.parametrize("workload", [3, 4])
def test_forward_parity_and_taps(tsn, rt, orc, workload):
    spec, m, w32 = _model(tsn, rt, workload)
    try:
        inp = tsn.synth_inputs(spec, 4242 + workload, cfg_pairs=True)
        dev = {k: rt.array(v) for k, v in inp.items()}
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
        print("workload %d (B=%d La=%d): velocity rel-L2 %.3g; worst block %.3g"
              % (workload, spec.B, spec.La, err, max(blk)))
        assert err <= 1e-3
        assert max(blk) <= 2e-3
        # per sample: no arm may hide behind the others
        for b in range(spec.B):
            assert rel_l2(v.numpy()[b], vr[b]) <= 1e-3
    finally:
        m.close()


def test_batch16_sampler_step_and_graph_replays(tsn, rt, orc):
    spec, m, w32 = _model(tsn, rt, 4)
    try:
        inp = tsn.synth_inputs(spec, 9, cfg_pairs=True)
        dev = {k: rt.array(v) for k, v in inp.items()}
        x0 = inp["z"][0::2].copy()
        x = rt.array(x0)
        m.sample(x, dev["text"], dev["pooled"], 1, 5.0)
        rt.sync()
        out = x.numpy()
        ref = orc.dit_sample(spec, w32, x0, inp["text"], inp["pooled"], 1, 5.0)
        err = rel_l2(out - x0, ref - x0)
        print("batch-16 sampler step displacement rel-L2 %.3g" % err)
        assert out.shape == (spec.B // 2, spec.La, spec.latent)
        assert err <= 2e-3
        for p in range(spec.B // 2):
            assert rel_l2(out[p] - x0[p], ref[p] - x0[p]) <= 2e-3
        # graph replays, with eager work of the same model between them, reproduce the eager result
        x2 = rt.array(x0)
        m.capture_sample(x2, dev["text"], dev["pooled"], 1, 5.0)
        scratch = rt.empty((spec.B, spec.La, spec.latent))
        for _ in range(3):
            x2.upload(x0)
            m.replay()
            rt.sync()
            assert np.array_equal(out.view(np.uint32), x2.numpy().view(np.uint32))
            m.forward_ex(dev["z"], dev["t"], dev["text"], dev["pooled"], scratch)
            rt.sync()
    finally:
        m.close()


def test_sampler_30s_24_steps_against_fixture(tsn, rt):
    """The whole 24-step CFG sampler on the 30 s workload (La=960, S=1101, one prompt as a
    cond/uncond pair) on the benchmark's weights (every weight N(0, 0.02), seed 4242) against the
    oracle's final latent (tests/golden/sampler_30s_24steps.npz, written by make_sampler_golden.py
    30s; the oracle needs about 42 minutes for it): displacement x - z0 within rel-L2 2e-3, eager
    and graph-captured runs bit-identical."""
    import os
    spec = tsn.default_spec(3)
    g = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "sampler_30s_24steps.npz"))
    assert int(g["seeds"][0]) == 4242 and int(g["seeds"][1]) == 24 and float(g["norm_mean"]) == 0.0
    w16 = tsn.synth_weights(spec, 4242, 0.0)
    assert np.isclose(tsn.bf16_to_f32(w16).astype(np.float64).sum(), float(g["w_checksum"]), rtol=0, atol=1e-6)
    m = tsn.DitModel(rt, spec)
    try:
        m.upload_weights(w16)
        inp = tsn.synth_inputs(spec, 4242, cfg_pairs=True)
        dev = {k: rt.array(v) for k, v in inp.items()}
        x0 = inp["z"][0::2].copy()
        assert np.array_equal(x0, g["x0"])
        x = rt.array(x0)
        m.sample(x, dev["text"], dev["pooled"], 24, float(g["cfg"]))
        rt.sync()
        out = x.numpy()
        err = rel_l2(out - x0, g["x"] - x0)
        print("30 s 24-step sampler: displacement rel-L2 %.3g, final latent rel-L2 %.3g" % (err, rel_l2(out, g["x"])))
        assert err <= 2e-3
        x2 = rt.array(x0)
        m.capture_sample(x2, dev["text"], dev["pooled"], 24, float(g["cfg"]))
        m.replay()
        rt.sync()
        assert np.array_equal(out.view(np.uint32), x2.numpy().view(np.uint32))
    finally:
        m.close()


def test_sampler_batch16_24_steps_against_fixture(tsn, rt):
    """The whole 24-step CFG sampler of the throughput batch: eight independent prompts as
    cond/uncond pairs (batch 16, La = 256, Lt = 141), prompt p's z0, text and pooled features from
    seed p + 1 (p = 0..7), on the benchmark's weights (every weight N(0, 0.02), seed 4242), against
    the oracle's final latents (tests/golden/sampler_b16_24steps.npz, written by
    make_sampler_golden.py b16; about 30 minutes of oracle time): the displacement x - z0 of every
    prompt within rel-L2 2e-3, eager and graph-captured runs bit-identical."""
    import os
    spec = tsn.default_spec(4)
    g = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "sampler_b16_24steps.npz"))
    seeds = [int(x) for x in g["prompt_seeds"]]
    assert seeds == list(range(1, 9)) and spec.B == 2 * len(seeds)
    assert int(g["seeds"][0]) == 4242 and int(g["seeds"][1]) == 24 and float(g["norm_mean"]) == 0.0
    w16 = tsn.synth_weights(spec, 4242, 0.0)
    assert np.isclose(tsn.bf16_to_f32(w16).astype(np.float64).sum(), float(g["w_checksum"]), rtol=0, atol=1e-6)
    inp = tsn.synth_prompt_inputs(spec, seeds)
    x0 = inp["z"][0::2].copy()
    assert np.allclose(x0.astype(np.float64).reshape(len(seeds), -1).sum(axis=1), g["x0_checksums"], rtol=0, atol=1e-9)
    assert np.isclose(inp["text"].astype(np.float64).sum(), float(g["text_checksum"]), rtol=0, atol=1e-6)
    m = tsn.DitModel(rt, spec)
    try:
        m.upload_weights(w16)
        dev = {k: rt.array(v) for k, v in inp.items()}
        x = rt.array(x0)
        m.sample(x, dev["text"], dev["pooled"], 24, float(g["cfg"]))
        rt.sync()
        out = x.numpy()
        ref = g["x"]
        errs = [rel_l2(out[p] - x0[p], ref[p] - x0[p]) for p in range(len(seeds))]
        print("batch-16 24-step sampler: displacement rel-L2 per prompt " + " ".join("%.3g" % e for e in errs))
        assert max(errs) <= 2e-3
        x2 = rt.array(x0)
        m.capture_sample(x2, dev["text"], dev["pooled"], 24, float(g["cfg"]))
        m.replay()
        rt.sync()
        assert np.array_equal(out.view(np.uint32), x2.numpy().view(np.uint32))
    finally:
        m.close()
