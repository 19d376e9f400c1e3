"""Frozen vectors: tests/golden/dit_small.npz holds the outputs of a small DiT evaluation (B=2,
La=12, Lt=5, H=256, one joint + one fused block) computed by an independent float64 NumPy
restatement of the graph (tests/golden/make_golden.py). The reference ships no vectors for this
path; these pin the oracle and the GPU path to one fixed answer that neither of them produced.
"""
import os

import numpy as np
import pytest

from conftest import rel_l2

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "dit_small.npz")


def _load(tsn):
    g = np.load(GOLDEN)   # plain arrays only (allow_pickle stays False)
    spec = tsn.DitSpec(**{k: (float(v) if k in ("rope_theta", "t_max_period", "ln_eps", "rms_eps") else int(v))
                          for k, v in zip(g["spec_keys"], g["spec_vals"])})
    wseed, iseed = (int(x) for x in g["seeds"])
    w16 = tsn.synth_weights(spec, wseed, float(g["norm_mean"]))
    inp = tsn.synth_inputs(spec, iseed, cfg_pairs=False)
    # the generator still produces the inputs the vectors were computed from
    assert np.isclose(tsn.bf16_to_f32(w16).astype(np.float64).sum(), float(g["w_checksum"]), rtol=0, atol=1e-6)
    assert np.isclose(inp["z"].astype(np.float64).sum(), float(g["z_checksum"]), rtol=0, atol=1e-9)
    return g, spec, w16, inp


def test_oracle_matches_golden(tsn, orc):
    g, spec, w16, inp = _load(tsn)
    v, taps, _ = orc.dit_forward(spec, tsn.bf16_to_f32(w16), inp["z"], inp["t"], inp["text"], inp["pooled"], taps=True)
    assert rel_l2(v, g["v"]) < 1e-5
    for i in range(taps.shape[0]):
        assert rel_l2(taps[i], g["taps"][i]) < 1e-5


@pytest.mark.gpu
def test_gpu_matches_golden(tsn, rt):
    g, spec, w16, inp = _load(tsn)
    m = tsn.DitModel(rt, spec)
    try:
        m.upload_weights(w16)
        dev = {k: rt.array(x) for k, x in inp.items()}
        nblk = spec.n_joint + spec.n_fused
        v = rt.empty((spec.B, spec.La, spec.latent))
        taps = rt.empty((nblk, spec.B, spec.La + spec.Lt, spec.H))
        m.forward_ex(dev["z"], dev["t"], dev["text"], dev["pooled"], v, taps)
        rt.sync()
        err = rel_l2(v.numpy(), g["v"])
        tg = taps.numpy()
        blk = [rel_l2(tg[i], g["taps"][i]) for i in range(nblk)]
        print("golden: velocity rel-L2 %.3g, blocks %s" % (err, ["%.3g" % e for e in blk]))
        assert err <= 1e-3
        assert max(blk) <= 2e-3
    finally:
        m.close()
