"""Size-independent properties of the DiT path at full size (B=2, La=256, Lt=141, H=1024), checked
on the GPU without the oracle:

  * zero gates (modulation chunks 2 and 5, weights and bias) make every block the identity, bit
    for bit: the gated residual adds exactly zero;
  * no cross-sample mixing: changing sample 0's inputs leaves sample 1's velocity bit-identical
    (same shapes, so the same tiling and split-K);
  * a zero output layer makes the velocity the output bias, and the 24-step Euler sampler then
    moves every latent by exactly -bias (t runs from 1 to 0), whatever the CFG scale.
"""
import numpy as np
import pytest

from conftest import rel_l2

pytestmark = pytest.mark.gpu


def _weights(tsn, spec, seed=4242):
    w16 = tsn.synth_weights(spec, seed, 1.0)
    idx = {name: (off, n) for name, n, off in tsn.manifest(spec)}
    return w16, idx


def test_zero_gates_make_blocks_identity(tsn, rt):
    spec = tsn.default_spec(1)
    H = spec.H
    w16, idx = _weights(tsn, spec)
    prefixes = ["joint_blocks.0.latent_block", "joint_blocks.0.text_block", "fused_blocks.0"]
    for p in prefixes:
        ow, _ = idx[p + ".adaLN_modulation.1.weight"]
        ob, _ = idx[p + ".adaLN_modulation.1.bias"]
        for gate in (2, 5):
            w16[ow + gate * H * H: ow + (gate + 1) * H * H] = 0
            w16[ob + gate * H: ob + (gate + 1) * H] = 0
    m = tsn.DitModel(rt, spec)
    try:
        m.upload_weights(w16)
        S = spec.La + spec.Lt
        X = tsn.synth_normal_f32(5, tsn.IDX_X, 0.0, 1.0, (spec.B, S, H))
        g = tsn.synth_normal_f32(5, tsn.IDX_G, 0.0, 1.0, (spec.B, H))
        gd = rt.array(g)
        for kind in ("joint", "fused"):
            Xd = rt.array(X)
            (m.joint_block if kind == "joint" else m.fused_block)(0, Xd, gd)
            rt.sync()
            assert np.array_equal(Xd.numpy().view(np.uint32), X.view(np.uint32)), kind
    finally:
        m.close()


def test_samples_do_not_mix(tsn, rt):
    # same shapes (so the same tiling and split-K), different inputs for sample 0 only: sample 1's
    # velocity must not change by a single bit
    spec = tsn.default_spec(1)
    w16, _ = _weights(tsn, spec)
    a = tsn.synth_inputs(spec, 31, cfg_pairs=False)
    b = tsn.synth_inputs(spec, 32, cfg_pairs=False)
    for k in a:
        b[k][1:] = a[k][1:]
    m = tsn.DitModel(rt, spec)
    try:
        m.upload_weights(w16)
        out = []
        for inp in (a, b):
            dev = {k: rt.array(x) for k, x in inp.items()}
            v = rt.empty((spec.B, spec.La, spec.latent))
            m.forward_ex(dev["z"], dev["t"], dev["text"], dev["pooled"], v)
            rt.sync()
            out.append(v.numpy())
        assert not np.array_equal(out[0][0], out[1][0])          # sample 0 did change
        assert np.array_equal(out[0][1].view(np.uint32), out[1][1].view(np.uint32))
    finally:
        m.close()


def test_constant_velocity_sampler_closed_form(tsn, rt):
    spec = tsn.default_spec(2)
    w16, idx = _weights(tsn, spec)
    ow, n = idx["final_layer.linear.weight"]
    w16[ow:ow + n] = 0
    ob, nb = idx["final_layer.linear.bias"]
    bias = np.linspace(-1.0, 1.0, nb).astype(np.float32)
    w16[ob:ob + nb] = (bias.view(np.uint32) >> 16).astype(np.uint16)   # exact in bf16 (truncation
    bias = tsn.bf16_to_f32(w16[ob:ob + nb])                            # is recomputed as the value)
    m = tsn.DitModel(rt, spec)
    try:
        m.upload_weights(w16)
        inp = tsn.synth_inputs(spec, 8, cfg_pairs=True)
        dev = {k: rt.array(x) for k, x in inp.items()}
        x0 = inp["z"][0::2].copy()
        x = rt.array(x0)
        m.sample(x, dev["text"], dev["pooled"], 24, 5.0)
        rt.sync()
        out = x.numpy()
        # 24 steps of dt = -1/24 with v = bias in both arms (cfg irrelevant): x0 - bias up to f32 rounding
        assert np.abs(out - (x0 - bias)).max() <= 1e-5 * (1.0 + np.abs(x0).max())
    finally:
        m.close()
