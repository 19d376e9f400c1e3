"""GPU parity of the reference's VAE decoder (tsn_vae_*: VaeModel::decode, src/vae.cpp:17-86) against
the oracle (oracle/oracle_vae.cpp), with the specified synthetic f32 weights:

  * the reference's widths (2048 .. 128, strides 8, 8, 4, 4, 2) at T = 3 latent rows, and narrow
    widths at an odd T = 9 and at a T = 1 latent, audio within rel-L2 1e-4;
  * 8 s (T = 172, 352,256 samples per channel): the samples of latent rows 85..94 of the full decode
    against the oracle's decode of the 32-row latent window 74..105 (the decoder's receptive field is
    about 10 latent rows, so the window's zero padding does not reach them), within 1e-4; the whole
    output finite;
  * bit-identical reruns, hipGraph replay equal to the eager decode;
  * a checkpoint load (GGUF, F32 tensors) decodes bit-identically to the flat upload.
"""
import numpy as np
import pytest

from conftest import rel_l2, rng

pytestmark = pytest.mark.gpu

TOL = 1e-4


def _decode(tsn, rt, m, latent):
    spec = m.spec
    z = rt.array(np.ascontiguousarray(latent, np.float32))
    a = rt.empty((tsn.vae_audio_len(spec), spec.out_ch))
    m.decode(z, a)
    rt.sync()
    return a.numpy()


def _model(tsn, rt, spec, seed):
    w = tsn.vae_synth_weights(spec, seed)
    m = tsn.VaeModel(rt, spec)
    m.upload_weights(w)
    return m, w


@pytest.mark.parametrize("case", ["ref_widths_T3", "narrow_T9", "narrow_T1"])
def test_vae_decode_parity(tsn, rt, orc, case):
    spec = tsn.vae_spec_for_duration(8)
    if case == "ref_widths_T3":
        spec = spec.copy(T=3)
    elif case == "narrow_T9":
        spec = spec.copy(T=9, width=[256, 128, 128, 64, 64, 64])
    else:
        spec = spec.copy(T=1, width=[128, 64, 64, 64, 64, 64], stride=[2, 4, 2, 2, 2], kt=[4, 8, 4, 4, 4])
    m, w = _model(tsn, rt, spec, 11)
    try:
        latent = rng(5).standard_normal((spec.T, spec.latent)).astype(np.float32)
        a = _decode(tsn, rt, m, latent)
        ref = orc.vae_decode(spec.as_dict(), w, latent)
        err = rel_l2(a, ref)
        print("vae %s: audio %s rel-L2 %.3g, max |ref| %.3g" % (case, a.shape, err, np.abs(ref).max()))
        assert a.shape == ref.shape
        assert err <= TOL
        again = _decode(tsn, rt, m, latent)
        assert np.array_equal(again.view(np.uint32), a.view(np.uint32))
    finally:
        m.close()


def test_vae_8s_window_and_graph(tsn, rt, orc):
    spec = tsn.vae_spec_for_duration(8)
    m, w = _model(tsn, rt, spec, 12)
    try:
        latent = rng(6).standard_normal((spec.T, spec.latent)).astype(np.float32)
        a = _decode(tsn, rt, m, latent)
        assert a.shape == (172 * 2048, 2) and np.isfinite(a).all()
        lo, n, margin = 74, 32, 11
        ref = orc.vae_decode(spec.copy(T=n).as_dict(), w, latent[lo:lo + n])
        hop = 2048
        got = a[(lo + margin) * hop:(lo + n - margin) * hop]
        want = ref[margin * hop:(n - margin) * hop]
        err = rel_l2(got, want)
        print("vae 8 s: interior latent rows %d..%d rel-L2 %.3g" % (lo + margin, lo + n - margin - 1, err))
        assert err <= TOL
        # graph replay of the same decode equals the eager one
        z = rt.array(latent)
        out = rt.empty((tsn.vae_audio_len(spec), spec.out_ch))
        m.capture_decode(z, out)
        for _ in range(2):
            m.replay()
        rt.sync()
        assert np.array_equal(out.numpy().view(np.uint32), a.view(np.uint32))
    finally:
        m.close()


def test_vae_gguf_load(tsn, rt, tmp_path):
    from gguf_writer import F32, write
    spec = tsn.vae_spec_for_duration(1).copy(T=4, width=[128, 64, 64, 64, 64, 64])
    w = tsn.vae_synth_weights(spec, 13)
    tensors = []
    for name, n, off in tsn.vae_manifest(spec):
        tensors.append((name, (n,), F32, w[off:off + n]))
    # conv weights as 3-d tensors (K, IC, OC) like the checkpoint
    shapes = {"decoder.layers.0.weight": (7, spec.latent, spec.width[0]),
              "decoder.layers.7.weight": (7, spec.width[5], spec.out_ch)}
    for k in range(5):
        shapes["decoder.layers.%d.layers.1.weight" % (k + 1)] = (spec.kt[k], spec.width[k], spec.width[k + 1])
    tensors = [(nm, shapes.get(nm, ne), t, v) for nm, ne, t, v in tensors]
    path = str(tmp_path / "vae.gguf")
    write(path, tensors)
    gspec = tsn.vae_spec_from_gguf(path, T=4)
    assert gspec.as_dict() == spec.as_dict()
    a_m, _ = _model(tsn, rt, spec, 13)
    b_m = tsn.VaeModel(rt, gspec)
    try:
        b_m.load_gguf(path)
        latent = rng(7).standard_normal((spec.T, spec.latent)).astype(np.float32)
        a = _decode(tsn, rt, a_m, latent)
        b = _decode(tsn, rt, b_m, latent)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    finally:
        a_m.close()
        b_m.close()
