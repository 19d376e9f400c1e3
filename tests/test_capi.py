"""C ABI of libtsn without a GPU: the library loads, exports every entry point include/tsn.h
declares, agrees with the oracle on the weight manifest, reproduces the specified synthetic-data
generator, and reports errors on bad input (no compute call needs a device here)."""
import ctypes
import os
import re

import numpy as np
import pytest

from conftest import ROOT


def declared_symbols():
    text = open(os.path.join(ROOT, "include", "tsn.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(tsn_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol(tsn):
    L = tsn.lib()
    syms = declared_symbols()
    assert len(syms) >= 40
    missing = [s for s in syms if not hasattr(L, s)]
    assert not missing, missing


def test_python_binding_covers_every_symbol(tsn):
    bound = set(tsn._SIGS) | {"tsn_last_error", "tsn_last_gpu_ms", "tsn_version"}
    assert set(declared_symbols()) <= bound


def test_manifest_matches_oracle(tsn, orc):
    for wl in (0, 1, 3, 4):
        spec = tsn.default_spec(wl)
        assert tsn.manifest(spec) == orc.manifest(spec.as_dict())
    spec = tsn.default_spec(1)
    assert tsn.manifest_total(spec) == 649757248
    assert len(tsn.manifest(spec)) == 290


def _mix64(z):
    z = (z + np.uint64(0x9E3779B97F4A7C15))
    z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
    z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return z ^ (z >> np.uint64(31))


def _synth_normal_ref(seed, index, mean, std, n):
    """independent numpy restatement of the generator specified in csrc/synth.cpp"""
    with np.errstate(over="ignore"):
        key = _mix64(_mix64(np.uint64(seed)) ^ (np.uint64(index) * np.uint64(0xD1B54A32D192ED03)))
        i = np.arange(n, dtype=np.uint64)
        p = i >> np.uint64(1)
        def uni(j):
            return ((_mix64(key ^ _mix64(j)) >> np.uint64(11)).astype(np.float64) + 0.5) * 2.0 ** -53
        u1, u2 = uni(np.uint64(2) * p), uni(np.uint64(2) * p + np.uint64(1))
    rad = np.sqrt(-2.0 * np.log(u1))
    ang = 2 * np.pi * u2
    z = np.where(i & np.uint64(1), rad * np.sin(ang), rad * np.cos(ang))
    return (mean + std * z).astype(np.float32)


def test_synth_generator_known_answers(tsn):
    ref = _synth_normal_ref(4242, 1000, 0.0, 1.0, 4096)
    got = tsn.synth_normal_f32(4242, 1000, 0.0, 1.0, (4096,))
    assert np.abs(got.astype(np.float64) - ref).max() <= 1e-6
    assert (got == ref).mean() > 0.999
    # bf16 rounding: nearest-even of the f32 value
    w = tsn.synth_normal_bf16(4242, 3, 0.0, 0.02, (4096,))
    f = _synth_normal_ref(4242, 3, 0.0, 0.02, 4096)
    u = f.view(np.uint32).astype(np.uint64)
    rne = ((u + np.uint64(0x7FFF) + ((u >> np.uint64(16)) & np.uint64(1))) >> np.uint64(16)).astype(np.uint16)
    assert (w == rne).mean() > 0.999
    # moments
    big = tsn.synth_normal_f32(1, 1, 0.0, 1.0, (1 << 18,))
    assert abs(big.mean()) < 0.01 and abs(big.std() - 1) < 0.01
    u01 = tsn.synth_uniform_f32(1, 2, 0.0, 1.0, (1 << 16,))
    assert u01.min() > 0 and u01.max() < 1 and abs(u01.mean() - 0.5) < 0.01


def test_synth_weights_layout(tsn):
    spec = tsn.default_spec(1).copy(La=8, Lt=4, n_joint=1, n_fused=1)
    w = tsn.synth_weights(spec, 4242, 1.0)
    man = tsn.manifest(spec)
    for name, n, off in man:
        vals = tsn.bf16_to_f32(w[off:off + n])
        if "norm.weight" in name:
            assert abs(vals.mean() - 1.0) < 0.02
        else:
            assert abs(vals.mean()) < 0.01 and 0.015 < vals.std() < 0.025
    # tensor k is drawn from stream (seed, k): regenerating one tensor alone gives the same bits
    name, n, off = man[7]
    alone = tsn.synth_normal_bf16(4242, 7, 0.0, 0.02, (n,))
    assert np.array_equal(alone, w[off:off + n])


def test_error_paths_without_gpu(tsn):
    L = tsn.lib()
    h = ctypes.c_void_p()
    rc = L.tsn_runtime_create(0, ctypes.byref(h))
    if rc == 0:
        L.tsn_runtime_destroy(h)
        pytest.skip("a GPU is present")
    assert rc == 2 and L.tsn_last_error()
    assert L.tsn_alloc(None, 16, ctypes.byref(h)) == 1
    assert L.tsn_gemm(None, 1, None, None, 0, None, 0, None, 1, 1, 8, 0, 0, 0) == 1
    s = tsn.DitSpec()
    assert L.tsn_dit_default_spec(7, ctypes.byref(s)) == 1
    assert L.tsn_dit_default_spec(1, ctypes.byref(s)) == 0 and s.La == 256 and s.Lt == 141
    assert L.tsn_dit_manifest_entry(ctypes.byref(s), 100000, None, 0, None, None) == 1
    with pytest.raises(tsn.TsnError):
        tsn.call("tsn_dit_forward", None, None, 0.5, None, None, None)


def test_oracle_builds_and_reports_threads(orc):
    assert orc.num_threads() >= 1


def test_ref_manifest_matches_oracle(tsn, orc):
    spec = tsn.ref_spec_for_duration(8, 2)
    # src/models.h:20-22 and src/pipeline.cpp:81-83 at 8 s
    assert (spec.T, spec.C, spec.TS, spec.H, spec.F, spec.n_joint, spec.n_fused) == (172, 64, 154, 1024, 2816, 7, 14)
    assert tsn.ref_spec_for_duration(30, 2).T == 646
    man = tsn.ref_manifest(spec)
    assert man == orc.ref_manifest(spec.as_dict())
    assert tsn.ref_manifest_total(spec) == man[-1][1] + man[-1][2]
    names = [n for n, _, _ in man]
    # the pre-only last joint block has no clip/text out-proj or FFN, 2 modulation chunks
    assert "joint_blocks.6.clip_block.linear1.weight" not in names
    assert "joint_blocks.6.latent_block.linear1.weight" in names
    d = dict((n, k) for n, k, _ in man)
    assert d["joint_blocks.6.text_block.adaLN_modulation.1.weight"] == 2 * 1024 * 1024
    assert d["final_layer.conv.weight"] == 64 * 1024 * 7
    small = spec.copy(n_joint=2, n_fused=1, T=6, C=3, TS=4, H=256, NH=4, F=128, latent=32)
    assert tsn.ref_manifest(small) == orc.ref_manifest(small.as_dict())


def test_ref_spec_errors(tsn):
    spec = tsn.ref_spec_for_duration(8, 2)
    with pytest.raises(RuntimeError):
        tsn.ref_spec_for_duration(0, 2)
    with pytest.raises(RuntimeError):
        tsn.ref_spec_for_duration(8, 3)   # batch must be 1, 2, 4, 8 or 16
    rt_null = ctypes.c_void_p()
    h = ctypes.c_void_p()
    assert tsn.lib().tsn_refdit_create(rt_null, ctypes.byref(spec), ctypes.byref(h)) == 1
    assert tsn.lib().tsn_refdit_replay(None) == 1


def test_cond_manifest_matches_oracle(tsn, orc):
    spec = tsn.cond_spec_for_duration(8)
    assert (spec.H, spec.F, spec.T, spec.C, spec.sync_S, spec.TS) == (1024, 2816, 172, 64, 192, 154)
    assert (spec.sync_dim, spec.clip_dim, spec.text_dim, spec.gtext_dim) == (768, 1024, 2048, 1024)
    assert tsn.cond_manifest(spec) == orc.cond_manifest(spec.as_dict())
    small = spec.copy(H=256, F=128, sync_dim=64, clip_dim=128, text_dim=192, gtext_dim=32)
    assert tsn.cond_manifest(small) == orc.cond_manifest(small.as_dict())


def test_vae_manifest_matches_oracle(tsn, orc):
    spec = tsn.vae_spec_for_duration(8)
    # src/models.h:16-21 and src/vae.cpp:20 at 8 s: T = 172 latent rows, hop 2048
    d = spec.as_dict()
    assert (d["T"], d["latent"], d["width"], d["stride"], d["kt"], d["out_ch"]) == \
        (172, 64, [2048, 1024, 512, 256, 128, 128], [8, 8, 4, 4, 2], [16, 16, 8, 8, 4], 2)
    assert tsn.vae_audio_len(spec) == 172 * 2048 == orc.vae_audio_len(d)
    assert tsn.vae_manifest(spec) == orc.vae_manifest(d)
    small = spec.copy(T=5, width=[128, 64, 64, 64, 64, 64], stride=[2, 4, 2, 2, 2], kt=[4, 8, 4, 4, 4])
    assert tsn.vae_manifest(small) == orc.vae_manifest(small.as_dict())


def test_vae_synth_weights_layout(tsn):
    spec = tsn.vae_spec_for_duration(1).copy(width=[256, 128, 128, 64, 64, 64])
    w = tsn.vae_synth_weights(spec, 7)
    man = tsn.vae_manifest(spec)
    assert w.size == man[-1][1] + man[-1][2]
    for name, n, off in man:
        x = w[off:off + n].astype(np.float64)
        if name.endswith(".alpha") or name.endswith(".beta"):
            want = 0.1
        elif name.endswith(".bias"):
            want = 0.02
        else:
            layer = int(name.split(".")[2])
            oc = spec.width[0] if layer == 0 else spec.out_ch if layer == 7 else spec.width[layer]
            want = 1.0 / np.sqrt(n / oc) * (0.5 if name.endswith(".layers.3.weight") else 1.0)
        if n >= 1000:
            assert abs(x.std() / want - 1) < 0.1, name
    # each tensor is its own stream of the generator: the same seed reproduces it alone
    name, n, off = man[4]
    assert name == "decoder.layers.1.layers.1.weight"
    alone = np.empty(n, np.float32)
    tsn.call("tsn_synth_normal_f32", 7, 4, 0.0, 1.0 / np.sqrt(n / spec.width[1]), n, tsn.ptr(alone))
    assert np.array_equal(alone, w[off:off + n])


def test_vae_spec_from_gguf(tsn, tmp_path):
    """widths from the conv shapes (ne = K, IC, OC), transposed-conv kernels from ne[0]"""
    from gguf_writer import F32, write
    path = str(tmp_path / "v.gguf")
    w = [128, 64, 64, 64, 64, 64]
    kt = [16, 16, 8, 8, 6]
    tensors = [("decoder.layers.0.weight", (7, 64, w[0]), F32, np.zeros(7 * 64 * w[0], np.float32))]
    for n in range(5):
        shape = (kt[n], w[n], w[n + 1])
        tensors.append(("decoder.layers.%d.layers.1.weight" % (n + 1), shape, F32,
                        np.zeros(int(np.prod(shape)), np.float32)))
    tensors.append(("decoder.layers.7.weight", (7, 64, 2), F32, np.zeros(7 * 64 * 2, np.float32)))
    write(path, tensors)
    s = tsn.vae_spec_from_gguf(path, T=11)
    assert s.as_dict() == dict(T=11, latent=64, width=w, stride=[8, 8, 4, 4, 2], kt=kt, out_ch=2)
    # a transposed-conv kernel that is not a multiple of its stride is rejected
    tensors[1] = ("decoder.layers.1.layers.1.weight", (20, w[0], w[1]), F32, np.zeros(20 * w[0] * w[1], np.float32))
    write(path, tensors)
    with pytest.raises(RuntimeError):
        tsn.vae_spec_from_gguf(path, T=11)


def test_model_wrappers_check_array_sizes(tsn):
    """DitModel / RefDitModel refuse device arrays shorter than the spec needs before calling the
    library (a short buffer would otherwise be an out-of-bounds device access)"""
    class Fake:
        def __init__(self, n, itemsize=4):
            self.nbytes, self.p = n * itemsize, None

    spec = tsn.default_spec(1)
    m = tsn.DitModel.__new__(tsn.DitModel)
    m.spec, m.h = spec, None
    B, La, Lt, H, L = spec.B, spec.La, spec.Lt, spec.H, spec.latent
    ok = dict(z=Fake(B * La * L), text=Fake(B * Lt * H), pooled=Fake(B * H), v=Fake(B * La * L))
    for k in ok:
        bad = dict(ok, **{k: Fake(1)})
        with pytest.raises(ValueError):
            m.forward(bad["z"], 0.5, bad["text"], bad["pooled"], bad["v"])
    with pytest.raises(ValueError):
        m.sample(Fake(B * La * L // 2 - 1), ok["text"], ok["pooled"], 2, 5.0)
    with pytest.raises(ValueError):
        m.joint_block(0, Fake(B * (La + Lt) * H - 1), Fake(B * H))
    with pytest.raises(TypeError):
        m.forward(np.zeros(4), 0.5, ok["text"], ok["pooled"], ok["v"])
    rs = tsn.ref_spec_for_duration(8, 2)
    r = tsn.RefDitModel.__new__(tsn.RefDitModel)
    r.spec, r.h = rs, None
    good = dict(x=Fake(rs.B * rs.T * rs.latent), clip_pp=Fake(rs.B * rs.C * rs.H), text_pp=Fake(rs.B * rs.TS * rs.H),
                gcmlp=Fake(rs.B * rs.H), sync_gather=Fake(rs.B * rs.T * rs.H), flow=Fake(rs.B * rs.T * rs.latent))
    for k in good:
        bad = dict(good, **{k: Fake(3)})
        with pytest.raises(ValueError):
            r.forward(bad["x"], 0.5, bad["clip_pp"], bad["text_pp"], bad["gcmlp"], bad["sync_gather"], bad["flow"])


def test_sampler_fixture_inputs(tsn):
    """tests/golden/sampler_8s_24steps.npz still describes what the generator produces (the GPU test
    compares the 24-step sampler with it)"""
    g = np.load(os.path.join(ROOT, "tests", "golden", "sampler_8s_24steps.npz"))
    spec = tsn.default_spec(2)
    seed, steps = (int(v) for v in g["seeds"])
    inp = tsn.synth_inputs(spec, seed, cfg_pairs=True)
    assert np.array_equal(inp["z"][0::2], g["x0"])
    assert np.isclose(inp["text"].astype(np.float64).sum(), float(g["text_checksum"]), rtol=0, atol=1e-6)
    assert np.isclose(inp["pooled"].astype(np.float64).sum(), float(g["pooled_checksum"]), rtol=0, atol=1e-9)
    w = tsn.bf16_to_f32(tsn.synth_weights(spec, seed, float(g["norm_mean"])))
    assert np.isclose(w.astype(np.float64).sum(), float(g["w_checksum"]), rtol=0, atol=1e-6)
    assert steps == 24 and g["x"].shape == (1, spec.La, spec.latent) and np.isfinite(g["x"]).all()
