"""GGUF checkpoint reader (tsn_gguf_*, tsn_refdit_spec_from_gguf) on files written by
tests/gguf_writer.py — CPU only.

Checked: tensor names, types and dims (ne[0] fastest) at alignments 32 and 64; typed metadata
(integers, floats, strings, arrays skipped); dequantization with the reference's semantics
(src/gguf.cpp: F32 as is, BF16 exact, F16 and the Q8_0 block scale with subnormals flushed to
zero, Q8_0 = scale * int8), including known answers; the hyperparameters of a checkpoint
(src/dit.cpp:29-47); malformed files are rejected with an error.
"""
import os

import numpy as np
import pytest

import gguf_writer as gw
from conftest import rng


def _sample_tensors(r):
    sub = np.array([3e-6, -1e-7, 6e-5, 1.0, -2.5, 65504.0, 1e-3, 0.0] * 4, np.float32)   # f16 subnormals and edges
    return [
        ("a.f32", (5,), gw.F32, r.standard_normal(5).astype(np.float32)),
        ("b.f16", (8, 4), gw.F16, np.concatenate([sub, r.standard_normal(0)]).astype(np.float32)),
        ("c.bf16", (3, 2, 4), gw.BF16, r.standard_normal(24).astype(np.float32)),
        ("d.q8", (64, 2), gw.Q8_0, (0.1 * r.standard_normal(128)).astype(np.float32)),
        # Q8_0 block whose f16 scale is subnormal (max |x| ~ 1e-6): the block reads as zero
        ("e.q8small", (32,), gw.Q8_0, (1e-6 * np.linspace(-1, 1, 32)).astype(np.float32)),
    ]


@pytest.mark.parametrize("alignment", [32, 64])
def test_reader_tensors_and_values(tsn, tmp_path, alignment):
    r = rng(5)
    ts = _sample_tensors(r)
    meta = [("dit.hidden_dim", gw.KV_U32, 256), ("dit.rope_theta", gw.KV_F32, 500.0),
            ("general.name", gw.KV_STRING, "unit"), ("tok.list", gw.KV_ARRAY, (gw.KV_STRING, ["a", "bb", "ccc"])),
            ("num.list", gw.KV_ARRAY, (gw.KV_U32, [1, 2, 3])), ("flag", gw.KV_BOOL, True),
            ("big", gw.KV_U64, 1 << 40), ("ratio", gw.KV_F64, 0.125)]
    path = str(tmp_path / "t.gguf")
    dec = gw.write(path, ts, meta, alignment=alignment)
    g = tsn.Gguf(path)
    try:
        info = g.tensors()
        assert [(n, t, ne) for n, t, ne in info] == [(n, ty, ne) for n, ne, ty, _ in ts]
        for name, ne, ty, _ in ts:
            got = g.to_f32(name, int(np.prod(ne)))
            assert np.array_equal(got.view(np.uint32), dec[name].view(np.uint32)), name
        assert g.get_i64("dit.hidden_dim") == 256
        assert g.get_f64("dit.rope_theta") == 500.0
        assert g.get_i64("big") == 1 << 40
        assert g.get_f64("ratio") == 0.125
        assert g.get_i64("flag") == 1
        assert g.get_i64("missing", 7) == 7
    finally:
        g.close()


def test_known_answers(tsn, tmp_path):
    """hand-computed decodes: f16 0x0001 (subnormal) -> 0, 0x3C00 -> 1, 0xC000 -> -2; Q8_0 with
    scale 0x3800 (0.5) and q = [-3, 0, 5, ...] -> [-1.5, 0, 2.5, ...]"""
    path = str(tmp_path / "k.gguf")
    gw.write(path, [("x", (4,), gw.F32, np.zeros(4, np.float32))])
    # patch raw payloads by writing a file by hand: F16 and Q8_0 tensors with chosen bits
    import struct
    f16_bits = np.array([0x0001, 0x3C00, 0xC000, 0x8001], np.uint16)
    q = np.zeros(32, np.int8)
    q[:3] = [-3, 0, 5]
    q8 = struct.pack("<H", 0x3800) + q.tobytes()
    head = b"GGUF" + struct.pack("<IQQ", 3, 2, 0)
    infos = gw._s("h") + struct.pack("<IQIQ", 1, 4, gw.F16, 0)
    infos += gw._s("q") + struct.pack("<IQIQ", 1, 32, gw.Q8_0, 32)
    hdr = head + infos
    hdr += b"\0" * ((-len(hdr)) % 32)
    with open(path, "wb") as fh:
        fh.write(hdr + f16_bits.tobytes() + b"\0" * 24 + q8)
    g = tsn.Gguf(path)
    try:
        h = g.to_f32("h", 4)
        assert list(h) == [0.0, 1.0, -2.0, 0.0] and np.signbit(h[3])
        assert list(g.to_f32("q", 32)[:4]) == [-1.5, 0.0, 2.5, 0.0]
    finally:
        g.close()


def test_malformed_files_rejected(tsn, tmp_path):
    good = str(tmp_path / "g.gguf")
    gw.write(good, [("x", (8,), gw.F32, np.arange(8, dtype=np.float32))])
    data = open(good, "rb").read()
    cases = {"magic": b"GGUX" + data[4:], "version": data[:4] + b"\x01\0\0\0" + data[8:],
             "truncated": data[:40], "short data": data[:-4]}
    for what, blob in cases.items():
        p = str(tmp_path / ("bad_%s.gguf" % what.replace(" ", "_")))
        open(p, "wb").write(blob)
        with pytest.raises(RuntimeError):
            tsn.Gguf(p)
    with pytest.raises(RuntimeError):
        tsn.Gguf(str(tmp_path / "does_not_exist.gguf"))


def test_spec_from_gguf(tsn, tmp_path):
    """dit.* metadata and the SwiGLU width from joint_blocks.0.latent_block.ffn.w1.weight ne[2]"""
    path = str(tmp_path / "s.gguf")
    meta = [("dit.hidden_dim", gw.KV_U32, 512), ("dit.num_heads", gw.KV_U32, 8), ("dit.depth", gw.KV_U32, 5),
            ("dit.fused_depth", gw.KV_U32, 2), ("dit.latent_dim", gw.KV_U32, 128),
            ("dit.rope_theta", gw.KV_F32, 5000.0), ("dit.t_embed_max_period", gw.KV_F32, 2.0)]
    w1 = np.zeros(3 * 512 * 192, np.float32)
    gw.write(path, [("joint_blocks.0.latent_block.ffn.w1.weight", (3, 512, 192), gw.F32, w1)], meta)
    s = tsn.ref_spec_from_gguf(path, B=4, T=40, C=16, TS=10)
    assert (s.B, s.T, s.C, s.TS, s.H, s.NH, s.HD, s.F, s.latent, s.n_joint, s.n_fused) == \
        (4, 40, 16, 10, 512, 8, 64, 192, 128, 3, 2)
    assert s.rope_theta == 5000.0 and s.t_max_period == 2.0
    assert abs(s.ln_eps - 1e-5) < 1e-12 and abs(s.rms_eps - 1e-6) < 1e-13
    # defaults when the metadata is absent (the reference's: 1024, 16 heads, 21/14 blocks, 64, F 2816)
    gw.write(path, [("x", (4,), gw.F32, np.zeros(4, np.float32))])
    d = tsn.ref_spec_from_gguf(path, B=2, T=172, C=64, TS=154)
    assert (d.H, d.NH, d.n_joint, d.n_fused, d.latent, d.F) == (1024, 16, 7, 14, 64, 2816)
