"""ctypes wrapper of the CPU oracle (oracle/_build/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's CPU-baseline
leg, as the checker. The product (libtsn) never uses it.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "liboracle.so")

_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float
_SZ = ctypes.c_size_t


class OrcSpec(ctypes.Structure):
    _fields_ = [("B", _I), ("La", _I), ("Lt", _I), ("H", _I), ("NH", _I), ("HD", _I), ("F", _I),
                ("latent", _I), ("temb_dim", _I), ("n_joint", _I), ("n_fused", _I), ("audio_ffn_conv", _I),
                ("rope_theta", _F), ("t_max_period", _F), ("ln_eps", _F), ("rms_eps", _F)]


class RefSpec(ctypes.Structure):
    """orc_ref_spec: the reference's three-stream graph"""
    _fields_ = [("B", _I), ("T", _I), ("C", _I), ("TS", _I), ("H", _I), ("NH", _I), ("HD", _I), ("F", _I),
                ("latent", _I), ("n_joint", _I), ("n_fused", _I),
                ("rope_theta", _F), ("t_max_period", _F), ("ln_eps", _F), ("rms_eps", _F)]


class CondSpec(ctypes.Structure):
    """orc_refcond_spec: the reference's conditioning prep"""
    _fields_ = [("H", _I), ("F", _I), ("T", _I), ("C", _I), ("sync_S", _I), ("TS", _I),
                ("sync_dim", _I), ("clip_dim", _I), ("text_dim", _I), ("gtext_dim", _I)]


class VaeSpec(ctypes.Structure):
    """orc_vae_spec: the reference's VAE decoder"""
    _fields_ = [("T", _I), ("latent", _I), ("width", _I * 6), ("stride", _I * 5), ("kt", _I * 5), ("out_ch", _I)]


_SIGS = {
    "orc_gemm": [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I],
    "orc_gemv": [_P, _P, _P, _P, _I, _I, _I],
    "orc_conv1d": [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I],
    "orc_conv1d_direct": [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I],
    "orc_adaln_ln": [_P, _P, _P, _I, _I, _I, _I, _I, _F],
    "orc_gate_add": [_P, _P, _P, _P, _I, _I, _I, _I, _I],
    "orc_rms_head": [_P, _P, _I, _I, _I, _I, _I, _I, _F],
    "orc_rope_pairs": [_P, _P, _I, _I, _I, _I, _I, _I, _F, _F],
    "orc_attention": [_P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _I, _F],
    "orc_silu": [_P, _SZ],
    "orc_swiglu": [_P, _P, _P, _SZ],
    "orc_add": [_P, _P, _P, _SZ],
    "orc_add_bcast_col": [_P, _P, _P, _I, _I],
    "orc_cfg_euler": [_P, _P, _P, _SZ, _F, _F],
    "orc_timestep_embedding": [_F, _I, _F, _P],
    "orc_manifest_count": [ctypes.POINTER(OrcSpec)],
    "orc_manifest_numel": [ctypes.POINTER(OrcSpec), _I],
    "orc_manifest_total": [ctypes.POINTER(OrcSpec)],
    "orc_manifest_name": [ctypes.POINTER(OrcSpec), _I, ctypes.c_char_p, _I],
    "orc_joint_block": [ctypes.POINTER(OrcSpec), _P, _I, _P, _P],
    "orc_fused_block": [ctypes.POINTER(OrcSpec), _P, _I, _P, _P],
    "orc_dit_forward": [ctypes.POINTER(OrcSpec), _P, _P, _P, _P, _P, _P, _P, _P],
    "orc_dit_sample": [ctypes.POINTER(OrcSpec), _P, _P, _P, _P, _I, _F],
    "orc_num_threads": [],
    "orc_ref_manifest_count": [ctypes.POINTER(RefSpec)],
    "orc_ref_manifest_numel": [ctypes.POINTER(RefSpec), _I],
    "orc_ref_manifest_name": [ctypes.POINTER(RefSpec), _I, ctypes.c_char_p, _I],
    "orc_ref_dit_forward": [ctypes.POINTER(RefSpec), _P, _P, _P, _P, _P, _P, _P, _P, _P],
    "orc_ref_dit_sample": [ctypes.POINTER(RefSpec), _P, _P, _P, _P, _P, _P, _I, _F],
    "orc_refcond_manifest_count": [ctypes.POINTER(CondSpec)],
    "orc_refcond_manifest_numel": [ctypes.POINTER(CondSpec), _I],
    "orc_refcond_manifest_name": [ctypes.POINTER(CondSpec), _I, ctypes.c_char_p, _I],
    "orc_ref_prep_conditioning": [ctypes.POINTER(CondSpec), _P, _P, _P, _P, _P, _P],
    "orc_ref_prep_text_arm": [ctypes.POINTER(CondSpec), _P, _P, _P, _P, _P, _P],
    "orc_vae_manifest_count": [ctypes.POINTER(VaeSpec)],
    "orc_vae_manifest_numel": [ctypes.POINTER(VaeSpec), _I],
    "orc_vae_manifest_name": [ctypes.POINTER(VaeSpec), _I, ctypes.c_char_p, _I],
    "orc_vae_audio_len": [ctypes.POINTER(VaeSpec)],
    "orc_snake": [_P, _P, _P, _P, _I, _I],
    "orc_conv1d_t": [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I],
    "orc_vae_decode": [ctypes.POINTER(VaeSpec), _P, _P, _P],
}
_RES = {"orc_manifest_count": _I, "orc_manifest_numel": ctypes.c_int64, "orc_manifest_total": ctypes.c_int64,
        "orc_num_threads": _I, "orc_ref_manifest_count": _I, "orc_ref_manifest_numel": ctypes.c_int64,
        "orc_refcond_manifest_count": _I, "orc_refcond_manifest_numel": ctypes.c_int64,
        "orc_vae_manifest_count": _I, "orc_vae_manifest_numel": ctypes.c_int64, "orc_vae_audio_len": ctypes.c_int64}

_lib = None


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError("oracle not built (%s); run make -C oracle" % LIB_PATH)
        L = ctypes.CDLL(LIB_PATH)
        for n, a in _SIGS.items():
            f = getattr(L, n)
            f.argtypes = a
            f.restype = _RES.get(n, None)
        _lib = L
    return _lib


def p(a):
    if a is None:
        return None
    assert a.dtype in (np.float32, np.int32) and a.flags["C_CONTIGUOUS"], (a.dtype, a.flags)
    return ctypes.c_void_p(a.ctypes.data)


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def spec_from(d):
    """OrcSpec from any object/dict with the tsn_dit_spec fields."""
    s = OrcSpec()
    for k, _ in OrcSpec._fields_:
        setattr(s, k, d[k] if isinstance(d, dict) else getattr(d, k))
    return s


# ---------------- single ops (numpy in / numpy out) ----------------
def gemm(W, X, bias=None):
    W, X = f32(W), f32(X)
    M, K = X.shape
    N = W.shape[0]
    Y = np.empty((M, N), np.float32)
    lib().orc_gemm(p(W), p(X), p(Y), p(f32(bias)) if bias is not None else None, M, N, K, K, K, N)
    return Y


def gemv(W, x, bias=None):
    W, x = f32(W), f32(x)
    N, K = W.shape
    y = np.empty(N, np.float32)
    lib().orc_gemv(p(W), p(x), p(y), p(f32(bias)) if bias is not None else None, N, K, K)
    return y


def conv1d(W, bias, x, pad, stride=1, dil=1, direct=False):
    """W [OC][IC][K], x [T, IC] -> y [OL, OC]"""
    W, x = f32(W), f32(x)
    OC, IC, K = W.shape
    T = x.shape[0]
    OL = (T + 2 * pad - dil * (K - 1) - 1) // stride + 1
    y = np.empty((OL, OC), np.float32)
    fn = lib().orc_conv1d_direct if direct else lib().orc_conv1d
    fn(p(W), p(f32(bias)) if bias is not None else None, p(x), p(y), T, OL, IC, OC, K, stride, pad, dil)
    return y


def adaln_ln(x, mod, per_row, chunks, base, eps=1e-5):
    x, mod = f32(x), f32(mod)
    rows, H = x.shape
    y = np.empty_like(x)
    lib().orc_adaln_ln(p(x), p(mod), p(y), rows, H, per_row, chunks, base, eps)
    return y


def gate_add(x, f, mod, per_row, chunks, gate_idx):
    x, f, mod = f32(x), f32(f), f32(mod)
    rows, H = x.shape
    y = np.empty_like(x)
    lib().orc_gate_add(p(x), p(f), p(mod), p(y), rows, H, per_row, chunks, gate_idx)
    return y


def rms_head(x, w, rows, nh, ld, hd, col_off, row_off, eps=1e-6):
    x = f32(x).copy()
    lib().orc_rms_head(p(x), p(f32(w)), rows, nh, ld, hd, col_off, row_off, eps)
    return x


def rope_pairs(x, pos, rows, nh, ld, hd, col_off, row_off, fscale=1.0, base=10000.0):
    x = f32(x).copy()
    lib().orc_rope_pairs(p(x), p(np.ascontiguousarray(pos, np.int32)) if pos is not None else None,
                         rows, nh, ld, hd, col_off, row_off, fscale, base)
    return x


def attention(qkv, S, nh, hd, ld, ldo, q_off, k_off, v_off, o_off, scale):
    qkv = f32(qkv)
    out = np.zeros((S, ldo), np.float32)
    lib().orc_attention(p(qkv), p(out), S, nh, hd, ld, ldo, q_off, k_off, v_off, o_off, scale)
    return out


def silu(x):
    x = f32(x).copy()
    lib().orc_silu(p(x), x.size)
    return x


def swiglu(a, b):
    a, b = f32(a), f32(b)
    y = np.empty_like(a)
    lib().orc_swiglu(p(a), p(b), p(y), a.size)
    return y


def add(a, b):
    a, b = f32(a), f32(b)
    y = np.empty_like(a)
    lib().orc_add(p(a), p(b), p(y), a.size)
    return y


def add_bcast_col(x, v):
    x, v = f32(x), f32(v)
    y = np.empty_like(x)
    lib().orc_add_bcast_col(p(x), p(v), p(y), x.shape[0], x.shape[1])
    return y


def cfg_euler(fc, fu, x, cfg, dt):
    x = f32(x).copy()
    lib().orc_cfg_euler(p(f32(fc)), p(f32(fu)), p(x), x.size, cfg, dt)
    return x


def timestep_embedding(t, D, max_period=1.0):
    out = np.empty(D, np.float32)
    lib().orc_timestep_embedding(t, D, max_period, p(out))
    return out


# ---------------- graph ----------------
def manifest(spec):
    s = spec_from(spec)
    L = lib()
    out, buf = [], ctypes.create_string_buffer(256)
    off = 0
    for i in range(L.orc_manifest_count(ctypes.byref(s))):
        L.orc_manifest_name(ctypes.byref(s), i, buf, 256)
        n = L.orc_manifest_numel(ctypes.byref(s), i)
        out.append((buf.value.decode(), n, off))
        off += n
    return out


def joint_block(spec, W, block, X, g):
    s = spec_from(spec)
    X = f32(X).copy()
    gs = silu(g)
    lib().orc_joint_block(ctypes.byref(s), p(W), block, p(X), p(gs))
    return X


def fused_block(spec, W, block, X, g):
    s = spec_from(spec)
    X = f32(X).copy()
    gs = silu(g)
    lib().orc_fused_block(ctypes.byref(s), p(W), block, p(X), p(gs))
    return X


def dit_forward(spec, W, z, t, text, pooled, taps=False):
    s = spec_from(spec)
    B, La, lat, S, H = s.B, s.La, s.latent, s.La + s.Lt, s.H
    v = np.empty((B, La, lat), np.float32)
    tp = np.empty((s.n_joint + s.n_fused, B, S, H), np.float32) if taps else None
    gs = np.empty((B, H), np.float32)
    lib().orc_dit_forward(ctypes.byref(s), p(W), p(f32(z)), p(f32(t)), p(f32(text)), p(f32(pooled)), p(v), p(tp), p(gs))
    return (v, tp, gs) if taps else v


def dit_sample(spec, W, x, text, pooled, steps, cfg):
    s = spec_from(spec)
    x = f32(x).copy()
    lib().orc_dit_sample(ctypes.byref(s), p(W), p(x), p(f32(text)), p(f32(pooled)), steps, cfg)
    return x


def num_threads():
    return lib().orc_num_threads()


# ---------------- the reference's three-stream graph ----------------
def ref_spec_from(spec):
    if isinstance(spec, RefSpec):
        return spec
    d = spec if isinstance(spec, dict) else {k: getattr(spec, k) for k, _ in RefSpec._fields_}
    return RefSpec(**{k: d[k] for k, _ in RefSpec._fields_})


def ref_manifest(spec):
    s = ref_spec_from(spec)
    L = lib()
    out, buf = [], ctypes.create_string_buffer(256)
    off = 0
    for i in range(L.orc_ref_manifest_count(ctypes.byref(s))):
        L.orc_ref_manifest_name(ctypes.byref(s), i, buf, 256)
        n = L.orc_ref_manifest_numel(ctypes.byref(s), i)
        out.append((buf.value.decode(), n, off))
        off += n
    return out


def ref_dit_forward(spec, W, x, t, clip_pp, text_pp, gcmlp, sync_gather, taps=False):
    s = ref_spec_from(spec)
    S = s.T + s.C + s.TS
    v = np.empty((s.B, s.T, s.latent), np.float32)
    tp = np.empty((s.n_joint + s.n_fused, s.B, S, s.H), np.float32) if taps else None
    lib().orc_ref_dit_forward(ctypes.byref(s), p(W), p(f32(x)), p(f32(t)), p(f32(clip_pp)), p(f32(text_pp)),
                              p(f32(gcmlp)), p(f32(sync_gather)), p(v), p(tp))
    return (v, tp) if taps else v


def ref_dit_sample(spec, W, x, clip_pp, text_pp, gcmlp, sync_gather, steps, cfg):
    s = ref_spec_from(spec)
    x = f32(x).copy()
    lib().orc_ref_dit_sample(ctypes.byref(s), p(W), p(x), p(f32(clip_pp)), p(f32(text_pp)), p(f32(gcmlp)),
                             p(f32(sync_gather)), steps, cfg)
    return x


# ---------------- the reference's conditioning prep ----------------
def cond_spec_from(spec):
    if isinstance(spec, CondSpec):
        return spec
    d = spec if isinstance(spec, dict) else {k: getattr(spec, k) for k, _ in CondSpec._fields_}
    return CondSpec(**{k: d[k] for k, _ in CondSpec._fields_})


def cond_manifest(spec):
    s = cond_spec_from(spec)
    L = lib()
    out, buf = [], ctypes.create_string_buffer(256)
    off = 0
    for i in range(L.orc_refcond_manifest_count(ctypes.byref(s))):
        L.orc_refcond_manifest_name(ctypes.byref(s), i, buf, 256)
        n = L.orc_refcond_manifest_numel(ctypes.byref(s), i)
        out.append((buf.value.decode(), n, off))
        off += n
    return out


def ref_prep_conditioning(spec, W, clip_f, sync_f):
    """-> clip_pp [C, H], sync_gather [T, H], clip_fc [H]"""
    s = cond_spec_from(spec)
    clip_pp = np.empty((s.C, s.H), np.float32)
    sync_gather = np.empty((s.T, s.H), np.float32)
    clip_fc = np.empty(s.H, np.float32)
    lib().orc_ref_prep_conditioning(ctypes.byref(s), p(W), p(f32(clip_f)), p(f32(sync_f)), p(clip_pp),
                                    p(sync_gather), p(clip_fc))
    return clip_pp, sync_gather, clip_fc


def ref_prep_text_arm(spec, W, text_cat, gtext, clip_fc):
    """-> text_pp [TS, H], gcmlp [H]"""
    s = cond_spec_from(spec)
    text_pp = np.empty((s.TS, s.H), np.float32)
    gcmlp = np.empty(s.H, np.float32)
    lib().orc_ref_prep_text_arm(ctypes.byref(s), p(W), p(f32(text_cat)), p(f32(gtext)), p(f32(clip_fc)),
                                p(text_pp), p(gcmlp))
    return text_pp, gcmlp


# ---------------- the reference's VAE decoder ----------------
def vae_spec_from(spec):
    """VaeSpec from a VaeSpec, a dict or an object with T, latent, width[6], stride[5], kt[5], out_ch"""
    if isinstance(spec, VaeSpec):
        return spec
    d = spec if isinstance(spec, dict) else {k: getattr(spec, k) for k, _ in VaeSpec._fields_}
    s = VaeSpec()
    s.T, s.latent, s.out_ch = d["T"], d["latent"], d["out_ch"]
    for i in range(6):
        s.width[i] = d["width"][i]
    for i in range(5):
        s.stride[i] = d["stride"][i]
        s.kt[i] = d["kt"][i]
    return s


def vae_manifest(spec):
    s = vae_spec_from(spec)
    L = lib()
    out, buf = [], ctypes.create_string_buffer(256)
    off = 0
    for i in range(L.orc_vae_manifest_count(ctypes.byref(s))):
        L.orc_vae_manifest_name(ctypes.byref(s), i, buf, 256)
        n = L.orc_vae_manifest_numel(ctypes.byref(s), i)
        out.append((buf.value.decode(), n, off))
        off += n
    return out


def vae_audio_len(spec):
    s = vae_spec_from(spec)
    return lib().orc_vae_audio_len(ctypes.byref(s))


def snake(x, alpha, beta):
    """x [S, C] -> x + sin(x*exp(alpha))^2 * exp(-beta)"""
    x = f32(x)
    S, C = x.shape
    y = np.empty_like(x)
    lib().orc_snake(p(x), p(y), p(f32(alpha)), p(f32(beta)), S, C)
    return y


def conv1d_t(W, bias, x, stride, pad):
    """reference-form transposed conv: W [OC][IC][K], x [T, IC] -> y [T*stride, OC]"""
    W, x = f32(W), f32(x)
    OC, IC, K = W.shape
    T = x.shape[0]
    y = np.empty((T * stride, OC), np.float32)
    lib().orc_conv1d_t(p(W), p(f32(bias)) if bias is not None else None, p(x), p(y), T, T * stride, IC, OC, K,
                       stride, pad)
    return y


def vae_decode(spec, W, latent):
    """latent [T, latent] -> audio [T_audio, out_ch]"""
    s = vae_spec_from(spec)
    audio = np.empty((vae_audio_len(s), s.out_ch), np.float32)
    lib().orc_vae_decode(ctypes.byref(s), p(f32(W)), p(f32(latent)), p(audio))
    return audio
