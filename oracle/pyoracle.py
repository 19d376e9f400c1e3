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


class ClipSpec(ctypes.Structure):
    """orc_clip_spec: the reference's CLIP text encoder"""
    _fields_ = [("H", _I), ("NL", _I), ("NH", _I), ("ctx", _I), ("vocab", _I), ("eps", _F)]


class T5Spec(ctypes.Structure):
    """orc_t5_spec: the reference's T5 v1.1 encoder"""
    _fields_ = [("d", _I), ("d_ff", _I), ("NL", _I), ("NH", _I), ("ctx", _I), ("vocab", _I), ("n_bucket", _I),
                ("max_dist", _I), ("eps", _F)]


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
    "orc_geglu": [_P, _P, _P, _SZ],
    "orc_gelu_quick": [_P, _SZ],
    "orc_ln_plain": [_P, _P, _I, _I, _F],
    "orc_mean_cols": [_P, _P, _I, _I],
    "orc_qkv_split3": [_P, _P, _I, _I, _I],
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
    "orc_clip_manifest_count": [ctypes.POINTER(ClipSpec)],
    "orc_clip_manifest_numel": [ctypes.POINTER(ClipSpec), _I],
    "orc_clip_manifest_name": [ctypes.POINTER(ClipSpec), _I, ctypes.c_char_p, _I],
    "orc_t5_manifest_count": [ctypes.POINTER(T5Spec)],
    "orc_t5_manifest_numel": [ctypes.POINTER(T5Spec), _I],
    "orc_t5_manifest_name": [ctypes.POINTER(T5Spec), _I, ctypes.c_char_p, _I],
    "orc_ln_wb": [_P, _P, _P, _P, _I, _I, _F],
    "orc_rms_w": [_P, _P, _P, _I, _I, _F],
    "orc_t5_bucket": [_I, _I, _I],
    "orc_enc_attention": [_P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _F, _I, _P, _P, _P, _I],
    "orc_clip_encode": [ctypes.POINTER(ClipSpec), _P, _P, _P, _P],
    "orc_t5_encode": [ctypes.POINTER(T5Spec), _P, _P, _P],
}
_RES = {"orc_manifest_count": _I, "orc_manifest_numel": ctypes.c_int64, "orc_manifest_total": ctypes.c_int64,
        "orc_num_threads": _I, "orc_ref_manifest_count": _I, "orc_ref_manifest_numel": ctypes.c_int64,
        "orc_refcond_manifest_count": _I, "orc_refcond_manifest_numel": ctypes.c_int64,
        "orc_vae_manifest_count": _I, "orc_vae_manifest_numel": ctypes.c_int64, "orc_vae_audio_len": ctypes.c_int64,
        "orc_clip_manifest_count": _I, "orc_clip_manifest_numel": ctypes.c_int64,
        "orc_t5_manifest_count": _I, "orc_t5_manifest_numel": ctypes.c_int64, "orc_t5_bucket": _I}

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
    # data_as keeps a reference to the array, so a temporary made by f32() lives through the call
    return a.ctypes.data_as(ctypes.c_void_p)


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


def geglu(a, b):
    a, b = f32(a), f32(b)
    y = np.empty_like(a)
    lib().orc_geglu(p(a), p(b), p(y), a.size)
    return y


def gelu_quick(x):
    x = f32(x).copy()
    lib().orc_gelu_quick(p(x), x.size)
    return x


def ln_plain(x, eps=1e-5):
    x = f32(x)
    y = np.empty_like(x)
    lib().orc_ln_plain(p(x), p(y), x.shape[0], x.shape[1], eps)
    return y


def mean_cols(x):
    x = f32(x)
    y = np.empty(x.shape[1], np.float32)
    lib().orc_mean_cols(p(x), p(y), x.shape[0], x.shape[1])
    return y


def qkv_split3(src, dst, row_off):
    """src [rows, 3H] element-interleaved -> copy of dst [., 3H] with rows row_off.. in q|k|v blocks"""
    src = f32(src)
    dst = f32(dst).copy()
    rows, H3 = src.shape
    lib().orc_qkv_split3(p(src), p(dst), rows, H3 // 3, row_off)
    return dst


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
    x, alpha, beta = f32(x), f32(alpha), f32(beta)
    S, C = x.shape
    y = np.empty_like(x)
    lib().orc_snake(p(x), p(y), p(alpha), p(beta), S, C)
    return y


def conv1d_t(W, bias, x, stride, pad):
    """reference-form transposed conv: W [OC][IC][K], x [T, IC] -> y [T*stride, OC]"""
    W, x = f32(W), f32(x)
    bias = None if bias is None else f32(bias)
    OC, IC, K = W.shape
    T = x.shape[0]
    y = np.empty((T * stride, OC), np.float32)
    lib().orc_conv1d_t(p(W), p(bias), p(x), p(y), T, T * stride, IC, OC, K, stride, pad)
    return y


def vae_decode(spec, W, latent):
    """latent [T, latent] -> audio [T_audio, out_ch]"""
    s = vae_spec_from(spec)
    W, latent = f32(W), f32(latent)
    audio = np.empty((vae_audio_len(s), s.out_ch), np.float32)
    lib().orc_vae_decode(ctypes.byref(s), p(W), p(latent), p(audio))
    return audio


# ---------------- the reference's text encoders ----------------
def _spec(cls, spec):
    if isinstance(spec, cls):
        return spec
    d = spec if isinstance(spec, dict) else {k: getattr(spec, k) for k, _ in cls._fields_}
    return cls(**{k: d[k] for k, _ in cls._fields_})


def _manifest(prefix, cls, spec):
    s = _spec(cls, spec)
    L = lib()
    out, buf = [], ctypes.create_string_buffer(256)
    off = 0
    for i in range(getattr(L, prefix + "_manifest_count")(ctypes.byref(s))):
        getattr(L, prefix + "_manifest_name")(ctypes.byref(s), i, buf, 256)
        n = getattr(L, prefix + "_manifest_numel")(ctypes.byref(s), i)
        out.append((buf.value.decode(), n, off))
        off += n
    return out


def clip_manifest(spec):
    return _manifest("orc_clip", ClipSpec, spec)


def t5_manifest(spec):
    return _manifest("orc_t5", T5Spec, spec)


def ln_wb(x, w, b, eps):
    x, w, b = f32(x), f32(w), f32(b)
    y = np.empty_like(x)
    lib().orc_ln_wb(p(x), p(y), p(w), p(b), x.shape[0], x.shape[1], eps)
    return y


def rms_w(x, w, eps):
    x, w = f32(x), f32(w)
    y = np.empty_like(x)
    lib().orc_rms_w(p(x), p(y), p(w), x.shape[0], x.shape[1], eps)
    return y


def t5_bucket(rel, n_bucket=32, max_dist=128):
    return lib().orc_t5_bucket(rel, n_bucket, max_dist)


def enc_attention(qkv, nh, scale, mode, bucket=None, rel=None, pad=None, eot=0, hd=64):
    """qkv [S, 3*nh*hd] (q | k | v) -> out [S, nh*hd]"""
    qkv = f32(qkv)
    S = qkv.shape[0]
    H = nh * hd
    out = np.empty((S, H), np.float32)
    bucket = None if bucket is None else np.ascontiguousarray(bucket, np.int32)
    pad = None if pad is None else np.ascontiguousarray(pad, np.int32)
    rel = None if rel is None else f32(rel)
    lib().orc_enc_attention(p(qkv), p(out), S, nh, hd, 3 * H, 0, H, 2 * H, H, scale, mode, p(bucket), p(rel), p(pad),
                            eot)
    return out


def clip_encode(spec, W, ids):
    """ids [ctx] -> per_token [ctx, H], global [H]"""
    s = _spec(ClipSpec, spec)
    ids, W = np.ascontiguousarray(ids, np.int32), f32(W)
    per_token = np.empty((s.ctx, s.H), np.float32)
    glob = np.empty(s.H, np.float32)
    lib().orc_clip_encode(ctypes.byref(s), p(W), p(ids), p(per_token), p(glob))
    return per_token, glob


def t5_encode(spec, W, ids):
    """ids [ctx] -> out [ctx, d]"""
    s = _spec(T5Spec, spec)
    ids, W = np.ascontiguousarray(ids, np.int32), f32(W)
    out = np.empty((s.ctx, s.d), np.float32)
    lib().orc_t5_encode(ctypes.byref(s), p(W), p(ids), p(out))
    return out


# ---------------- tokenizers: pure-Python restatement (src/tokenizers.cpp) ----------------
def _byte_symbols():
    """GPT-2 byte alphabet: printable bytes map to themselves, the rest to U+0100.. in byte order"""
    keep = set(range(ord("!"), ord("~") + 1)) | set(range(0xA1, 0xAD)) | set(range(0xAE, 0x100))
    out, nxt = {}, 256
    for b in range(256):
        if b in keep:
            out[b] = chr(b)
        else:
            out[b] = chr(nxt)
            nxt += 1
    return out


def clip_bpe_encode(vocab, merges, text, ctx, bos=49406, eos=49407):
    """ClipTokenizer::encode (src/tokenizers.cpp:61-96): ASCII-lowercased, split on C-locale
    whitespace, bytes -> symbols, '</w>' on the last, repeatedly merge the lowest-ranked adjacent
    pair (leftmost among equal ranks), look up (unknown symbols dropped), bos ... eos, cut / pad"""
    ids_of = {}
    for i, v in enumerate(vocab):
        ids_of[v] = i
    rank = {}
    for i, m in enumerate(merges):
        rank[m] = i
    bsym = _byte_symbols()
    low = "".join(chr(ord(c) + 32) if "A" <= c <= "Z" else c for c in text)
    words = [w for w in "".join(" " if c in " \t\n\v\f\r" else c for c in low).split(" ") if w]
    ids = [bos]
    for w in words:
        sym = [bsym[b] for b in w.encode("utf-8", "surrogateescape")]
        sym[-1] += "</w>"
        while len(sym) > 1:
            best, at = None, None
            for i in range(len(sym) - 1):
                r = rank.get(sym[i] + " " + sym[i + 1])
                if r is not None and (best is None or r < best):
                    best, at = r, i
            if best is None:
                break
            sym[at:at + 2] = [sym[at] + sym[at + 1]]
        ids += [ids_of[t] for t in sym if t in ids_of]
    ids.append(eos)
    if len(ids) > ctx:
        ids = ids[:ctx]
        ids[-1] = eos
    return ids + [eos] * (ctx - len(ids))


def t5_unigram_encode(pieces, scores, text, ctx, pad, unk_id=2, eos_id=1, pad_id=0):
    """T5Tokenizer::encode (src/tokenizers.cpp:98-140): trimmed, U+2581 for spaces and at the start,
    Viterbi over pieces (strictly better replaces; unknown chars at min(min score, 0) - 10), eos"""
    idx = {}
    for i, pc in enumerate(pieces):
        idx[pc] = i
    sc = list(scores) + [0.0] * (len(pieces) - len(scores))
    unk = min([0.0] + [float(x) for x in sc]) - 10.0
    t = "\u2581" + text.strip(" \t\n").replace(" ", "\u2581")
    chars = list(t)
    L = len(chars)
    best = [-1e18] * (L + 1)
    frm = [-1] * (L + 1)
    tok = [-1] * (L + 1)
    best[0] = 0.0
    for i in range(L):
        if best[i] <= -1e17:
            continue
        piece = ""
        for j in range(i, L):
            piece += chars[j]
            if piece in idx:
                v = best[i] + float(sc[idx[piece]])
                if v > best[j + 1]:
                    best[j + 1], frm[j + 1], tok[j + 1] = v, i, idx[piece]
            if len(piece.encode("utf-8")) > 64:
                break
        v = best[i] + unk
        if v > best[i + 1]:
            best[i + 1], frm[i + 1], tok[i + 1] = v, i, unk_id
    ids = []
    i = L
    while i > 0:
        ids.append(tok[i])
        if frm[i] < 0:
            break
        i = frm[i]
    ids = ids[::-1] + [eos_id]
    if len(ids) > ctx:
        ids = ids[:ctx]
        ids[-1] = eos_id
    if pad:
        ids += [pad_id] * (ctx - len(ids))
    return ids
