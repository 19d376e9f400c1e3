"""thinksound-native_amd: MI355X (gfx950) DiT velocity path behind the libtsn C ABI.

Python mirror of the reference host interface for this path — tn::Runtime launchers
(src/net.h:18-51) and tn::DitModel (src/models.h:55-85) — over ctypes. No compute happens in
Python; every call goes through libtsn.so (thinksound-native_amd/lib), which must have been built
(build.py). Loading fails loudly when it is missing: there is no CPU fallback.

The package directory name has a hyphen, so import it with importlib:
    tsn = importlib.import_module("thinksound-native_amd")
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libtsn.so")

F32, F16, BF16 = 0, 1, 2
_NP_DT = {F32: np.float32, F16: np.float16, BF16: np.uint16}

_lib = None


class TsnError(RuntimeError):
    def __init__(self, fn, code, msg):
        super().__init__("%s failed (status %d): %s" % (fn, code, msg))
        self.code = code


class DitSpec(ctypes.Structure):
    """tsn_dit_spec (include/tsn.h)."""
    _fields_ = [("B", ctypes.c_int), ("La", ctypes.c_int), ("Lt", ctypes.c_int),
                ("H", ctypes.c_int), ("NH", ctypes.c_int), ("HD", ctypes.c_int), ("F", ctypes.c_int),
                ("latent", ctypes.c_int), ("temb_dim", ctypes.c_int),
                ("n_joint", ctypes.c_int), ("n_fused", ctypes.c_int), ("audio_ffn_conv", ctypes.c_int),
                ("rope_theta", ctypes.c_float), ("t_max_period", ctypes.c_float),
                ("ln_eps", ctypes.c_float), ("rms_eps", ctypes.c_float)]

    def as_dict(self):
        return {k: getattr(self, k) for k, _ in self._fields_}

    def copy(self, **kw):
        s = DitSpec()
        for k, _ in self._fields_:
            setattr(s, k, kw.get(k, getattr(self, k)))
        return s


class RefDitSpec(ctypes.Structure):
    """tsn_refdit_spec (include/tsn.h): the reference checkpoint's three-stream graph."""
    _fields_ = [("B", ctypes.c_int), ("T", ctypes.c_int), ("C", ctypes.c_int), ("TS", ctypes.c_int),
                ("H", ctypes.c_int), ("NH", ctypes.c_int), ("HD", ctypes.c_int), ("F", ctypes.c_int),
                ("latent", ctypes.c_int), ("n_joint", ctypes.c_int), ("n_fused", ctypes.c_int),
                ("rope_theta", ctypes.c_float), ("t_max_period", ctypes.c_float),
                ("ln_eps", ctypes.c_float), ("rms_eps", ctypes.c_float)]

    def as_dict(self):
        return {k: getattr(self, k) for k, _ in self._fields_}

    def copy(self, **kw):
        s = RefDitSpec()
        for k, _ in self._fields_:
            setattr(s, k, kw.get(k, getattr(self, k)))
        return s


class VaeSpec(ctypes.Structure):
    """tsn_vae_spec (include/tsn.h): the reference's VAE decoder."""
    _fields_ = [("T", ctypes.c_int), ("latent", ctypes.c_int), ("width", ctypes.c_int * 6),
                ("stride", ctypes.c_int * 5), ("kt", ctypes.c_int * 5), ("out_ch", ctypes.c_int)]

    def as_dict(self):
        return {"T": self.T, "latent": self.latent, "width": list(self.width), "stride": list(self.stride),
                "kt": list(self.kt), "out_ch": self.out_ch}

    def copy(self, **kw):
        d = self.as_dict()
        d.update(kw)
        s = VaeSpec()
        s.T, s.latent, s.out_ch = d["T"], d["latent"], d["out_ch"]
        for i in range(6):
            s.width[i] = d["width"][i]
        for i in range(5):
            s.stride[i], s.kt[i] = d["stride"][i], d["kt"][i]
        return s


class ClipSpec(ctypes.Structure):
    """tsn_clip_spec (include/tsn.h): the reference's CLIP text encoder."""
    _fields_ = [("H", ctypes.c_int), ("NL", ctypes.c_int), ("NH", ctypes.c_int), ("ctx", ctypes.c_int),
                ("vocab", ctypes.c_int), ("eps", ctypes.c_float)]

    def as_dict(self):
        return {k: getattr(self, k) for k, _ in self._fields_}

    def copy(self, **kw):
        s = ClipSpec()
        for k, _ in self._fields_:
            setattr(s, k, kw.get(k, getattr(self, k)))
        return s


class T5Spec(ctypes.Structure):
    """tsn_t5_spec (include/tsn.h): the reference's T5 v1.1 encoder."""
    _fields_ = [("d", ctypes.c_int), ("d_ff", ctypes.c_int), ("NL", ctypes.c_int), ("NH", ctypes.c_int),
                ("ctx", ctypes.c_int), ("vocab", ctypes.c_int), ("n_bucket", ctypes.c_int),
                ("max_dist", ctypes.c_int), ("eps", ctypes.c_float)]

    def as_dict(self):
        return {k: getattr(self, k) for k, _ in self._fields_}

    def copy(self, **kw):
        s = T5Spec()
        for k, _ in self._fields_:
            setattr(s, k, kw.get(k, getattr(self, k)))
        return s


class RefCondSpec(ctypes.Structure):
    """tsn_refcond_spec (include/tsn.h): the reference's conditioning prep."""
    _fields_ = [("H", ctypes.c_int), ("F", ctypes.c_int), ("T", ctypes.c_int), ("C", ctypes.c_int),
                ("sync_S", ctypes.c_int), ("TS", ctypes.c_int), ("sync_dim", ctypes.c_int),
                ("clip_dim", ctypes.c_int), ("text_dim", ctypes.c_int), ("gtext_dim", ctypes.c_int)]

    def as_dict(self):
        return {k: getattr(self, k) for k, _ in self._fields_}

    def copy(self, **kw):
        s = RefCondSpec()
        for k, _ in self._fields_:
            setattr(s, k, kw.get(k, getattr(self, k)))
        return s


class KernelStat(ctypes.Structure):
    """tsn_kernel_stat (include/tsn.h)."""
    _fields_ = [("name", ctypes.c_char * 64), ("launches", ctypes.c_int), ("total_ms", ctypes.c_double),
                ("flops", ctypes.c_double), ("bytes", ctypes.c_double)]


_P = ctypes.c_void_p
_U32 = ctypes.c_uint32
_I = ctypes.c_int
_SZ = ctypes.c_size_t
_FL = ctypes.c_float
_SIGS = {
    "tsn_runtime_create": [_I, ctypes.POINTER(_P)],
    "tsn_runtime_destroy": [_P],
    "tsn_alloc": [_P, _SZ, ctypes.POINTER(_P)],
    "tsn_free": [_P, _P],
    "tsn_upload": [_P, _P, _P, _SZ],
    "tsn_download": [_P, _P, _P, _SZ],
    "tsn_begin": [_P],
    "tsn_commit": [_P],
    "tsn_sync": [_P],
    "tsn_runtime_alloc_stats": [_P, ctypes.POINTER(_SZ), ctypes.POINTER(_SZ)],
    "tsn_gemm": [_P, _I, _P, _P, _I, _P, _I, _P, _U32, _U32, _U32, _U32, _U32, _U32],
    "tsn_gemm_noalloc": [_P, _I, _P, _P, _I, _P, _I, _P, _U32, _U32, _U32, _U32, _U32, _U32],
    "tsn_gemm_noalloc_max_elems": [],
    "tsn_gemv": [_P, _P, _I, _P, _P, _P, _U32, _U32, _U32],
    "tsn_conv1d_prepared_bytes": [_I, _U32, _U32, _U32],
    "tsn_conv1d_prepare": [_P, _P, _I, _P, _U32, _U32, _U32],
    "tsn_conv1d": [_P, _I, _P, _P, _P, _P, _U32, _U32, _U32, _U32, _U32, _U32, _U32, _U32, _I],
    "tsn_geglu": [_P, _P, _P, _P, _SZ],
    "tsn_gelu_quick": [_P, _P, _SZ],
    "tsn_ln_plain": [_P, _P, _P, _U32, _U32, _FL],
    "tsn_ln_wb": [_P, _P, _P, _P, _P, _U32, _U32, _FL],
    "tsn_rms_w": [_P, _P, _P, _P, _U32, _U32, _FL],
    "tsn_mean_cols": [_P, _P, _P, _U32, _U32],
    "tsn_qkv_split3": [_P, _P, _P, _U32, _U32, _U32],
    "tsn_silu": [_P, _P, _SZ],
    "tsn_copy": [_P, _P, _P, _SZ],
    "tsn_swiglu": [_P, _P, _P, _P, _SZ],
    "tsn_add": [_P, _P, _P, _P, _SZ],
    "tsn_add_bcast_col": [_P, _P, _P, _P, _U32, _U32],
    "tsn_cfg_euler": [_P, _P, _P, _P, _SZ, _FL, _FL],
    "tsn_adaln_ln": [_P, _P, _P, _P, _I, _U32, _U32, _U32, _U32, _U32, _FL],
    "tsn_gate_add": [_P, _P, _P, _P, _P, _U32, _U32, _U32, _U32, _U32],
    "tsn_rms_head": [_P, _P, _P, _U32, _U32, _U32, _U32, _U32, _U32, _FL],
    "tsn_rope_pairs": [_P, _P, _P, _U32, _U32, _U32, _U32, _U32, _U32, _FL, _FL],
    "tsn_attention": [_P, _P, _P, _U32, _U32, _U32, _U32, _U32, _U32, _U32, _U32, _U32, _FL],
    "tsn_dit_default_spec": [_I, ctypes.POINTER(DitSpec)],
    "tsn_dit_manifest_count": [ctypes.POINTER(DitSpec)],
    "tsn_dit_manifest_entry": [ctypes.POINTER(DitSpec), _I, ctypes.c_char_p, _I,
                               ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(ctypes.c_int64)],
    "tsn_dit_manifest_total": [ctypes.POINTER(DitSpec)],
    "tsn_dit_create": [_P, ctypes.POINTER(DitSpec), ctypes.POINTER(_P)],
    "tsn_dit_destroy": [_P],
    "tsn_dit_upload_weights": [_P, _P, _SZ],
    "tsn_dit_forward": [_P, _P, _FL, _P, _P, _P],
    "tsn_dit_forward_ex": [_P, _P, _P, _P, _P, _P, _P],
    "tsn_dit_joint_block": [_P, _I, _P, _P],
    "tsn_dit_fused_block": [_P, _I, _P, _P],
    "tsn_dit_sample": [_P, _P, _P, _P, _I, _FL],
    "tsn_dit_capture_forward": [_P, _P, _P, _P, _P, _P],
    "tsn_dit_capture_sample": [_P, _P, _P, _P, _I, _FL],
    "tsn_dit_replay": [_P],
    "tsn_probe_peaks": [_P, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double)],
    "tsn_dit_profile_forward": [_P, _P, _P, _P, _P, _P, ctypes.POINTER(KernelStat), _I, ctypes.POINTER(_I)],
    "tsn_synth_normal_f32": [ctypes.c_uint64, ctypes.c_uint64, ctypes.c_double, ctypes.c_double, _SZ, _P],
    "tsn_synth_normal_bf16": [ctypes.c_uint64, ctypes.c_uint64, ctypes.c_double, ctypes.c_double, _SZ, _P],
    "tsn_synth_uniform_f32": [ctypes.c_uint64, ctypes.c_uint64, ctypes.c_double, ctypes.c_double, _SZ, _P],
    "tsn_dit_synth_weights": [ctypes.POINTER(DitSpec), ctypes.c_uint64, ctypes.c_double, _P],
    "tsn_refdit_spec_for_duration": [_I, _I, ctypes.POINTER(RefDitSpec)],
    "tsn_refdit_manifest_count": [ctypes.POINTER(RefDitSpec)],
    "tsn_refdit_manifest_entry": [ctypes.POINTER(RefDitSpec), _I, ctypes.c_char_p, _I,
                                  ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(ctypes.c_int64)],
    "tsn_refdit_manifest_total": [ctypes.POINTER(RefDitSpec)],
    "tsn_refdit_create": [_P, ctypes.POINTER(RefDitSpec), ctypes.POINTER(_P)],
    "tsn_refdit_destroy": [_P],
    "tsn_refdit_upload_weights": [_P, _P, _SZ],
    "tsn_refdit_forward": [_P, _P, _FL, _P, _P, _P, _P, _P],
    "tsn_refdit_forward_ex": [_P, _P, _P, _P, _P, _P, _P, _P, _P],
    "tsn_refdit_sample": [_P, _P, _P, _P, _P, _P, _I, _FL],
    "tsn_refdit_capture_forward": [_P, _P, _P, _P, _P, _P, _P, _P],
    "tsn_refdit_capture_sample": [_P, _P, _P, _P, _P, _P, _I, _FL],
    "tsn_refdit_replay": [_P],
    "tsn_refdit_profile_forward": [_P, _P, _P, _P, _P, _P, _P, _P, ctypes.POINTER(KernelStat), _I,
                                   ctypes.POINTER(_I)],
    "tsn_refdit_synth_weights": [ctypes.POINTER(RefDitSpec), ctypes.c_uint64, ctypes.c_double, _P],
    "tsn_refdit_upload_weights_f32": [_P, _P, _SZ],
    "tsn_refdit_load_gguf": [_P, ctypes.c_char_p],
    "tsn_refdit_spec_from_gguf": [ctypes.c_char_p, _I, _I, _I, _I, ctypes.POINTER(RefDitSpec)],
    "tsn_refcond_spec_for_duration": [_I, ctypes.POINTER(RefCondSpec)],
    "tsn_refcond_spec_from_gguf": [ctypes.c_char_p, _I, _I, _I, _I, ctypes.POINTER(RefCondSpec)],
    "tsn_refcond_manifest_count": [ctypes.POINTER(RefCondSpec)],
    "tsn_refcond_manifest_entry": [ctypes.POINTER(RefCondSpec), _I, ctypes.c_char_p, _I,
                                   ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(ctypes.c_int64)],
    "tsn_refcond_manifest_total": [ctypes.POINTER(RefCondSpec)],
    "tsn_refcond_create": [_P, ctypes.POINTER(RefCondSpec), ctypes.POINTER(_P)],
    "tsn_refcond_destroy": [_P],
    "tsn_refcond_upload_weights": [_P, _P, _SZ],
    "tsn_refcond_upload_weights_f32": [_P, _P, _SZ],
    "tsn_refcond_load_gguf": [_P, ctypes.c_char_p],
    "tsn_refcond_prep_conditioning": [_P, _P, _P, _P, _P, _P],
    "tsn_refcond_prep_text_arm": [_P, _P, _P, _P, _P, _P],
    "tsn_refcond_synth_weights": [ctypes.POINTER(RefCondSpec), ctypes.c_uint64, _P],
    "tsn_vae_spec_for_duration": [_I, ctypes.POINTER(VaeSpec)],
    "tsn_vae_spec_from_gguf": [ctypes.c_char_p, _I, ctypes.POINTER(VaeSpec)],
    "tsn_vae_audio_len": [ctypes.POINTER(VaeSpec)],
    "tsn_vae_manifest_count": [ctypes.POINTER(VaeSpec)],
    "tsn_vae_manifest_entry": [ctypes.POINTER(VaeSpec), _I, ctypes.c_char_p, _I,
                               ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(ctypes.c_int64)],
    "tsn_vae_manifest_total": [ctypes.POINTER(VaeSpec)],
    "tsn_vae_create": [_P, ctypes.POINTER(VaeSpec), ctypes.POINTER(_P)],
    "tsn_vae_destroy": [_P],
    "tsn_vae_upload_weights": [_P, _P, _SZ],
    "tsn_vae_load_gguf": [_P, ctypes.c_char_p],
    "tsn_vae_decode": [_P, _P, _P],
    "tsn_vae_capture_decode": [_P, _P, _P],
    "tsn_vae_replay": [_P],
    "tsn_vae_profile_decode": [_P, _P, _P, _P, _I, ctypes.POINTER(_I)],
    "tsn_vae_synth_weights": [ctypes.POINTER(VaeSpec), ctypes.c_uint64, _P],
    "tsn_clip_spec_default": [ctypes.POINTER(ClipSpec)],
    "tsn_clip_spec_from_gguf": [ctypes.c_char_p, ctypes.POINTER(ClipSpec)],
    "tsn_clip_manifest_count": [ctypes.POINTER(ClipSpec)],
    "tsn_clip_manifest_entry": [ctypes.POINTER(ClipSpec), _I, ctypes.c_char_p, _I,
                                ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(ctypes.c_int64)],
    "tsn_clip_manifest_total": [ctypes.POINTER(ClipSpec)],
    "tsn_clip_create": [_P, ctypes.POINTER(ClipSpec), ctypes.POINTER(_P)],
    "tsn_clip_destroy": [_P],
    "tsn_clip_upload_weights": [_P, _P, _SZ],
    "tsn_clip_load_gguf": [_P, ctypes.c_char_p],
    "tsn_clip_encode": [_P, _P, _P, _P],
    "tsn_clip_profile_encode": [_P, _P, _P, _P, _P, _I, ctypes.POINTER(_I)],
    "tsn_clip_synth_weights": [ctypes.POINTER(ClipSpec), ctypes.c_uint64, _P],
    "tsn_t5_spec_default": [ctypes.POINTER(T5Spec)],
    "tsn_t5_spec_from_gguf": [ctypes.c_char_p, ctypes.POINTER(T5Spec)],
    "tsn_t5_manifest_count": [ctypes.POINTER(T5Spec)],
    "tsn_t5_manifest_entry": [ctypes.POINTER(T5Spec), _I, ctypes.c_char_p, _I,
                              ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(ctypes.c_int64)],
    "tsn_t5_manifest_total": [ctypes.POINTER(T5Spec)],
    "tsn_t5_create": [_P, ctypes.POINTER(T5Spec), ctypes.POINTER(_P)],
    "tsn_t5_destroy": [_P],
    "tsn_t5_upload_weights": [_P, _P, _SZ],
    "tsn_t5_load_gguf": [_P, ctypes.c_char_p],
    "tsn_t5_encode": [_P, _P, _P],
    "tsn_t5_profile_encode": [_P, _P, _P, _P, _I, ctypes.POINTER(_I)],
    "tsn_t5_synth_weights": [ctypes.POINTER(T5Spec), ctypes.c_uint64, _P],
    "tsn_t5_bucket": [_I, _I, _I],
    "tsn_clip_tokenizer_load": [ctypes.c_char_p, ctypes.POINTER(_P)],
    "tsn_clip_tokenizer_destroy": [_P],
    "tsn_clip_tokenizer_encode": [_P, ctypes.c_char_p, _I, _P],
    "tsn_t5_tokenizer_load": [ctypes.c_char_p, ctypes.POINTER(_P)],
    "tsn_t5_tokenizer_destroy": [_P],
    "tsn_t5_tokenizer_encode": [_P, ctypes.c_char_p, _I, _I, _P, ctypes.POINTER(_I)],
    "tsn_gguf_open": [ctypes.c_char_p, ctypes.POINTER(_P)],
    "tsn_gguf_close": [_P],
    "tsn_gguf_tensor_count": [_P],
    "tsn_gguf_tensor_info": [_P, _I, ctypes.c_char_p, _I, ctypes.POINTER(ctypes.c_uint32),
                             ctypes.POINTER(ctypes.c_uint32), ctypes.POINTER(ctypes.c_uint64)],
    "tsn_gguf_tensor_to_f32": [_P, ctypes.c_char_p, _P, _SZ],
    "tsn_gguf_get_i64": [_P, ctypes.c_char_p, ctypes.c_int64],
    "tsn_gguf_get_f64": [_P, ctypes.c_char_p, ctypes.c_double],
}
_RESTYPES = {"tsn_last_error": ctypes.c_char_p, "tsn_last_gpu_ms": ctypes.c_double,
             "tsn_dit_manifest_total": ctypes.c_int64, "tsn_refdit_manifest_total": ctypes.c_int64,
             "tsn_gguf_get_i64": ctypes.c_int64, "tsn_gguf_get_f64": ctypes.c_double,
             "tsn_refcond_manifest_total": ctypes.c_int64, "tsn_version": _I,
             "tsn_vae_manifest_total": ctypes.c_int64, "tsn_vae_audio_len": ctypes.c_int64,
             "tsn_clip_manifest_total": ctypes.c_int64, "tsn_conv1d_prepared_bytes": _SZ,
             "tsn_gemm_noalloc_max_elems": _SZ, "tsn_t5_manifest_total": ctypes.c_int64, "tsn_t5_bucket": _I}


def lib():
    """Load libtsn.so (once). Raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError("libtsn.so is not built (%s); run thinksound-native_amd/build.py" % LIB_PATH)
        L = ctypes.CDLL(LIB_PATH)
        for name, args in _SIGS.items():
            f = getattr(L, name)
            f.argtypes = args
            f.restype = _RESTYPES.get(name, _I)
        L.tsn_last_error.restype = ctypes.c_char_p
        L.tsn_last_error.argtypes = []
        L.tsn_last_gpu_ms.restype = ctypes.c_double
        L.tsn_last_gpu_ms.argtypes = [_P]
        L.tsn_version.restype = _I
        _lib = L
    return _lib


def call(name, *args):
    """Call a tsn_* entry point; raise TsnError on a non-zero status."""
    rc = getattr(lib(), name)(*args)
    if rc != 0:
        raise TsnError(name, rc, lib().tsn_last_error().decode())
    return rc


def ptr(a):
    """Host pointer of a contiguous numpy array (keeps a reference to the array)."""
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.c_void_p)


def default_spec(workload):
    s = DitSpec()
    call("tsn_dit_default_spec", workload, ctypes.byref(s))
    return s


def manifest(spec):
    L = lib()
    n = L.tsn_dit_manifest_count(ctypes.byref(spec))
    out = []
    buf = ctypes.create_string_buffer(256)
    for i in range(n):
        numel, off = ctypes.c_int64(), ctypes.c_int64()
        call("tsn_dit_manifest_entry", ctypes.byref(spec), i, buf, 256, ctypes.byref(numel), ctypes.byref(off))
        out.append((buf.value.decode(), numel.value, off.value))
    return out


def manifest_total(spec):
    return int(lib().tsn_dit_manifest_total(ctypes.byref(spec)))


def synth_normal_f32(seed, index, mean, std, shape):
    a = np.empty(shape, np.float32)
    call("tsn_synth_normal_f32", seed, index, mean, std, a.size, ptr(a))
    return a


def synth_normal_bf16(seed, index, mean, std, shape):
    a = np.empty(shape, np.uint16)
    call("tsn_synth_normal_bf16", seed, index, mean, std, a.size, ptr(a))
    return a


def synth_uniform_f32(seed, index, lo, hi, shape):
    a = np.empty(shape, np.float32)
    call("tsn_synth_uniform_f32", seed, index, lo, hi, a.size, ptr(a))
    return a


def synth_weights(spec, seed=4242, norm_mean=0.0):
    w = np.empty(manifest_total(spec), np.uint16)
    call("tsn_dit_synth_weights", ctypes.byref(spec), seed, norm_mean, ptr(w))
    return w


def ref_spec_for_duration(dur_s, B=2):
    """Geometry of a dur-second generation with B samples (T = llround(44100/2048*dur), C = 8*dur, TS = 154)."""
    s = RefDitSpec()
    call("tsn_refdit_spec_for_duration", dur_s, B, ctypes.byref(s))
    return s


def ref_manifest(spec):
    L = lib()
    n = L.tsn_refdit_manifest_count(ctypes.byref(spec))
    out = []
    buf = ctypes.create_string_buffer(256)
    for i in range(n):
        numel, off = ctypes.c_int64(), ctypes.c_int64()
        call("tsn_refdit_manifest_entry", ctypes.byref(spec), i, buf, 256, ctypes.byref(numel), ctypes.byref(off))
        out.append((buf.value.decode(), numel.value, off.value))
    return out


def ref_manifest_total(spec):
    return int(lib().tsn_refdit_manifest_total(ctypes.byref(spec)))


def ref_synth_weights(spec, seed=4242, norm_mean=0.0):
    w = np.empty(ref_manifest_total(spec), np.uint16)
    call("tsn_refdit_synth_weights", ctypes.byref(spec), seed, norm_mean, ptr(w))
    return w


def ref_spec_from_gguf(path, B=2, T=172, C=64, TS=154):
    """tsn_refdit_spec_from_gguf: hyperparameters from a checkpoint, geometry from the caller."""
    s = RefDitSpec()
    call("tsn_refdit_spec_from_gguf", os.fsencode(path), B, T, C, TS, ctypes.byref(s))
    return s


def cond_spec_for_duration(dur_s):
    s = RefCondSpec()
    call("tsn_refcond_spec_for_duration", dur_s, ctypes.byref(s))
    return s


def cond_spec_from_gguf(path, T=172, C=64, sync_S=192, TS=154):
    s = RefCondSpec()
    call("tsn_refcond_spec_from_gguf", os.fsencode(path), T, C, sync_S, TS, ctypes.byref(s))
    return s


def cond_manifest(spec):
    L = lib()
    out, buf = [], ctypes.create_string_buffer(256)
    for i in range(L.tsn_refcond_manifest_count(ctypes.byref(spec))):
        numel, off = ctypes.c_int64(), ctypes.c_int64()
        call("tsn_refcond_manifest_entry", ctypes.byref(spec), i, buf, 256, ctypes.byref(numel), ctypes.byref(off))
        out.append((buf.value.decode(), numel.value, off.value))
    return out


def cond_synth_weights(spec, seed=4242):
    w = np.empty(int(lib().tsn_refcond_manifest_total(ctypes.byref(spec))), np.uint16)
    call("tsn_refcond_synth_weights", ctypes.byref(spec), seed, ptr(w))
    return w


class RefCondModel:
    """DitModel::prep_conditioning / prep_text_arm mirror (src/dit.cpp:55-191)."""

    def __init__(self, rt, spec):
        self.rt, self.spec = rt, spec
        h = ctypes.c_void_p()
        call("tsn_refcond_create", rt.h, ctypes.byref(spec), ctypes.byref(h))
        self.h = h

    def close(self):
        if self.h:
            lib().tsn_refcond_destroy(self.h)
            self.h = None

    def upload_weights(self, w_bf16):
        w_bf16 = np.ascontiguousarray(w_bf16, dtype=np.uint16)
        call("tsn_refcond_upload_weights", self.h, ptr(w_bf16), w_bf16.size)

    def upload_weights_f32(self, w):
        w = np.ascontiguousarray(w, dtype=np.float32)
        call("tsn_refcond_upload_weights_f32", self.h, ptr(w), w.size)

    def load_gguf(self, path):
        call("tsn_refcond_load_gguf", self.h, os.fsencode(path))

    def prep_conditioning(self, clip_f, sync_f, clip_pp, sync_gather, clip_fc):
        call("tsn_refcond_prep_conditioning", self.h, clip_f.p, sync_f.p, clip_pp.p, sync_gather.p, clip_fc.p)

    def prep_text_arm(self, text_cat, gtext, clip_fc, text_pp, gcmlp):
        call("tsn_refcond_prep_text_arm", self.h, text_cat.p, gtext.p, clip_fc.p, text_pp.p, gcmlp.p)


def vae_spec_for_duration(dur_s):
    s = VaeSpec()
    call("tsn_vae_spec_for_duration", dur_s, ctypes.byref(s))
    return s


def vae_spec_from_gguf(path, T=172):
    """tsn_vae_spec_from_gguf: widths and kernel sizes from a checkpoint, T from the caller."""
    s = VaeSpec()
    call("tsn_vae_spec_from_gguf", os.fsencode(path), T, ctypes.byref(s))
    return s


def vae_audio_len(spec):
    return int(lib().tsn_vae_audio_len(ctypes.byref(spec)))


def vae_manifest(spec):
    L = lib()
    out, buf = [], ctypes.create_string_buffer(256)
    for i in range(L.tsn_vae_manifest_count(ctypes.byref(spec))):
        numel, off = ctypes.c_int64(), ctypes.c_int64()
        call("tsn_vae_manifest_entry", ctypes.byref(spec), i, buf, 256, ctypes.byref(numel), ctypes.byref(off))
        out.append((buf.value.decode(), numel.value, off.value))
    return out


def vae_synth_weights(spec, seed=4242):
    w = np.empty(int(lib().tsn_vae_manifest_total(ctypes.byref(spec))), np.float32)
    call("tsn_vae_synth_weights", ctypes.byref(spec), seed, ptr(w))
    return w


class VaeModel:
    """tn::VaeModel mirror (src/models.h:87-94): load, then decode latent -> audio on the device."""

    def __init__(self, rt, spec):
        self.rt, self.spec = rt, spec
        h = ctypes.c_void_p()
        call("tsn_vae_create", rt.h, ctypes.byref(spec), ctypes.byref(h))
        self.h = h

    def close(self):
        if self.h:
            lib().tsn_vae_destroy(self.h)
            self.h = None

    def upload_weights(self, w):
        w = np.ascontiguousarray(w, dtype=np.float32)
        call("tsn_vae_upload_weights", self.h, ptr(w), w.size)

    def load_gguf(self, path):
        call("tsn_vae_load_gguf", self.h, os.fsencode(path))

    def _check(self, latent, audio):
        s = self.spec
        want_l, want_a = (s.T, s.latent), (vae_audio_len(s), s.out_ch)
        if int(np.prod(latent.shape)) != want_l[0] * want_l[1] or int(np.prod(audio.shape)) != want_a[0] * want_a[1]:
            raise ValueError("vae: latent %s and audio %s expected, got %s and %s"
                             % (want_l, want_a, latent.shape, audio.shape))

    def decode(self, latent, audio):
        """latent [T][latent] -> audio [T_audio][out_ch], device arrays, enqueued on the runtime's stream"""
        self._check(latent, audio)
        call("tsn_vae_decode", self.h, latent.p, audio.p)

    def capture_decode(self, latent, audio):
        self._check(latent, audio)
        call("tsn_vae_capture_decode", self.h, latent.p, audio.p)

    def replay(self):
        call("tsn_vae_replay", self.h)

    def profile_decode(self, latent, audio):
        self._check(latent, audio)
        cap = 64
        arr = (KernelStat * cap)()
        n = ctypes.c_int()
        call("tsn_vae_profile_decode", self.h, latent.p, audio.p, arr, cap, ctypes.byref(n))
        return [{"name": arr[i].name.decode(), "launches": arr[i].launches, "ms": arr[i].total_ms,
                 "flops": arr[i].flops, "bytes": arr[i].bytes} for i in range(n.value)]


def clip_spec_default():
    s = ClipSpec()
    call("tsn_clip_spec_default", ctypes.byref(s))
    return s


def t5_spec_default():
    s = T5Spec()
    call("tsn_t5_spec_default", ctypes.byref(s))
    return s


def clip_spec_from_gguf(path):
    s = ClipSpec()
    call("tsn_clip_spec_from_gguf", os.fsencode(path), ctypes.byref(s))
    return s


def t5_spec_from_gguf(path):
    s = T5Spec()
    call("tsn_t5_spec_from_gguf", os.fsencode(path), ctypes.byref(s))
    return s


def _enc_manifest(prefix, spec):
    L = lib()
    out, buf = [], ctypes.create_string_buffer(256)
    for i in range(getattr(L, prefix + "_manifest_count")(ctypes.byref(spec))):
        numel, off = ctypes.c_int64(), ctypes.c_int64()
        call(prefix + "_manifest_entry", ctypes.byref(spec), i, buf, 256, ctypes.byref(numel), ctypes.byref(off))
        out.append((buf.value.decode(), numel.value, off.value))
    return out


def clip_manifest(spec):
    return _enc_manifest("tsn_clip", spec)


def t5_manifest(spec):
    return _enc_manifest("tsn_t5", spec)


def clip_synth_weights(spec, seed=4242):
    w = np.empty(int(lib().tsn_clip_manifest_total(ctypes.byref(spec))), np.float32)
    call("tsn_clip_synth_weights", ctypes.byref(spec), seed, ptr(w))
    return w


def t5_synth_weights(spec, seed=4242):
    w = np.empty(int(lib().tsn_t5_manifest_total(ctypes.byref(spec))), np.float32)
    call("tsn_t5_synth_weights", ctypes.byref(spec), seed, ptr(w))
    return w


def t5_bucket(rel, n_bucket=32, max_dist=128):
    return int(lib().tsn_t5_bucket(rel, n_bucket, max_dist))


def _stats(arr, n):
    return [{"name": arr[i].name.decode(), "launches": arr[i].launches, "ms": arr[i].total_ms,
             "flops": arr[i].flops, "bytes": arr[i].bytes} for i in range(n.value)]


class ClipModel:
    """tn::ClipModel mirror (src/models.h:24-38): encode host ids -> per-token features and pooled vector."""

    def __init__(self, rt, spec):
        self.rt, self.spec = rt, spec
        h = ctypes.c_void_p()
        call("tsn_clip_create", rt.h, ctypes.byref(spec), ctypes.byref(h))
        self.h = h

    def close(self):
        if self.h:
            lib().tsn_clip_destroy(self.h)
            self.h = None

    def upload_weights(self, w):
        w = np.ascontiguousarray(w, dtype=np.float32)
        call("tsn_clip_upload_weights", self.h, ptr(w), w.size)

    def load_gguf(self, path):
        call("tsn_clip_load_gguf", self.h, os.fsencode(path))

    def _ids(self, ids):
        ids = np.ascontiguousarray(ids, np.int32)
        if ids.shape != (self.spec.ctx,):
            raise ValueError("clip: %d ids expected, got shape %s" % (self.spec.ctx, ids.shape))
        return ids

    def _outs(self, per_token, glob):
        s = self.spec
        if int(np.prod(per_token.shape)) != s.ctx * s.H or int(np.prod(glob.shape)) != s.H:
            raise ValueError("clip: per_token [%d, %d] and global [%d] expected" % (s.ctx, s.H, s.H))

    def encode(self, ids, per_token, glob):
        ids = self._ids(ids)
        self._outs(per_token, glob)
        call("tsn_clip_encode", self.h, ptr(ids), per_token.p, glob.p)

    def profile_encode(self, ids, per_token, glob):
        ids = self._ids(ids)
        self._outs(per_token, glob)
        arr, n = (KernelStat * 64)(), ctypes.c_int()
        call("tsn_clip_profile_encode", self.h, ptr(ids), per_token.p, glob.p, arr, 64, ctypes.byref(n))
        return _stats(arr, n)


class T5Model:
    """tn::T5Model mirror (src/models.h:40-52): encode host ids -> per-token features."""

    def __init__(self, rt, spec):
        self.rt, self.spec = rt, spec
        h = ctypes.c_void_p()
        call("tsn_t5_create", rt.h, ctypes.byref(spec), ctypes.byref(h))
        self.h = h

    def close(self):
        if self.h:
            lib().tsn_t5_destroy(self.h)
            self.h = None

    def upload_weights(self, w):
        w = np.ascontiguousarray(w, dtype=np.float32)
        call("tsn_t5_upload_weights", self.h, ptr(w), w.size)

    def load_gguf(self, path):
        call("tsn_t5_load_gguf", self.h, os.fsencode(path))

    def _ids(self, ids):
        ids = np.ascontiguousarray(ids, np.int32)
        if ids.shape != (self.spec.ctx,):
            raise ValueError("t5: %d ids expected, got shape %s" % (self.spec.ctx, ids.shape))
        return ids

    def _out(self, out):
        if int(np.prod(out.shape)) != self.spec.ctx * self.spec.d:
            raise ValueError("t5: out [%d, %d] expected, got %s" % (self.spec.ctx, self.spec.d, out.shape))

    def encode(self, ids, out):
        ids = self._ids(ids)
        self._out(out)
        call("tsn_t5_encode", self.h, ptr(ids), out.p)

    def profile_encode(self, ids, out):
        ids = self._ids(ids)
        self._out(out)
        arr, n = (KernelStat * 64)(), ctypes.c_int()
        call("tsn_t5_profile_encode", self.h, ptr(ids), out.p, arr, 64, ctypes.byref(n))
        return _stats(arr, n)


class ClipTokenizer:
    """tn::ClipTokenizer mirror (src/tokenizers.h:12-21), host only."""

    def __init__(self, path):
        h = ctypes.c_void_p()
        call("tsn_clip_tokenizer_load", os.fsencode(path), ctypes.byref(h))
        self.h = h

    def close(self):
        if self.h:
            lib().tsn_clip_tokenizer_destroy(self.h)
            self.h = None

    def encode(self, text, ctx=77):
        ids = np.empty(ctx, np.int32)
        call("tsn_clip_tokenizer_encode", self.h, text.encode("utf-8", "surrogateescape"), ctx, ptr(ids))
        return ids.tolist()


class T5Tokenizer:
    """tn::T5Tokenizer mirror (src/tokenizers.h:23-31), host only."""

    def __init__(self, path):
        h = ctypes.c_void_p()
        call("tsn_t5_tokenizer_load", os.fsencode(path), ctypes.byref(h))
        self.h = h

    def close(self):
        if self.h:
            lib().tsn_t5_tokenizer_destroy(self.h)
            self.h = None

    def encode(self, text, ctx=77, pad=True):
        ids, n = np.empty(ctx, np.int32), ctypes.c_int()
        call("tsn_t5_tokenizer_encode", self.h, text.encode("utf-8", "surrogateescape"), ctx, 1 if pad else 0, ptr(ids),
             ctypes.byref(n))
        return ids[:n.value].tolist()


class Gguf:
    """tsn_gguf_* reader: tensors (name, type, shape ne[0] fastest), metadata, host dequantization."""

    def __init__(self, path):
        h = ctypes.c_void_p()
        call("tsn_gguf_open", os.fsencode(path), ctypes.byref(h))
        self.h = h

    def close(self):
        if self.h:
            lib().tsn_gguf_close(self.h)
            self.h = None

    def tensors(self):
        L = lib()
        out, buf = [], ctypes.create_string_buffer(256)
        ty, nd, ne = ctypes.c_uint32(), ctypes.c_uint32(), (ctypes.c_uint64 * 4)()
        for i in range(L.tsn_gguf_tensor_count(self.h)):
            call("tsn_gguf_tensor_info", self.h, i, buf, 256, ctypes.byref(ty), ctypes.byref(nd), ne)
            out.append((buf.value.decode(), ty.value, tuple(ne[d] for d in range(nd.value))))
        return out

    def to_f32(self, name, numel):
        a = np.empty(numel, np.float32)
        call("tsn_gguf_tensor_to_f32", self.h, name.encode(), ptr(a), a.size)
        return a

    def get_i64(self, key, default=0):
        return int(lib().tsn_gguf_get_i64(self.h, key.encode(), default))

    def get_f64(self, key, default=0.0):
        return float(lib().tsn_gguf_get_f64(self.h, key.encode(), default))


def bf16_to_f32(u16):
    return (u16.astype(np.uint32) << 16).view(np.float32)


class DeviceArray:
    """A device allocation owned by a Runtime (freed with it or by free())."""

    def __init__(self, rt, shape, dtype):
        self.rt, self.shape, self.dtype = rt, tuple(shape), np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape)) * self.dtype.itemsize
        p = ctypes.c_void_p()
        call("tsn_alloc", rt.h, max(self.nbytes, 1), ctypes.byref(p))
        self.ptr = p

    @property
    def p(self):
        return self.ptr

    def offset(self, elems):
        return ctypes.c_void_p(self.ptr.value + elems * self.dtype.itemsize)

    def upload(self, a):
        a = np.ascontiguousarray(a, dtype=self.dtype)
        assert a.nbytes == self.nbytes, (a.shape, self.shape)
        call("tsn_upload", self.rt.h, self.ptr, ptr(a), a.nbytes)
        return self

    def numpy(self):
        a = np.empty(self.shape, self.dtype)
        call("tsn_download", self.rt.h, ptr(a), self.ptr, self.nbytes)
        return a

    def free(self):
        if self.ptr is not None:
            call("tsn_free", self.rt.h, self.ptr)
            self.ptr = None


class Runtime:
    """tn::Runtime mirror (src/net.h:18-51) over one GPU and one HIP stream."""

    def __init__(self, device=0):
        h = ctypes.c_void_p()
        call("tsn_runtime_create", device, ctypes.byref(h))
        self.h = h

    def close(self):
        if self.h:
            lib().tsn_runtime_destroy(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def empty(self, shape, dtype=np.float32):
        return DeviceArray(self, shape, dtype)

    def array(self, a, dtype=None):
        a = np.ascontiguousarray(a, dtype=dtype or a.dtype)
        return DeviceArray(self, a.shape, a.dtype).upload(a)

    def sync(self):
        call("tsn_sync", self.h)

    def alloc_stats(self):
        """(count, bytes) of the device allocations this runtime owns"""
        c, b = _SZ(), _SZ()
        call("tsn_runtime_alloc_stats", self.h, ctypes.byref(c), ctypes.byref(b))
        return c.value, b.value

    def begin(self):
        call("tsn_begin", self.h)

    def commit(self):
        call("tsn_commit", self.h)
        return lib().tsn_last_gpu_ms(self.h)

    # --- launchers (names follow src/net.h) ---
    def gemm(self, wdtype, W, X, xdtype, Y, ydtype, bias, M, N, K, ldx=0, ldw=0, ldy=0):
        call("tsn_gemm", self.h, wdtype, W.p, X.p, xdtype, Y.p, ydtype, bias.p if bias is not None else None,
             M, N, K, ldx, ldw, ldy)

    def gemm_noalloc(self, wdtype, W, X, xdtype, Y, ydtype, bias, M, N, K, ldx=0, ldw=0, ldy=0):
        """tsn_gemm on a fixed per-GPU device array instead of the runtime's scratch (allocates nothing)"""
        call("tsn_gemm_noalloc", self.h, wdtype, W.p, X.p, xdtype, Y.p, ydtype, bias.p if bias is not None else None,
             M, N, K, ldx, ldw, ldy)

    @staticmethod
    def gemm_noalloc_max_elems():
        return int(lib().tsn_gemm_noalloc_max_elems())

    def gemv(self, W, wdtype, x, y, bias, N, K, ldw=0):
        call("tsn_gemv", self.h, W.p, wdtype, x.p, y.p, bias.p if bias is not None else None, N, K, ldw)

    @staticmethod
    def conv1d_prepared_bytes(wdtype, OC, IC, K):
        return int(lib().tsn_conv1d_prepared_bytes(wdtype, OC, IC, K))

    def conv1d_prepare(self, W, wdtype, Wp, OC, IC, K):
        call("tsn_conv1d_prepare", self.h, W.p, int(wdtype), Wp.p, OC, IC, K)

    def conv1d(self, wdtype, Wp, bias, x, y, T, OL, IC, OC, K, stride, pad, dil, convt=False):
        call("tsn_conv1d", self.h, int(wdtype), Wp.p, bias.p if bias is not None else None, x.p, y.p, T, OL, IC,
             OC, K, stride, pad, dil, int(bool(convt)))

    def geglu(self, a, b, y, n):
        call("tsn_geglu", self.h, a.p, b.p, y.p, n)

    def gelu_quick(self, x, n):
        call("tsn_gelu_quick", self.h, x.p, n)

    def ln_plain(self, x, y, S, H, eps):
        call("tsn_ln_plain", self.h, x.p, y.p, S, H, eps)

    def ln_wb(self, x, y, w, b, S, H, eps):
        call("tsn_ln_wb", self.h, x.p, y.p, w.p, b.p, S, H, eps)

    def rms_w(self, x, y, w, S, H, eps):
        call("tsn_rms_w", self.h, x.p, y.p, w.p, S, H, eps)

    def mean_cols(self, x, y, S, H):
        call("tsn_mean_cols", self.h, x.p, y.p, S, H)

    def qkv_split3(self, src, dst, rows, H, row_off):
        call("tsn_qkv_split3", self.h, src.p, dst.p, rows, H, row_off)

    def adaln_ln(self, x, mod, y, ydtype, rows, H, per_row, chunks, base, eps):
        call("tsn_adaln_ln", self.h, x.p, mod.p, y.p, ydtype, rows, H, per_row, chunks, base, eps)

    def gate_add(self, x, f, mod, y, rows, H, per_row, chunks, gate_idx):
        call("tsn_gate_add", self.h, x.p, f.p, mod.p, y.p, rows, H, per_row, chunks, gate_idx)

    def rms_head(self, x, w, rows, nh, ld, hd, col_off, row_off, eps):
        call("tsn_rms_head", self.h, x.p, w.p, rows, nh, ld, hd, col_off, row_off, eps)

    def rope_pairs(self, x, pos, rows, nh, ld, hd, col_off, row_off, fscale, base):
        call("tsn_rope_pairs", self.h, x.p, pos.p if pos is not None else None, rows, nh, ld, hd, col_off,
             row_off, fscale, base)

    def attention(self, qkv, out, S, nh, hd, ld, ldo, q_off, k_off, v_off, o_off, scale):
        call("tsn_attention", self.h, qkv.p, out.p, S, nh, hd, ld, ldo, q_off, k_off, v_off, o_off, scale)

    def silu(self, x, n):
        call("tsn_silu", self.h, x.p, n)

    def copy(self, x, y, n):
        call("tsn_copy", self.h, x.p, y.p, n)

    def swiglu(self, a, b, y, n):
        call("tsn_swiglu", self.h, a.p, b.p, y.p, n)

    def add_(self, a, b, y, n):
        call("tsn_add", self.h, a.p, b.p, y.p, n)

    def add_bcast_col(self, x, v, y, S, H):
        call("tsn_add_bcast_col", self.h, x.p, v.p, y.p, S, H)

    def cfg_euler(self, fc, fu, x, n, cfg, dt):
        call("tsn_cfg_euler", self.h, fc.p, fu.p, x.p, n, cfg, dt)

    def probe_peaks(self):
        """(achievable dense f16 MFMA TFLOP/s, device copy GB/s) measured on this GPU"""
        t, g = ctypes.c_double(), ctypes.c_double()
        call("tsn_probe_peaks", self.h, ctypes.byref(t), ctypes.byref(g))
        return t.value, g.value


def _need(what, arr, numel, itemsize=4, optional=False):
    """A device array must hold at least numel elements of itemsize bytes: a short buffer would
    otherwise become an out-of-bounds device access instead of an error."""
    if arr is None:
        if optional:
            return
        raise ValueError("%s: a device array is required" % what)
    have = getattr(arr, "nbytes", None)
    if have is None or not hasattr(arr, "p"):
        raise TypeError("%s: expected a DeviceArray, got %r" % (what, type(arr)))
    if have < numel * itemsize:
        raise ValueError("%s: %d bytes needed, the array holds %d" % (what, numel * itemsize, have))


class DitModel:
    """tn::DitModel mirror (src/models.h:55-85) for the batched two-stream graph."""

    def __init__(self, rt, spec):
        self.rt, self.spec = rt, spec
        h = ctypes.c_void_p()
        call("tsn_dit_create", rt.h, ctypes.byref(spec), ctypes.byref(h))
        self.h = h

    def close(self):
        if self.h:
            lib().tsn_dit_destroy(self.h)
            self.h = None

    def upload_weights(self, w_bf16):
        w_bf16 = np.ascontiguousarray(w_bf16, dtype=np.uint16)
        call("tsn_dit_upload_weights", self.h, ptr(w_bf16), w_bf16.size)

    def _io(self, z=None, t_dev=None, text=None, pooled=None, v=None, taps=None, x=None, X=None, g=None):
        s = self.spec
        S = s.La + s.Lt
        if z is not None or v is not None:
            _need("dit z", z, s.B * s.La * s.latent)
            _need("dit v", v, s.B * s.La * s.latent)
            _need("dit pooled", pooled, s.B * s.H)
            _need("dit text", text, s.B * s.Lt * s.H, optional=s.Lt == 0)
        if t_dev is not None:
            _need("dit t", t_dev, s.B)
        _need("dit taps", taps, (s.n_joint + s.n_fused) * s.B * S * s.H, optional=True)
        if x is not None:
            _need("dit x", x, (s.B // 2) * s.La * s.latent)
            _need("dit pooled", pooled, s.B * s.H)
            _need("dit text", text, s.B * s.Lt * s.H, optional=s.Lt == 0)
        if X is not None:
            _need("dit X", X, s.B * S * s.H)
            _need("dit g", g, s.B * s.H)

    def forward(self, z, t, text, pooled, v):
        self._io(z=z, text=text, pooled=pooled, v=v)
        call("tsn_dit_forward", self.h, z.p, float(t), text.p if text is not None else None, pooled.p, v.p)

    def forward_ex(self, z, t_dev, text, pooled, v, taps=None):
        self._io(z=z, t_dev=t_dev, text=text, pooled=pooled, v=v, taps=taps)
        call("tsn_dit_forward_ex", self.h, z.p, t_dev.p, text.p if text is not None else None, pooled.p, v.p,
             taps.p if taps is not None else None)

    def joint_block(self, block, X, g):
        self._io(X=X, g=g)
        call("tsn_dit_joint_block", self.h, block, X.p, g.p)

    def fused_block(self, block, X, g):
        self._io(X=X, g=g)
        call("tsn_dit_fused_block", self.h, block, X.p, g.p)

    def sample(self, x, text, pooled, steps, cfg):
        self._io(x=x, text=text, pooled=pooled)
        call("tsn_dit_sample", self.h, x.p, _p(text), pooled.p, steps, cfg)

    def capture_forward(self, z, t_dev, text, pooled, v):
        self._io(z=z, t_dev=t_dev, text=text, pooled=pooled, v=v)
        call("tsn_dit_capture_forward", self.h, z.p, t_dev.p, _p(text), pooled.p, v.p)

    def capture_sample(self, x, text, pooled, steps, cfg):
        self._io(x=x, text=text, pooled=pooled)
        call("tsn_dit_capture_sample", self.h, x.p, _p(text), pooled.p, steps, cfg)

    def replay(self):
        call("tsn_dit_replay", self.h)

    def profile_forward(self, z, t_dev, text, pooled, v):
        """Per-kernel stats of one eager evaluation: list of dicts (name, launches, ms, flops, bytes)."""
        self._io(z=z, t_dev=t_dev, text=text, pooled=pooled, v=v)
        cap = 64
        arr = (KernelStat * cap)()
        n = ctypes.c_int()
        call("tsn_dit_profile_forward", self.h, z.p, t_dev.p, text.p, pooled.p, v.p, arr, cap, ctypes.byref(n))
        return [{"name": arr[i].name.decode(), "launches": arr[i].launches, "ms": arr[i].total_ms,
                 "flops": arr[i].flops, "bytes": arr[i].bytes} for i in range(n.value)]


def _p(a):
    return a.p if a is not None else None


class RefDitModel:
    """tn::DitModel mirror (src/models.h:55-85) for the reference checkpoint's three-stream graph."""

    def __init__(self, rt, spec):
        self.rt, self.spec = rt, spec
        h = ctypes.c_void_p()
        call("tsn_refdit_create", rt.h, ctypes.byref(spec), ctypes.byref(h))
        self.h = h

    def close(self):
        if self.h:
            lib().tsn_refdit_destroy(self.h)
            self.h = None

    def upload_weights(self, w_bf16):
        w_bf16 = np.ascontiguousarray(w_bf16, dtype=np.uint16)
        call("tsn_refdit_upload_weights", self.h, ptr(w_bf16), w_bf16.size)

    def upload_weights_f32(self, w):
        w = np.ascontiguousarray(w, dtype=np.float32)
        call("tsn_refdit_upload_weights_f32", self.h, ptr(w), w.size)

    def load_gguf(self, path):
        call("tsn_refdit_load_gguf", self.h, os.fsencode(path))

    def _io(self, x, clip_pp, text_pp, gcmlp, sync_gather, flow=None, t_dev=None, taps=None, sampler=False):
        s = self.spec
        rows = s.B // 2 if sampler else s.B
        _need("refdit x", x, rows * s.T * s.latent)
        _need("refdit flow", flow, s.B * s.T * s.latent, optional=sampler)
        _need("refdit t", t_dev, s.B, optional=True)
        _need("refdit clip_pp", clip_pp, s.B * s.C * s.H, optional=s.C == 0)
        _need("refdit text_pp", text_pp, s.B * s.TS * s.H, optional=s.TS == 0)
        _need("refdit gcmlp", gcmlp, s.B * s.H)
        _need("refdit sync_gather", sync_gather, s.B * s.T * s.H)
        _need("refdit taps", taps, (s.n_joint + s.n_fused) * s.B * (s.T + s.C + s.TS) * s.H, optional=True)

    def forward(self, x, t, clip_pp, text_pp, gcmlp, sync_gather, flow):
        self._io(x, clip_pp, text_pp, gcmlp, sync_gather, flow)
        call("tsn_refdit_forward", self.h, x.p, float(t), _p(clip_pp), _p(text_pp), gcmlp.p, sync_gather.p, flow.p)

    def forward_ex(self, x, t_dev, clip_pp, text_pp, gcmlp, sync_gather, flow, taps=None):
        self._io(x, clip_pp, text_pp, gcmlp, sync_gather, flow, t_dev, taps)
        call("tsn_refdit_forward_ex", self.h, x.p, t_dev.p, _p(clip_pp), _p(text_pp), gcmlp.p, sync_gather.p,
             flow.p, _p(taps))

    def sample(self, x, clip_pp, text_pp, gcmlp, sync_gather, steps, cfg):
        self._io(x, clip_pp, text_pp, gcmlp, sync_gather, sampler=True)
        call("tsn_refdit_sample", self.h, x.p, _p(clip_pp), _p(text_pp), gcmlp.p, sync_gather.p, steps, cfg)

    def capture_forward(self, x, t_dev, clip_pp, text_pp, gcmlp, sync_gather, flow):
        self._io(x, clip_pp, text_pp, gcmlp, sync_gather, flow, t_dev)
        call("tsn_refdit_capture_forward", self.h, x.p, t_dev.p, _p(clip_pp), _p(text_pp), gcmlp.p,
             sync_gather.p, flow.p)

    def capture_sample(self, x, clip_pp, text_pp, gcmlp, sync_gather, steps, cfg):
        self._io(x, clip_pp, text_pp, gcmlp, sync_gather, sampler=True)
        call("tsn_refdit_capture_sample", self.h, x.p, _p(clip_pp), _p(text_pp), gcmlp.p, sync_gather.p, steps, cfg)

    def replay(self):
        call("tsn_refdit_replay", self.h)

    def profile_forward(self, x, t_dev, clip_pp, text_pp, gcmlp, sync_gather, flow):
        self._io(x, clip_pp, text_pp, gcmlp, sync_gather, flow, t_dev)
        cap = 64
        arr = (KernelStat * cap)()
        n = ctypes.c_int()
        call("tsn_refdit_profile_forward", self.h, x.p, t_dev.p, _p(clip_pp), _p(text_pp), gcmlp.p, sync_gather.p,
             flow.p, arr, cap, ctypes.byref(n))
        return [{"name": arr[i].name.decode(), "launches": arr[i].launches, "ms": arr[i].total_ms,
                 "flops": arr[i].flops, "bytes": arr[i].bytes} for i in range(n.value)]


# Input index space of the synthetic generator (weights use their manifest index).
IDX_Z, IDX_TEXT, IDX_POOLED, IDX_T, IDX_G, IDX_X = 1000, 1001, 1002, 1003, 1004, 1005


def synth_inputs(spec, seed=4242, cfg_pairs=False):
    """Seeded inputs of a workload. cfg_pairs: samples come in (cond, uncond) pairs — the
    unconditional arm gets zeroed text and pooled features, both arms share z and t."""
    B, La, Lt, H, lat = spec.B, spec.La, spec.Lt, spec.H, spec.latent
    if cfg_pairs:
        P = B // 2
        z1 = synth_normal_f32(seed, IDX_Z, 0.0, 1.0, (P, La, lat))
        z = np.repeat(z1, 2, axis=0)
        text = np.zeros((B, Lt, H), np.float32)
        pooled = np.zeros((B, H), np.float32)
        text[0::2] = synth_normal_f32(seed, IDX_TEXT, 0.0, 1.0, (P, Lt, H))
        pooled[0::2] = synth_normal_f32(seed, IDX_POOLED, 0.0, 1.0, (P, H))
        t = np.repeat(synth_uniform_f32(seed, IDX_T, 0.0, 1.0, (1,)), B).astype(np.float32)
    else:
        z = synth_normal_f32(seed, IDX_Z, 0.0, 1.0, (B, La, lat))
        text = synth_normal_f32(seed, IDX_TEXT, 0.0, 1.0, (B, Lt, H))
        pooled = synth_normal_f32(seed, IDX_POOLED, 0.0, 1.0, (B, H))
        t = np.repeat(synth_uniform_f32(seed, IDX_T, 0.0, 1.0, (1,)), B).astype(np.float32)
    return {"z": z, "t": t, "text": text, "pooled": pooled}


def synth_prompt_inputs(spec, prompt_seeds, t_seed=4242):
    """Independent prompts as (cond, uncond) pairs: prompt p's latent, text and pooled features come
    from its own seed prompt_seeds[p] (the batch-16 throughput workload uses seeds 1..8), the
    unconditional arm of each pair gets zeroed text and pooled features, and every sample shares
    one t drawn from t_seed."""
    B, La, Lt, H, lat = spec.B, spec.La, spec.Lt, spec.H, spec.latent
    if len(prompt_seeds) * 2 != B:
        raise ValueError("need B/2 = %d prompt seeds, got %d" % (B // 2, len(prompt_seeds)))
    z = np.empty((B, La, lat), np.float32)
    text = np.zeros((B, Lt, H), np.float32)
    pooled = np.zeros((B, H), np.float32)
    for p, s in enumerate(prompt_seeds):
        z[2 * p] = z[2 * p + 1] = synth_normal_f32(s, IDX_Z, 0.0, 1.0, (La, lat))
        text[2 * p] = synth_normal_f32(s, IDX_TEXT, 0.0, 1.0, (Lt, H))
        pooled[2 * p] = synth_normal_f32(s, IDX_POOLED, 0.0, 1.0, (H,))
    t = np.repeat(synth_uniform_f32(t_seed, IDX_T, 0.0, 1.0, (1,)), B).astype(np.float32)
    return {"z": z, "t": t, "text": text, "pooled": pooled}


IDX_CLIP, IDX_GCMLP, IDX_SYNC = 1006, 1007, 1008


def ref_synth_inputs(spec, seed=4242, cfg_pairs=False):
    """Seeded inputs of the reference graph: x [B,T,latent], t [B], clip_pp [B,C,H], text_pp [B,TS,H],
    gcmlp [B,H], sync_gather [B,T,H]. cfg_pairs: (cond, uncond) pairs share x, t, clip_pp and
    sync_gather (src/pipeline.cpp:146-147); the unconditional arm has its own text_pp and gcmlp."""
    B, T, C, TS, H, lat = spec.B, spec.T, spec.C, spec.TS, spec.H, spec.latent
    n = B // 2 if cfg_pairs else B
    rep = (lambda a: np.repeat(a, 2, axis=0)) if cfg_pairs else (lambda a: a)
    x = rep(synth_normal_f32(seed, IDX_X, 0.0, 1.0, (n, T, lat)))
    clip = rep(synth_normal_f32(seed, IDX_CLIP, 0.0, 1.0, (n, C, H)))
    sync = rep(synth_normal_f32(seed, IDX_SYNC, 0.0, 1.0, (n, T, H)))
    text = synth_normal_f32(seed, IDX_TEXT, 0.0, 1.0, (B, TS, H))
    gcmlp = synth_normal_f32(seed, IDX_GCMLP, 0.0, 1.0, (B, H))
    t = np.repeat(synth_uniform_f32(seed, IDX_T, 0.0, 1.0, (1,)), B).astype(np.float32)
    return {"x": x, "t": t, "clip_pp": clip, "text_pp": text, "gcmlp": gcmlp, "sync_gather": sync}
