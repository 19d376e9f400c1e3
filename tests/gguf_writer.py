"""Minimal GGUF v3 writer for tests (test infrastructure, not part of the library).

Writes the header (magic "GGUF", version, tensor count, metadata count), typed metadata, tensor
infos (name, dims with ne[0] fastest, GGML type, offset) and the data section aligned to
`general.alignment`. Tensor types: F32 (0), F16 (1), Q8_0 (8: blocks of 32 = f16 scale + 32 int8)
and BF16 (30). Returns, per tensor, the values a reader must produce (f16 subnormals flushed to
zero, Q8_0 = f16 scale * int8).
"""
import struct

import numpy as np

F32, F16, Q8_0, BF16 = 0, 1, 8, 30
KV_U32, KV_I32, KV_F32, KV_BOOL, KV_STRING, KV_ARRAY, KV_U64, KV_F64 = 4, 5, 6, 7, 8, 9, 10, 12


def _s(x):
    b = x.encode()
    return struct.pack("<Q", len(b)) + b


def _kv(key, kind, value):
    out = _s(key) + struct.pack("<I", kind)
    if kind == KV_U32:
        out += struct.pack("<I", value)
    elif kind == KV_I32:
        out += struct.pack("<i", value)
    elif kind == KV_U64:
        out += struct.pack("<Q", value)
    elif kind == KV_F32:
        out += struct.pack("<f", value)
    elif kind == KV_F64:
        out += struct.pack("<d", value)
    elif kind == KV_BOOL:
        out += struct.pack("<B", 1 if value else 0)
    elif kind == KV_STRING:
        out += _s(value)
    elif kind == KV_ARRAY:
        et, items = value
        out += struct.pack("<IQ", et, len(items))
        for it in items:
            out += _s(it) if et == KV_STRING else struct.pack({KV_U32: "<I", KV_F32: "<f", KV_I32: "<i"}[et], it)
    else:
        raise ValueError(kind)
    return out


def f16_ftz(h):
    """f16 array -> f32 with subnormals flushed to signed zero"""
    f = h.astype(np.float32)
    sub = (h.view(np.uint16) & 0x7C00) == 0
    f[sub] = np.copysign(0.0, f[sub])
    return f


def encode(x, ttype):
    """tensor payload bytes and the f32 values a reader returns"""
    x = np.ascontiguousarray(x, np.float32).ravel()
    if ttype == F32:
        return x.tobytes(), x.copy()
    if ttype == F16:
        h = x.astype(np.float16)
        return h.tobytes(), f16_ftz(h)
    if ttype == BF16:
        u = x.view(np.uint32)
        b = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)   # round to nearest even
        return b.tobytes(), (b.astype(np.uint32) << 16).view(np.float32)
    if ttype == Q8_0:
        assert x.size % 32 == 0
        blk = x.reshape(-1, 32)
        amax = np.abs(blk).max(1)
        scale = (amax / 127.0).astype(np.float16)
        sf = scale.astype(np.float32)
        q = np.where(sf[:, None] > 0, np.round(blk / np.where(sf > 0, sf, 1)[:, None]), 0)
        q = np.clip(q, -127, 127).astype(np.int8)
        raw = b"".join(s.tobytes() + qq.tobytes() for s, qq in zip(scale, q))
        dec = (f16_ftz(scale)[:, None] * q.astype(np.float32)).ravel()
        return raw, dec
    raise ValueError(ttype)


def write(path, tensors, metadata=(), alignment=32, version=3):
    """tensors: list of (name, ne tuple (ne[0] fastest), ggml type, f32 values);
    metadata: list of (key, kind, value). Returns {name: decoded f32 values}."""
    meta = list(metadata)
    if alignment != 32:
        meta.append(("general.alignment", KV_U32, alignment))
    head = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(meta))
    head += b"".join(_kv(k, kind, v) for k, kind, v in meta)
    blobs, decoded, infos, off = [], {}, b"", 0
    for name, ne, ttype, vals in tensors:
        raw, dec = encode(vals, ttype)
        assert int(np.prod(ne)) == dec.size, name
        pad = (-off) % alignment
        blobs.append(b"\0" * pad + raw)
        off += pad
        infos += _s(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", n) for n in ne)
        infos += struct.pack("<IQ", ttype, off)
        off += len(raw)
        decoded[name] = dec
    hdr = head + infos
    hdr += b"\0" * ((-len(hdr)) % alignment)
    with open(path, "wb") as f:
        f.write(hdr)
        f.write(b"".join(blobs))
    return decoded


def ref_ne(name, numel, spec):
    """GGUF dims (ne[0] fastest) of a reference-graph tensor: conv [OC][IC][K] -> (K, IC, OC),
    linear [N][K] -> (K, N), vectors (n,)"""
    H, F, L = spec["H"], spec["F"], spec["latent"]
    if not name.endswith(".weight") or "norm" in name:
        return (numel,)
    if name == "final_layer.conv.weight":
        return (7, H, L)
    if name == "audio_input_proj.0.weight":
        return (3, L, H)
    if name.endswith("ffn.w1.weight") or name.endswith("ffn.w3.weight") or ".2.w1." in name or ".2.w3." in name:
        return (3, H, F) if numel == 3 * H * F else (H, F)
    if name.endswith("w2.weight"):
        return (3, F, H) if numel == 3 * H * F else (F, H)
    if name.endswith("linear1.weight"):
        return (3, H, H) if numel == 3 * H * H else (H, H)
    return (H, numel // H)


def write_bf16(path, tensors, metadata=(), alignment=32, version=3):
    """BF16 tensors given as raw bf16 bits, streamed to the file one tensor at a time (for
    checkpoints of reference size, without an f32 copy in memory). tensors: list of (name, ne tuple
    (ne[0] fastest), uint16 array). Returns the file size in bytes."""
    meta = list(metadata)
    if alignment != 32:
        meta.append(("general.alignment", KV_U32, alignment))
    head = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(meta))
    head += b"".join(_kv(k, kind, v) for k, kind, v in meta)
    infos, off, offs = b"", 0, []
    for name, ne, bits in tensors:
        assert bits.dtype == np.uint16 and int(np.prod(ne)) == bits.size, name
        off += (-off) % alignment
        offs.append(off)
        infos += _s(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", n) for n in ne)
        infos += struct.pack("<IQ", BF16, off)
        off += 2 * bits.size
    hdr = head + infos
    hdr += b"\0" * ((-len(hdr)) % alignment)
    with open(path, "wb") as f:
        f.write(hdr)
        pos = 0
        for (name, ne, bits), o in zip(tensors, offs):
            f.write(b"\0" * (o - pos))
            np.ascontiguousarray(bits).tofile(f)
            pos = o + 2 * bits.size
    return len(hdr) + pos
