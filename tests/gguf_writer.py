"""Minimal GGUF v3 writer for tests: header, typed metadata, tensor infos, aligned data section.

Follows the layout src/gguf.rs:1-10 documents and src/gguf.rs:225-286 parses (the same layout
src/gguf_write.rs:121-166 emits): magic "GGUF", u32 version, u64 tensor count, u64 KV count, KVs
(u64-length string key, u32 type, payload), tensor infos (name, u32 n_dims, u64 dims with dims[0] the
contiguous axis, u32 ggml type, u64 offset relative to the data section), zero padding to
general.alignment, tensor data at those offsets.
"""
import struct

import numpy as np

# GGUF metadata value types (src/gguf.rs:196-223).
U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B", U64: "<Q",
        I64: "<q", F64: "<d"}


def _str(s):
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _payload(vt, v):
    if vt == STR:
        return _str(v)
    if vt == ARR:
        et, items = v
        return struct.pack("<IQ", et, len(items)) + b"".join(_payload(et, x) for x in items)
    return struct.pack(_FMT[vt], v)


def gguf_bytes(meta, tensors, alignment=32, version=3):
    """meta: {key: (vtype, value)} (ARR value = (elem_type, [items])).
    tensors: {name: (raw bytes-like, ggml_type, dims)} with dims in GGUF order (dims[0] contiguous).
    An alignment other than the default 32 is recorded as general.alignment unless meta sets it."""
    if alignment != 32 and "general.alignment" not in meta:
        meta = dict(meta, **{"general.alignment": (U32, alignment)})
    out = bytearray(b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(meta)))
    for k, (vt, v) in meta.items():
        out += _str(k) + struct.pack("<I", vt) + _payload(vt, v)
    offs, cur = [], 0
    blobs = [np.ascontiguousarray(raw).view(np.uint8).tobytes() for raw, _, _ in tensors.values()]
    for b in blobs:
        offs.append(cur)
        cur = -(-(cur + len(b)) // alignment) * alignment
    for (name, (_, t, dims)), off in zip(tensors.items(), offs):
        out += _str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        out += struct.pack("<IQ", t, off)
    out += b"\0" * (-len(out) % alignment)
    base = len(out)
    for b, off in zip(blobs, offs):
        out += b"\0" * (base + off - len(out))
        out += b
    return bytes(out)


def model_meta(cfg, arch, extra=None, omit=()):
    """The metadata keys Model::load reads (src/model.rs:721-771) for a ModelConfig-like cfg."""
    m = {
        "general.architecture": (STR, arch),
        f"{arch}.embedding_length": (U32, cfg.dim),
        f"{arch}.block_count": (U32, cfg.n_layers),
        f"{arch}.attention.head_count": (U32, cfg.n_heads),
        f"{arch}.attention.head_count_kv": (U32, cfg.n_kv_heads),
        f"{arch}.feed_forward_length": (U32, cfg.ffn_dim),
        f"{arch}.attention.layer_norm_rms_epsilon": (F32, cfg.rms_eps),
        f"{arch}.rope.freq_base": (F32, cfg.rope_base),
        f"{arch}.attention.key_length": (U32, cfg.head_dim),
        "tokenizer.ggml.tokens": (ARR, (STR, [f"t{i}" for i in range(8)])),
        "tokenizer.ggml.scores": (ARR, (F32, [0.5] * 8)),
    }
    for k in omit:
        m.pop(k.replace("{arch}", arch))
    m.update(extra or {})
    return m


def model_tensors(tensors, norm_type=0):
    """{name: (raw, type, rows, cols)} as hos_peft_set_tensor takes them -> writer form. 1-D tensors
    (norms, biases) are written as F32 (norm_type 0) or F16 (norm_type 1)."""
    out = {}
    for name, (raw, t, rows, cols) in tensors.items():
        if rows == 1 and t == 0:
            v = np.frombuffer(np.ascontiguousarray(raw).view(np.uint8).tobytes(), np.float32)
            if norm_type == 1:
                out[name] = (v.astype(np.float16), 1, [cols])
            else:
                out[name] = (v, 0, [cols])
        else:
            out[name] = (raw, t, [cols, rows])
    return out
