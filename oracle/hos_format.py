"""ORACLE — test infrastructure only.

A restatement of HOS's ``.hos`` capsule format (src/format.rs) used by the tests to check what the
library writes and to make files for it to read. Only ``tests/`` may import this module.

  fnv1a64         src/format.rs:183-190 (FNV-1a 64; docs/HOS_FORMAT.md:17-18)
  model_id        src/format.rs:100-111
  write (v1, v2)  src/format.rs:287-346 (v2, all tensors F32) and the v1 table of :10-16
  load_raw        src/format.rs:401-485 (per-tensor checksum verified)
"""
import struct

import numpy as np

MAGIC = b"HOSF"
ROLE_WEIGHT, ROLE_BIAS, ROLE_NORM, ROLE_EMBED, ROLE_OPT_STATE, ROLE_SCALAR = range(6)
DTYPE_F32, DTYPE_Q8_0 = 0, 1
FNV_OFFSET, FNV_PRIME, MASK = 0xCBF29CE484222325, 0x100000001B3, (1 << 64) - 1


def fnv1a64(data, h=FNV_OFFSET):
    for b in bytes(data):
        h = ((h ^ b) * FNV_PRIME) & MASK
    return h


def model_id(tensors):
    """tensors: [(name, role, shape, f32 array)] -> 16 hex digits over every tensor's f32 LE bytes."""
    h = FNV_OFFSET
    for _, _, _, data in tensors:
        h = fnv1a64(np.ascontiguousarray(data, "<f4").tobytes(), h)
    return f"{h:016x}"


def _pad32(b):
    b += b"\0" * (-len(b) % 32)


def write(tensors, card, version=2, stored=None):
    """Bytes of a capsule. tensors: [(name, role, shape, f32 array)]; card: JSON text.
    stored: optional {name: (dtype, raw bytes)} to store a tensor in another encoding (v2 only)."""
    stored = stored or {}
    cb = card.encode()
    b = bytearray(MAGIC + struct.pack("<III", version, 0, len(cb)) + cb + struct.pack("<I", len(tensors)))
    blobs = []
    for name, role, shape, data in tensors:
        data = np.ascontiguousarray(data, "<f4").ravel()
        dtype, raw = stored.get(name, (DTYPE_F32, data.tobytes()))
        blobs.append(raw)
        nb = name.encode()
        b += struct.pack("<I", len(nb)) + nb + struct.pack("<B", role)
        if version >= 2:
            b += struct.pack("<B", dtype)
        b += struct.pack("<I", len(shape)) + b"".join(struct.pack("<I", d) for d in shape)
        b += struct.pack("<Q", data.size)
        if version >= 2:
            b += struct.pack("<Q", len(raw))
        b += struct.pack("<Q", fnv1a64(raw))
    _pad32(b)
    for raw in blobs:
        b += raw
        _pad32(b)
    b += struct.pack("<Q", fnv1a64(b))
    return bytes(b)


def read(buf):
    """(version, card text, [(name, role, dtype, shape, nfloats, raw bytes)], file checksum ok)."""
    p = 0

    def take(n):
        nonlocal p
        if p + n > len(buf):
            raise ValueError("truncated")
        r = buf[p:p + n]
        p += n
        return r

    if take(4) != MAGIC:
        raise ValueError("not a HOS file")
    ver, _flags, clen = struct.unpack("<III", take(12))
    card = take(clen).decode()
    (n,) = struct.unpack("<I", take(4))
    metas = []
    for _ in range(n):
        (nl,) = struct.unpack("<I", take(4))
        name = take(nl).decode()
        role = take(1)[0]
        dtype = take(1)[0] if ver >= 2 else DTYPE_F32
        (nd,) = struct.unpack("<I", take(4))
        shape = list(struct.unpack(f"<{nd}I", take(4 * nd)))
        (nf,) = struct.unpack("<Q", take(8))
        nbytes = struct.unpack("<Q", take(8))[0] if ver >= 2 else nf * 4
        (ck,) = struct.unpack("<Q", take(8))
        metas.append((name, role, dtype, shape, nf, nbytes, ck))
    p += -p % 32
    out = []
    for name, role, dtype, shape, nf, nbytes, ck in metas:
        raw = take(nbytes)
        p += -p % 32
        if fnv1a64(raw) != ck:
            raise ValueError(f"checksum mismatch in tensor {name}")
        out.append((name, role, dtype, shape, nf, raw))
    (fck,) = struct.unpack("<Q", take(8))
    return ver, card, out, fck == fnv1a64(buf[:p - 8])
