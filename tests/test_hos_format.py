"""The .hos capsule oracle (oracle/hos_format.py) pinned, and the library's CPU-side card reader.

Pins: FNV-1a 64 against the published test vectors of the FNV reference suite; the reference's own
format tests (tests/hos_format.rs: bit-identical round trip with card fields, corruption detection,
non-HOS rejection, model_id stable and data-sensitive); the layout's invariants (32-byte aligned data,
file checksum over everything before it, v1 table without dtype / byte count). hos_format_card
(src/format.rs:270-285 read_card) is called on oracle-written files (no device work).
"""
import ctypes
import json
import os
import struct

import numpy as np
import pytest

from oracle import hos_format as hf

LIB = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "hos_amd", "libhos_hip.so")


def sample_tensors():
    """tests/hos_format.rs:19-34."""
    return [("blk.0.w", hf.ROLE_WEIGHT, [3, 2], np.array([0.5, -1.0, 2.0, 0.25, -0.75, 1.5], np.float32)),
            ("blk.0.norm", hf.ROLE_NORM, [2], np.array([1.0, 0.9], np.float32))]


def card_json(**kw):
    c = {"format": "hos", "spec": 1, "name": "test-model", "id": "", "mode": "trainable",
         "arch": {"layers": [], "type": "sequential"},
         "provenance": {"created": "", "engine": "hos", "dataset": "", "dataset_hash": ""},
         "resume": {"seed": 42, "step": 100, "rng_state": 0},
         "history": [{"steps": 100, "final_loss": 0.25, "optimizer": "adamw", "lr": 0.001}],
         "lineage": ["deadbeefdeadbeef"]}
    c.update(kw)
    return json.dumps(c, separators=(",", ":"))


@pytest.mark.parametrize("data,want", [
    (b"", 0xCBF29CE484222325), (b"a", 0xAF63DC4C8601EC8C), (b"foobar", 0x85944171F73967E8)])
def test_fnv1a64_published_vectors(data, want):
    assert hf.fnv1a64(data) == want


def test_round_trip_bit_identical():
    ts = sample_tensors()
    buf = hf.write(ts, card_json(id=hf.model_id(ts)))
    ver, card, out, file_ok = hf.read(buf)
    assert ver == 2 and file_ok
    for (n, r, s, d), (n2, r2, dt, s2, nf, raw) in zip(ts, out):
        assert (n, r, hf.DTYPE_F32, s, d.size) == (n2, r2, dt, s2, nf)
        assert np.frombuffer(raw, "<f4").tobytes() == d.tobytes()
    c = json.loads(card)
    assert c["name"] == "test-model" and c["id"] == hf.model_id(ts) and c["resume"]["step"] == 100
    assert c["lineage"] == ["deadbeefdeadbeef"] and c["history"][0]["steps"] == 100


def test_layout_invariants():
    ts = sample_tensors()
    buf = hf.write(ts, card_json())
    assert buf[:4] == b"HOSF" and struct.unpack("<II", buf[4:12]) == (2, 0)
    assert (len(buf) - 8) % 32 == 0  # data region padded to 32, then the u64 file checksum
    assert struct.unpack("<Q", buf[-8:])[0] == hf.fnv1a64(buf[:-8])
    # the last tensor's bytes end at the last 32-byte boundary before the padding
    raw = ts[-1][3].tobytes()
    assert buf[len(buf) - 8 - 32: len(buf) - 8 - 32 + len(raw)] == raw
    v1 = hf.write(ts, card_json(), version=1)
    ver, _, out, ok = hf.read(v1)
    assert ver == 1 and ok and [o[0] for o in out] == ["blk.0.w", "blk.0.norm"]


def test_corruption_detected():
    ts = [("w", hf.ROLE_WEIGHT, [256], (np.arange(256) * 0.01).astype(np.float32))]
    buf = bytearray(hf.write(ts, card_json()))
    hf.read(bytes(buf))
    buf[len(buf) // 2] ^= 0xFF
    with pytest.raises(ValueError, match="checksum"):
        hf.read(bytes(buf))


def test_rejects_non_hos():
    with pytest.raises(ValueError):
        hf.read(b"not a hos file at all")


def test_model_id_stable_and_sensitive():
    a, b, c = sample_tensors(), sample_tensors(), sample_tensors()
    assert hf.model_id(a) == hf.model_id(b)
    c[0][3][0] += np.float32(1e-4)
    assert hf.model_id(a) != hf.model_id(c)


def _card(path):
    from hos_amd._lib import lib
    need = ctypes.c_size_t()
    buf = ctypes.create_string_buffer(8192)
    rc = lib().hos_format_card(str(path).encode(), buf, len(buf), ctypes.byref(need))
    return rc, buf.value.decode(errors="replace"), need.value


@pytest.mark.skipif(not os.path.exists(LIB), reason="libhos_hip.so not built")
def test_library_reads_card(tmp_path):
    ts = sample_tensors()
    text = card_json(id=hf.model_id(ts))
    for ver in (1, 2):
        p = tmp_path / f"c{ver}.hos"
        p.write_bytes(hf.write(ts, text, version=ver))
        rc, got, need = _card(p)
        assert rc == 0 and got == text and need == len(text) + 1
    from hos_amd.peft import read_card
    assert read_card(tmp_path / "c2.hos")["lineage"] == ["deadbeefdeadbeef"]
    big = card_json(arch={"blob": "x" * 10000})
    (tmp_path / "big.hos").write_bytes(hf.write(ts, big))
    assert read_card(tmp_path / "big.hos")["arch"]["blob"] == "x" * 10000
    (tmp_path / "bad.hos").write_bytes(b"not a hos file at all")
    assert _card(tmp_path / "bad.hos")[0] == 2
    assert _card(tmp_path / "absent.hos")[0] == 1
    (tmp_path / "trunc.hos").write_bytes(hf.write(ts, text)[:30])
    assert _card(tmp_path / "trunc.hos")[0] == 2


def _verify(path):
    from hos_amd._lib import lib
    n = ctypes.c_size_t()
    err = ctypes.create_string_buffer(256)
    rc = lib().hos_format_verify(str(path).encode(), ctypes.byref(n), err, len(err))
    return rc, n.value, err.value.decode(errors="replace")


@pytest.mark.skipif(not os.path.exists(LIB), reason="libhos_hip.so not built")
def test_library_verifies_capsules_and_survives_fuzz(tmp_path):
    """hos_format_verify (load_raw, src/format.rs:401-485): oracle-written v1/v2 capsules verify; every
    truncation and random byte flip (tests/fuzz_gguf.rs-style robustness for the second file parser) returns
    a status — ok only if the bytes still verify — and never crashes."""
    ts = sample_tensors()
    for ver in (1, 2):
        p = tmp_path / f"v{ver}.hos"
        p.write_bytes(hf.write(ts, card_json(), version=ver))
        assert _verify(p)[:2] == (0, 2)
    good = hf.write(ts, card_json(), version=2)
    p = tmp_path / "fz.hos"
    rng = np.random.default_rng(17)
    for cut in range(0, len(good), 7):
        p.write_bytes(good[:cut])
        # load_raw does not read the file checksum trailer, so only cuts into the tensor data must fail
        assert _verify(p)[0] == 2 if cut <= len(good) // 2 else _verify(p)[0] in (0, 2)
    for _ in range(400):
        b = bytearray(good)
        for _ in range(1 + rng.integers(3)):
            b[rng.integers(len(b))] ^= int(rng.integers(1, 256))
        p.write_bytes(bytes(b))
        assert _verify(p)[0] in (0, 2, 4)
    for _ in range(100):
        p.write_bytes(b"HOSF" + rng.integers(0, 256, int(rng.integers(0, 300)), dtype=np.uint8).tobytes())
        assert _verify(p)[0] in (0, 2, 4)
