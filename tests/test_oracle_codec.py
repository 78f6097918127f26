"""Pins the oracle's GGUF codec (restating src/gguf.rs + src/gguf_write.rs).

Known-answer vectors follow tests/gguf_codec.rs:99-263 (independent encoders, exact
decode) and extend them to the K-quants, which the reference only checks on real model
files (tests/gguf_codec.rs:292-331, absent here). Round-trip bounds follow
src/gguf_write.rs:558-659.
"""
import numpy as np
import pytest

from oracle import binding as o

F32, F16, Q4_0, Q5_0, Q8_0, Q4_K, Q5_K, Q6_K, BF16 = 0, 1, 2, 6, 8, 12, 13, 14, 30


def f16le(x):
    return np.array([x], np.float16).view(np.uint8).tolist()


def test_f16_encode_matches_ieee_rne():
    rng = np.random.default_rng(1)
    bits = rng.integers(0, 2**32, size=20000, dtype=np.uint64).astype(np.uint32)
    edge = np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 2**-24, 2**-25, 2**-25 * 1.0001, 3 * 2**-26,
                     6.1035156e-05, 6.1e-05, 1.0 + 2**-11, 1.0 + 3 * 2**-11, np.inf, -np.inf], np.float32)
    f = np.concatenate([bits.view(np.float32), edge, (rng.standard_normal(5000) * 1e-5).astype(np.float32)])
    f = f[np.isfinite(f)]
    with np.errstate(over="ignore"):
        ref = f.astype(np.float16).view(np.uint16)
    got = np.array([o.f32_to_f16_bits(v) for v in f], np.uint16)
    assert np.array_equal(got, ref)


def test_f16_decode_exact_all_codes():
    h = np.arange(65536, dtype=np.uint16)
    ref = h.view(np.float16).astype(np.float32)
    got = np.array([o.f16_bits_to_f32(x) for x in h], np.float32)
    same = (got.view(np.uint32) == ref.view(np.uint32)) | (np.isnan(got) & np.isnan(ref))
    assert same.all()


def test_dequant_f32_exact():  # tests/gguf_codec.rs:153-170
    vals = np.array([0.0, 1.5, -2.25, 3.5, -100.0, 42.0], np.float32)
    assert np.array_equal(o.dequant(vals.view(np.uint8), F32, 6), vals)


def test_dequant_f16_bf16():  # tests/gguf_codec.rs:173-190
    vals = np.array([0.0, 1.0, -2.5, 0.5, 0.25, 3.0, -7.0, 0.125], np.float32)
    assert np.array_equal(o.dequant(vals.astype(np.float16).view(np.uint8), F16, 8), vals)
    bf = (vals.view(np.uint32) >> 16).astype(np.uint16)
    assert np.array_equal(o.dequant(bf.view(np.uint8), BF16, 8), vals)


def enc_q8_0(vals, d):  # tests/gguf_codec.rs:109-119
    b = []
    for blk in vals.reshape(-1, 32):
        b += f16le(d)
        b += [int(np.round(v / d)) & 0xFF for v in blk]
    return np.array(b, np.uint8)


def test_dequant_q8_0_exact():  # tests/gguf_codec.rs:193-215
    d = 0.5
    vals = np.array([((i - 32) % 40) * d if (i - 32) >= 0 else -((32 - i) % 40) * d for i in range(64)], np.float32)
    assert np.array_equal(o.dequant(enc_q8_0(vals, d), Q8_0, 64), vals)


def test_dequant_q4_0_q5_0_exact():  # tests/gguf_codec.rs:218-263
    d = 0.25
    vals = np.array([((i % 16) - 8) * d for i in range(32)], np.float32)
    b = f16le(d) + [(((int(vals[j] / d) + 8) & 15) | (((int(vals[j + 16] / d) + 8) & 15) << 4)) for j in range(16)]
    assert np.array_equal(o.dequant(np.array(b, np.uint8), Q4_0, 32), vals)
    d = 0.5
    vals = np.array([(b_ - 16) * d for b_ in range(32)], np.float32)
    qh, qs = 0, [0] * 16
    for e, v in enumerate(vals):
        code = int(round(v / d)) + 16
        if code & 16:
            qh |= 1 << e
        if e < 16:
            qs[e] |= code & 15
        else:
            qs[e - 16] |= (code & 15) << 4
    raw = np.array(f16le(d) + list(int(qh).to_bytes(4, "little")) + qs, np.uint8)
    assert np.array_equal(o.dequant(raw, Q5_0, 32), vals)


def unpack_scale_min(j, q):
    """get_scale_min_k4 from the byte layout description (src/gguf.rs:43-51)."""
    if j < 4:
        return q[j] & 63, q[j + 4] & 63
    return (q[j + 4] & 15) | ((q[j - 4] >> 6) << 4), (q[j + 4] >> 4) | ((q[j] >> 6) << 4)


def test_pack_scales_mins_inverts_unpack():  # src/gguf_write.rs:268-285
    rng = np.random.default_rng(2)
    for _ in range(300):
        s = rng.integers(0, 64, 8).astype(np.uint8)
        m = rng.integers(0, 64, 8).astype(np.uint8)
        q = np.zeros(12, np.uint8)
        o.lib().orc_pack_scales_mins(s.ctypes.data, m.ctypes.data, q.ctypes.data)
        for j in range(8):
            assert unpack_scale_min(j, q.tolist()) == (s[j], m[j])


def hand_q4k(rng, d, dmin):
    """Independent Q4_K super-block encoder built from the layout: sub-block j (32 values)
    takes low nibbles of qs[32*(j//2):] for even j, high nibbles for odd j."""
    sc = rng.integers(0, 64, 8)
    mn = rng.integers(0, 64, 8)
    q = rng.integers(0, 16, 256)
    scales = np.zeros(12, np.int64)
    for j in range(8):
        if j < 4:
            scales[j] |= sc[j]
            scales[j + 4] |= mn[j]
        else:
            scales[j + 4] |= (sc[j] & 15) | ((mn[j] & 15) << 4)
            scales[j - 4] |= (sc[j] >> 4) << 6
            scales[j] |= (mn[j] >> 4) << 6
    qs = np.zeros(128, np.int64)
    for j in range(8):
        for l in range(32):
            qs[32 * (j // 2) + l] |= q[32 * j + l] << (4 * (j % 2))
    raw = np.array(f16le(d) + f16le(dmin) + scales.tolist() + qs.tolist(), np.uint8)
    # d, dmin powers of two and small integers: every product/difference is exact in f32
    exp = np.array([d * sc[e // 32] * q[e] - dmin * mn[e // 32] for e in range(256)], np.float64)
    return raw, exp.astype(np.float32)


def test_dequant_q4_k_hand_encoded():
    rng = np.random.default_rng(3)
    raws, exps = [], []
    for d, dmin in [(0.5, 0.25), (2.0**-6, 2.0**-7), (1.0, 0.0)]:
        r, e = hand_q4k(rng, d, dmin)
        raws.append(r)
        exps.append(e)
    got = o.dequant(np.concatenate(raws), Q4_K, 768)
    assert np.array_equal(got, np.concatenate(exps))


def test_dequant_q5_k_hand_encoded():
    rng = np.random.default_rng(4)
    d, dmin = 0.125, 0.0625
    sc, mn = rng.integers(0, 64, 8), rng.integers(0, 64, 8)
    q = rng.integers(0, 32, 256)
    scales = np.zeros(12, np.int64)
    for j in range(8):
        if j < 4:
            scales[j] |= sc[j]
            scales[j + 4] |= mn[j]
        else:
            scales[j + 4] |= (sc[j] & 15) | ((mn[j] & 15) << 4)
            scales[j - 4] |= (sc[j] >> 4) << 6
            scales[j] |= (mn[j] >> 4) << 6
    qs = np.zeros(128, np.int64)
    qh = np.zeros(32, np.int64)
    for j in range(8):
        for l in range(32):
            v = q[32 * j + l]
            qs[32 * (j // 2) + l] |= (v & 15) << (4 * (j % 2))
            if v & 16:
                qh[l] |= 1 << j
    raw = np.array(f16le(d) + f16le(dmin) + scales.tolist() + qh.tolist() + qs.tolist(), np.uint8)
    exp = np.array([d * sc[e // 32] * q[e] - dmin * mn[e // 32] for e in range(256)], np.float32)
    assert np.array_equal(o.dequant(raw, Q5_K, 256), exp)


def hand_q6k(rng, d):
    """Independent Q6_K encoder from the layout (src/gguf.rs:449-477): value e in half
    n128 = e//128, l = e%32, quarter qq = (e%128)//32; low 4 bits from ql[64*n128 + l + 32*(qq&1)]
    (high nibble when qq >= 2), high 2 bits from qh[32*n128 + l] >> (2*qq); scale sc[e//16]."""
    sc = rng.integers(-128, 128, 16)
    q = rng.integers(-32, 32, 256)
    ql = np.zeros(128, np.int64)
    qh = np.zeros(64, np.int64)
    for e in range(256):
        n128, r = divmod(e, 128)
        qq, l = divmod(r, 32)
        u = q[e] + 32
        ql[64 * n128 + l + 32 * (qq & 1)] |= (u & 15) << (4 * (qq >> 1))
        qh[32 * n128 + l] |= (u >> 4) << (2 * qq)
    raw = np.array(ql.tolist() + qh.tolist() + [int(s) & 0xFF for s in sc] + f16le(d), np.uint8)
    exp = np.array([d * sc[e // 16] * q[e] for e in range(256)], np.float32)
    return raw, exp


def test_dequant_q6_k_hand_encoded():
    rng = np.random.default_rng(5)
    r1, e1 = hand_q6k(rng, 2.0**-8)
    r2, e2 = hand_q6k(rng, 1.0)
    got = o.dequant(np.concatenate([r1, r2]), Q6_K, 512)
    assert np.array_equal(got, np.concatenate([e1, e2]))


def test_bytes_for():  # src/gguf.rs:548-561
    assert [o.bytes_for(t, 512) for t in (F32, F16, Q8_0, Q4_0, Q5_0, Q4_K, Q5_K, Q6_K)] == \
        [2048, 1024, 544, 288, 352, 288, 352, 420]


def test_q8_0_quantizer_kat():
    """Exact-grid input: amax = 127·d with d a power of two -> d and every q known."""
    d = 2.0**-7
    q = np.concatenate([np.arange(-127, 128, 8), [127]])[:32].astype(np.int64)
    q[0] = 127
    x = (q * d).astype(np.float32)
    raw = o.quantize(x, Q8_0)
    assert raw[:2].tolist() == f16le(d)
    assert raw[2:].view(np.int8).tolist() == q.tolist()


def test_q8_0_roundtrip_bound():  # src/gguf_write.rs:563-589
    n = 256
    x = (np.sin(np.arange(n, dtype=np.float32) * np.float32(0.013)) * 3 - 1).astype(np.float32)
    out = o.dequant(o.quantize(x, Q8_0), Q8_0, n)
    for b in range(n // 32):
        blk = slice(32 * b, 32 * b + 32)
        tol = np.abs(x[blk]).max() / 127 + 1e-4
        assert np.all(np.abs(x[blk] - out[blk]) <= tol)


@pytest.mark.parametrize("t,levels", [(Q4_0, 8.0), (Q5_0, 16.0)])
def test_qx_0_roundtrip_bound(t, levels):  # src/gguf_write.rs:591-621
    n = 256
    x = (np.sin(np.arange(n, dtype=np.float32) * np.float32(0.017)) * 4 - 0.7).astype(np.float32)
    out = o.dequant(o.quantize(x, t), t, n)
    for b in range(n // 32):
        blk = slice(32 * b, 32 * b + 32)
        tol = np.abs(x[blk]).max() / levels + 1e-3
        assert np.all(np.abs(x[blk] - out[blk]) <= tol)


@pytest.mark.parametrize("t,rel", [(Q4_K, 0.08), (Q5_K, 0.04), (Q6_K, 0.02)])
def test_k_roundtrip_bound(t, rel):  # src/gguf_write.rs:625-658
    n = 512
    x = (np.sin(np.arange(n, dtype=np.float32) * np.float32(0.011)) * 5 + 0.3).astype(np.float32)
    out = o.dequant(o.quantize(x, t), t, n)
    assert np.abs(x - out).max() <= rel * np.abs(x).max()


@pytest.mark.parametrize("t", [Q8_0, Q4_K, Q6_K])
def test_quantizer_gaussian_error_and_determinism(t):
    rng = np.random.default_rng(7)
    x = (rng.standard_normal(256 * 64) * 0.02).astype(np.float32)
    a = o.quantize(x, t)
    assert np.array_equal(a, o.quantize(x, t))
    y = o.dequant(a, t, x.size)
    rel = np.linalg.norm(y - x) / np.linalg.norm(x)
    assert rel < {Q8_0: 0.01, Q4_K: 0.12, Q6_K: 0.03}[t]


def test_qkx_scale_min_constant_block():  # src/gguf_write.rs:303-305 (mx == mn)
    assert o.qkx_scale_min(np.full(32, -0.5, np.float32), 15) == (0.0, 0.5)
    s, m = o.qkx_scale_min(np.linspace(0, 1.5, 32).astype(np.float32), 15)
    assert s > 0 and m >= 0.0
