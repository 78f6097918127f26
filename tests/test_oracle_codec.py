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


# ---- exact-byte pins of the K-quant quantizers (src/gguf_write.rs:293-495) ----
# Values placed exactly on a grid the reference's search provably recovers, so every output byte is known in
# closed form (header scales, packed 6-bit scales/mins, codes) without restating the algorithm; plus blocks that
# force each branch of qkx_scale_min.


def q4k_grid_block(rng, nmax=15):
    """A super-block whose sub-block j holds v = s_j·l − m_j, l integers in 0..nmax with both ends present,
    s_j = a_j·U, m_j = b_j·V (U, V powers of two, a_j, b_j in 1..63 with 63 present in each). Then for every
    sub-block the candidate iscale (nmax − 1 + 0.1·10)/span = 1/s_j recovers l exactly, the least-squares refit
    is exact (err 0, so (s_j, m_j) is returned), d = max s / 63 = U, dmin = V, ls = a, lm = b, codes = l."""
    U, V = 2.0 ** -9, 2.0 ** -8
    a = rng.integers(1, 64, 8)
    b = rng.integers(1, 64, 8)
    a[rng.integers(8)] = 63
    b[rng.integers(8)] = 63
    l = rng.integers(0, nmax + 1, (8, 32))
    l[:, 0], l[:, 1] = 0, nmax
    x = np.array([[a[j] * U * l[j, i] - b[j] * V for i in range(32)] for j in range(8)], np.float64)
    assert np.array_equal(x.astype(np.float32).astype(np.float64), x)  # the grid is exact in f32
    return x.astype(np.float32).ravel(), U, V, a, b, l


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_q4_k_quantizer_exact_bytes_on_grid(seed):
    x, U, V, a, b, l = q4k_grid_block(np.random.default_rng(seed))
    raw = o.quantize(x, Q4_K).tolist()
    assert raw[0:2] == f16le(U) and raw[2:4] == f16le(V)
    for j in range(8):
        assert unpack_scale_min(j, raw[4:16]) == (a[j], b[j])
    qs = raw[16:]
    for j in range(8):
        got = [(qs[32 * (j // 2) + i] >> (4 * (j % 2))) & 15 for i in range(32)]
        assert got == l[j].tolist()
    assert np.array_equal(o.dequant(np.array(raw, np.uint8), Q4_K, 256), x)  # and the round trip is exact


def test_q5_k_quantizer_exact_bytes_on_grid():
    x, U, V, a, b, l = q4k_grid_block(np.random.default_rng(5), nmax=31)
    raw = o.quantize(x, Q5_K).tolist()
    assert raw[0:2] == f16le(U) and raw[2:4] == f16le(V)
    for j in range(8):
        assert unpack_scale_min(j, raw[4:16]) == (a[j], b[j])
    qh, qs = raw[16:48], raw[48:]
    for j in range(8):
        got = [((qs[32 * (j // 2) + i] >> (4 * (j % 2))) & 15) | (((qh[i] >> j) & 1) << 4) for i in range(32)]
        assert got == l[j].tolist()


def test_q6_k_quantizer_exact_bytes_on_grid():
    """Sub-block s holds c_s·k with k integers in −32..31 and exactly one k = −32 (the unique max-abs element),
    c_s = m_s·u, m_s in 1..128 with 128 present, u a power of two. Then subscale_s = max/−32 = c_s, max_scale =
    128u, d = max_scale/−128 = −u, sc_s = round(c_s·(−128/max_scale)) = −m_s, scale = d·sc = c_s and q = k:
    sc bytes = −m_s, d = f16(−u), codes k + 32."""
    rng = np.random.default_rng(9)
    u = 2.0 ** -12
    m = rng.integers(1, 129, 16)
    m[3] = 128
    k = rng.integers(-31, 32, (16, 16))
    k[:, 5] = -32
    x = np.array([[m[s] * u * k[s, i] for i in range(16)] for s in range(16)], np.float32).ravel()
    raw = o.quantize(x, Q6_K).tolist()
    assert [(v if v < 128 else v - 256) for v in raw[192:208]] == (-m).tolist()
    assert raw[208:210] == f16le(-u)
    ql, qh = raw[0:128], raw[128:192]
    q6 = []
    for e in range(256):  # element e: half n128, quarter qq of 32, lane l (the layout of src/gguf.rs:449-477)
        n128, r = divmod(e, 128)
        qq, lane = divmod(r, 32)
        low = ql[64 * n128 + lane + 32 * (qq & 1)] >> (4 * (qq >> 1)) & 15
        high = (qh[32 * n128 + lane] >> (2 * qq)) & 3
        q6.append((low | (high << 4)) - 32)
    assert q6 == k.ravel().tolist()
    assert np.array_equal(o.dequant(np.array(raw, np.uint8), Q6_K, 256), x)


def test_q6_k_quantizer_all_zero_block():
    """amax = 0 everywhere: subscale 0, d = 0, every code 0 (stored 32 = 0b10_0000): ql all 0, qh all
    0b10101010, scales 0, d = +0."""
    raw = o.quantize(np.zeros(256, np.float32), Q6_K).tolist()
    assert raw[:128] == [0] * 128 and raw[128:192] == [0xAA] * 64 and raw[192:210] == [0] * 18


def test_qkx_scale_min_branches():  # src/gguf_write.rs:293-351
    # mx == mn (constant non-positive block): (0, −mn)
    assert o.qkx_scale_min(np.full(32, -0.25, np.float32), 15) == (0.0, 0.25)
    # mn > 0: the minimum is taken as 0; values s·l with l in 1..15 refit exactly to (s, 0)
    s = 2.0 ** -6
    l = np.random.default_rng(3).integers(1, 16, 32)
    l[0], l[1] = 1, 15
    sc, mn = o.qkx_scale_min((s * l).astype(np.float32), 15)
    assert sc == s and mn == 0.0
    # denom <= 0: a constant positive block puts every element on one level for every candidate scale, so the
    # fallback (span / nmax, −mn) = (c / 15, 0) is returned
    c = 15 * 2.0 ** -4
    assert o.qkx_scale_min(np.full(32, c, np.float32), 15) == (2.0 ** -4, 0.0)
    # (−b).max(0): two level clusters, the level-0 one {−ε, 0.4·step ×15} has a positive mean, so every
    # candidate's refit intercept b is positive and the clamp returns a minimum of exactly 0 (unclamped: −b < 0)
    step = 2.0 ** -5
    x = np.array([-2.0 ** -12] + [0.4 * step] * 15 + [15 * step] * 16, np.float32)
    sc, mn = o.qkx_scale_min(x, 15)
    assert mn == 0.0 and sc > 0
    # (s <= 0 is not forced: levels are a non-decreasing function of v, so with two or more distinct levels the
    # refit slope is positive in exact arithmetic; the branch is the reference's guard against f32 cancellation.)


# ---- qkx_scale_min's candidate search itself (src/gguf_write.rs:311-346) ----
# The grid blocks above are recovered exactly by many candidates, so they cannot tell a wrong candidate count,
# step or comparison apart. The blocks below can: each candidate's result is recomputed here independently — the
# level assignment in f32 exactly as the reference writes it (iscale = (nmax − 1 + 0.1·i)/span, round half away
# from zero, clamp), the refit as a float64 least-squares solve (numpy lstsq, not the reference's running sums),
# the error in float64 — and the test asserts that each block's winner is separated from the runner-up and that
# every plausible mistake (18 or 20 candidates, a 0.09 / 0.11 step, the start at nmax, `<=`) picks a different
# (scale, min), so the oracle's answer pins those constants.


def _qkx_candidates(x, nmax, start=-1, step=0.1, count=19):
    x32 = np.asarray(x, np.float32)
    x64 = x32.astype(np.float64)
    mn32 = np.float32(min(x32.min(), np.float32(0)))
    span32 = np.float32(x32.max() - mn32)
    out = []
    for i in range(count):
        isc = np.float32(np.float32(nmax + start) + np.float32(np.float32(step) * np.float32(i))) / span32
        t = (np.float32(isc) * (x32 - mn32)).astype(np.float64)
        lv = np.clip(np.floor(t + 0.5), 0, nmax)
        (s, b), *_ = np.linalg.lstsq(np.stack([lv, np.ones_like(lv)], 1), x64, rcond=None)
        if s > 0:
            m = max(-b, 0.0)
        else:
            s, m = float(span32) / nmax, -float(mn32)
        l2 = np.clip(np.floor((x64 + m) / s + 0.5), 0, nmax)
        out.append((float(((s * l2 - m - x64) ** 2).sum()), float(s), float(m)))
    return out


def _qkx_winner(fits, strict=True):
    e = [f[0] for f in fits]
    best = min(e)
    idx = [i for i, v in enumerate(e) if v == best]
    return idx[0] if strict else idx[-1]


_ALL_MISTAKES = ((-1, 0.1, 18), (-1, 0.1, 20), (-1, 0.09, 19), (-1, 0.11, 19), (0, 0.1, 19))


@pytest.mark.parametrize("seed,want_i,mistakes", [(75, 18, _ALL_MISTAKES), (561, 18, _ALL_MISTAKES),
                                                  (736, 18, _ALL_MISTAKES), (1105, 18, _ALL_MISTAKES),
                                                  (20, 6, _ALL_MISTAKES[2:])])
def test_qkx_scale_min_candidate_search_pinned(seed, want_i, mistakes):
    x = np.random.default_rng(seed).standard_normal(32).astype(np.float32)
    fits = _qkx_candidates(x, 15)
    i = _qkx_winner(fits)
    assert i == want_i
    errs = sorted(f[0] for f in fits)
    assert errs[1] - errs[0] > 1e-3 * errs[0]  # the winner is not a near-tie that f32 sums could flip
    s, m = fits[i][1:]
    # the mistakes this block detects (the test's own discrimination check)
    for alt in mistakes:
        af = _qkx_candidates(x, 15, *alt)
        assert abs(af[_qkx_winner(af)][1] - s) > 1e-3 * s, alt
    so, mo = o.qkx_scale_min(x, 15)
    assert abs(so - s) <= 1e-6 * s and abs(mo - m) <= 1e-6 * max(m, 1e-30), (so, s, mo, m)


def test_qkx_scale_min_keeps_the_first_of_equal_errors():
    """Two value clusters {0, a} with a = 14·15·2^-8: candidates 0-4 put a on level 14, candidates 5-18 on level 15,
    and both refits are exact (error exactly 0 in f32), so only the comparison decides. The strict `<` keeps the
    first candidate: scale a/14 = 15·2^-8 (with `<=` the last: a/15 = 14·2^-8), min 0."""
    a = 14 * 15 * 2.0 ** -8
    x = np.array([0.0] * 20 + [a] * 12, np.float32)
    fits = _qkx_candidates(x, 15)
    assert all(f[0] <= 1e-20 for f in fits)  # every candidate's refit is exact
    assert all(abs(f[1] - 15 * 2.0 ** -8) < 1e-12 for f in fits[:5])
    assert all(abs(f[1] - 14 * 2.0 ** -8) < 1e-12 for f in fits[5:])
    assert o.qkx_scale_min(x, 15) == (15 * 2.0 ** -8, 0.0)
    # the same sub-block inside a Q4_K super-block: scale code and level 14 in the bytes
    blk = np.zeros(256, np.float32)
    blk[:32] = x
    raw = o.quantize(blk, Q4_K).tolist()
    codes = [raw[16 + i] & 15 for i in range(32)]
    assert max(codes) == 14 and codes.count(14) == 12
