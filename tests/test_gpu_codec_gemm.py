"""GPU parity of the quant codec and GEMMs against the oracle (restated src/gguf.rs, src/gguf_write.rs,
src/tensor.rs matmul), through the C ABI.

Bars: dequantized weights and quantizer bytes bit-exact; fp16-MFMA qGEMMs within relative L2 1e-3 of the f32
matmul on the same dequantized weights; f32-MFMA keyed GEMMs within 1e-5 (tests/autograd.rs:332-354 uses
1e-3 + 1e-3·|c| elementwise for its GPU matmul; both are checked).
"""
import numpy as np
import pytest

from oracle import binding as o

pytestmark = pytest.mark.gpu

Q8_0, Q4_K, Q6_K = 8, 12, 14


@pytest.fixture(scope="module")
def gpu():
    from hos_amd import Gpu
    g = Gpu(0)
    yield g
    g.close()


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30)


def weights(rows, cols, seed, std=0.02):
    return (np.random.default_rng(seed).standard_normal((rows, cols)) * std).astype(np.float32)


@pytest.mark.parametrize("t", [Q8_0, Q4_K, Q6_K])
def test_quantize_bytes_identical(gpu, t):
    print(f"quantize type {t}", flush=True)
    x = weights(256, 1024, 10 + t)
    x[3, :32] = 0.0  # an all-zero block exercises the d == 0 paths
    x[5] *= 1e-6  # tiny and large magnitudes, one-signed rows
    x[6] *= 1e3
    x[7] = np.abs(x[7])
    x[8] = -np.abs(x[8])
    # sub-blocks whose qkx_scale_min result depends on the candidate count / step / comparison (pinned on the
    # oracle in tests/test_oracle_codec.py), and the equal-error block the strict `<` decides
    x[9, :32] = [0.0] * 20 + [14 * 15 * 2.0 ** -8] * 12
    for j, seed in enumerate((75, 561, 736, 1105, 20)):
        x[10, 32 * j:32 * j + 32] = np.random.default_rng(seed).standard_normal(32).astype(np.float32)
    assert np.array_equal(gpu.quantize(x, t), o.quantize(x, t))


@pytest.mark.parametrize("t", [Q8_0, Q4_K, Q6_K])
def test_dequant_bit_exact(gpu, t):
    print(f"dequant type {t}", flush=True)
    rows, cols = 96, 768
    raw = o.quantize(weights(rows, cols, 20 + t), t)
    gpu.upload_quant(100 + t, raw, t, rows, cols)
    got = gpu.dequant(100 + t, rows, cols)
    want = o.dequant(raw, t, rows * cols).reshape(rows, cols)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("passes", [1, 2, 3, 4, 5])
@pytest.mark.parametrize("t", [Q8_0, Q4_K, Q6_K])
@pytest.mark.parametrize("shape", [(256, 512, 512), (200, 576, 768), (128, 1152, 256),
                                   # large enough for the 128-row / 128-column tile variants
                                   (2560, 2048, 2048), (1280, 4096, 1024)])
def test_qgemm_fwd_and_dx(gpu, t, shape, passes):
    T, N, K = shape  # W [N, K]
    print(f"qgemm type {t} T={T} N={N} K={K} passes={passes}", flush=True)
    gpu.set_gemm_passes(passes)
    raw = o.quantize(weights(N, K, 30 + t), t)
    key = 1000 + t
    gpu.upload_quant(key, raw, t, N, K)
    w = o.dequant(raw, t, N * K).reshape(N, K)
    rng = np.random.default_rng(5)
    x = rng.standard_normal((T, K)).astype(np.float32)
    dy = (rng.standard_normal((T, N)) * 1e-6).astype(np.float32)  # tiny gradients: row scaling keeps fp16 exact
    y = gpu.qgemm_fwd(key, x, N)
    dx = gpu.qgemm_dx(key, dy, K)
    gpu.set_gemm_passes(1)
    ref_y, _, _ = o.op_matmul(x, w.T.copy())
    ref_dx, _, _ = o.op_matmul(dy, w)
    # 1 pass: both operands rounded to fp16; 2: activation exact to ~22 bits; 3: both; 4: weight only;
    # 5: activation to ~22 bits against the exact integer weight codes (forward, Q8_0), else as 3
    tol = {1: 1e-3, 2: 5e-4, 3: 2e-6, 4: 5e-4, 5: 2e-6}[passes]
    assert rel_l2(y, ref_y) < tol
    assert rel_l2(dx, ref_dx) < tol


def test_qgemm_rejects_bad_shapes(gpu):
    from hos_amd import HosError
    raw = o.quantize(weights(64, 256, 1), Q4_K)
    with pytest.raises(HosError):
        gpu.upload_quant(7, raw[:-1], Q4_K, 64, 256)  # truncated bytes -> Format
    with pytest.raises(HosError):
        gpu.upload_quant(7, raw, 3, 64, 256)  # unsupported type
    with pytest.raises(HosError):
        gpu.qgemm_fwd(424242, np.zeros((4, 256), np.float32), 64)  # unknown key


@pytest.mark.parametrize("m,k,n", [(17, 23, 11), (64, 64, 64), (130, 70, 257)])
def test_keyed_f32_gemms(gpu, m, k, n):
    print(f"f32 keyed m={m} k={k} n={n}", flush=True)
    rng = np.random.default_rng(m + k + n)
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((k, n)).astype(np.float32)
    g = rng.standard_normal((m, n)).astype(np.float32)
    out = gpu.matmul_f32_keyed(a, m, k, b, n, b_key=77)
    out2 = gpu.matmul_f32_keyed(a, m, k, b, n, b_key=77)  # cached operand reused
    ref, da, db = o.op_matmul(a, b, g)
    assert np.all(np.abs(out - ref) <= 1e-3 + 1e-3 * np.abs(ref))  # tests/autograd.rs:350-352
    assert rel_l2(out, ref) < 1e-5 and np.array_equal(out, out2)
    got_da = gpu.matmul_abt_keyed(g, m, n, b, k, b_key=77)
    got_db = gpu.matmul_atb_keyed(a, k, m, g, n, a_key=None)
    assert rel_l2(got_da, da) < 1e-5
    assert rel_l2(got_db, db) < 1e-5
    gpu.evict(77)
    gpu.clear_cache()


# ---- the other encodings the reference decodes (src/gguf.rs:330-505): F32, F16, BF16, Q4_0, Q5_0, Q5_K ----
F32, F16, Q4_0, Q5_0, Q5_K, BF16 = 0, 1, 2, 6, 13, 30
OTHER = [F32, F16, BF16, Q4_0, Q5_0, Q5_K]


def encoded(rows, cols, t, seed):
    """GGUF bytes of a ~N(0, 0.02) [rows, cols] matrix in type t (the oracle's quantizers for the block types;
    BF16 keeps the top half of each f32)."""
    w = weights(rows, cols, seed)
    if t == F32:
        return w.view(np.uint8).ravel()
    if t == BF16:
        return (w.view(np.uint32) >> 16).astype(np.uint16).view(np.uint8).ravel()
    return o.quantize(w, t)


def random_q5k(rows, cols, seed):
    """Q5_K super-blocks with random scales, mins, high bits and nibbles (sane f16 d and dmin): every
    code/scale/min combination the decode must handle, not only what the quantizer emits."""
    rng = np.random.default_rng(seed)
    nb = rows * cols // 256
    blk = rng.integers(0, 256, size=(nb, 176), dtype=np.uint8)
    d = (rng.uniform(1e-4, 4e-3, nb) * rng.choice([-1, 1], nb)).astype(np.float16)
    dmin = rng.uniform(0, 4e-3, nb).astype(np.float16)
    blk[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
    blk[:, 2:4] = dmin.view(np.uint8).reshape(nb, 2)
    return blk.ravel()


@pytest.mark.parametrize("t", OTHER + ["q5k_random"])
def test_dequant_other_encodings_bit_exact(gpu, t):
    print(f"dequant encoding {t}", flush=True)
    rows, cols = 64, 512
    raw = random_q5k(rows, cols, 7) if t == "q5k_random" else encoded(rows, cols, t, 40)
    t = Q5_K if t == "q5k_random" else t
    gpu.upload_quant(200 + t, raw, t, rows, cols)
    got = gpu.dequant(200 + t, rows, cols)
    want = o.dequant(raw, t, rows * cols).reshape(rows, cols)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    gpu.evict(200 + t)


@pytest.mark.parametrize("passes", [1, 3, 5])
@pytest.mark.parametrize("t", OTHER)
@pytest.mark.parametrize("shape", [(200, 576, 768), (2560, 2048, 2048)])
def test_qgemm_other_encodings(gpu, t, shape, passes):
    T, N, K = shape
    print(f"qgemm encoding {t} T={T} N={N} K={K} passes={passes}", flush=True)
    gpu.set_gemm_passes(passes)
    raw = encoded(N, K, t, 50 + t)
    gpu.upload_quant(300 + t, raw, t, N, K)
    w = o.dequant(raw, t, N * K).reshape(N, K)
    rng = np.random.default_rng(6)
    x = rng.standard_normal((T, K)).astype(np.float32)
    dy = (rng.standard_normal((T, N)) * 1e-3).astype(np.float32)
    y = gpu.qgemm_fwd(300 + t, x, N)
    dx = gpu.qgemm_dx(300 + t, dy, K)
    gpu.set_gemm_passes(1)
    gpu.evict(300 + t)
    ref_y, _, _ = o.op_matmul(x, w.T.copy())
    ref_dx, _, _ = o.op_matmul(dy, w)
    tol = {1: 1e-3, 3: 2e-6, 5: 2e-6}[passes]
    if t == F16 and passes == 1:
        tol = 5e-4  # the weight is exact in fp16: only the activation rounds
    assert rel_l2(y, ref_y) < tol
    assert rel_l2(dx, ref_dx) < tol


def planes(w):
    """The GEMM's weight planes of the f32 dequantized w: hi = fp16(w), lo = fp16(w - hi)."""
    hi = w.astype(np.float16)
    lo = (w - hi.astype(np.float32)).astype(np.float16)
    return hi.astype(np.float32), lo.astype(np.float32)


def random_kquant(rows, cols, t, seed):
    """Q4_K (144-byte) / Q6_K (210-byte) super-blocks of random bytes with sane f16 scale fields (Q4_K: d of either
    sign and dmin at bytes 0-3; Q6_K: d at bytes 208-209, its int8 sub-scales random of either sign): every code and
    sub-scale combination, not only what the quantizer emits."""
    rng = np.random.default_rng(seed)
    nb = rows * cols // 256
    size = 144 if t == Q4_K else 210
    blk = rng.integers(0, 256, size=(nb, size), dtype=np.uint8)
    d = (rng.uniform(1e-4, 4e-3, nb) * rng.choice([-1, 1], nb)).astype(np.float16)
    if t == Q4_K:
        dmin = rng.uniform(0, 4e-3, nb).astype(np.float16)
        blk[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
        blk[:, 2:4] = dmin.view(np.uint8).reshape(nb, 2)
    else:
        blk[:, 208:210] = d.view(np.uint8).reshape(nb, 2)
    return blk.ravel()


@pytest.mark.parametrize("passes", [1, 3, 4])
@pytest.mark.parametrize("t", [Q8_0, Q4_K, Q6_K] + OTHER + ["q5k_random", "q4k_random", "q6k_random"])
@pytest.mark.parametrize("shape", [(576, 768), (2048, 2048)])
def test_qgemm_weight_planes_bit_exact(gpu, t, shape, passes):
    """The weight as the qGEMM dequantizes it in registers (not the standalone dequant kernel): with one-hot
    activation rows every output element is one product 1·w_hi (+ 1·w_lo), exact in the fp32 accumulators, so
    the forward returns deq(W)ᵀ's hi plane (1 pass) or hi + lo (3 and 4 passes) bit for bit, and the dX returns
    deq(W)'s, both on the tiles the rule picks at these sizes."""
    N, K = shape
    print(f"qgemm weight planes type {t} N={N} K={K} passes={passes}", flush=True)
    if t == "q5k_random":
        raw, t = random_q5k(N, K, 9), Q5_K
    elif t in ("q4k_random", "q6k_random"):
        t = Q4_K if t == "q4k_random" else Q6_K
        raw = random_kquant(N, K, t, 11)
    else:
        raw = encoded(N, K, t, 60)
    key = 400 + t
    gpu.upload_quant(key, raw, t, N, K)
    w = o.dequant(raw, t, N * K).reshape(N, K)
    hi, lo = planes(w)
    # the f32 sum of the two planes is exact; + 0 turns a -0 weight into the +0 that 0 + (-0) accumulates to
    want = (hi if passes == 1 else hi + lo) + np.float32(0.0)
    gpu.set_gemm_passes(passes)
    try:
        y = gpu.qgemm_fwd(key, np.eye(K, dtype=np.float32), N)  # y[k, n] = w[n, k]
        dx = gpu.qgemm_dx(key, np.eye(N, dtype=np.float32), K)  # dx[n, k] = w[n, k]
    finally:
        gpu.set_gemm_passes(1)
        gpu.evict(key)
    assert np.array_equal(y.view(np.uint32), np.ascontiguousarray(want.T).view(np.uint32))
    assert np.array_equal(dx.view(np.uint32), want.view(np.uint32))
