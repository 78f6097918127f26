"""The isolated configs[1] workload at its full size, through the C ABI: W [4096, 4096] ~N(0, 0.02) quantized
to Q4_K, dY [4096, 4096] ~N(0, 1e-2); dX = dY·deq(W), the forward X·deq(W)ᵀ and a LoRA rank-16 A/B gradient
on the same shapes (reference: src/tensor.rs:307-391 matmul and its VJPs, src/gguf.rs:385-413 Q4_K decode,
src/peft.rs:508-512 LoRA branch).

At 4096³ the tile rule sends single-pass and weight-split (mode 4) GEMMs to the 256×128 eight-wave kernel and
the 2/3-pass GEMMs to 128×128, so every instantiation the bench times is checked here.

Checks (the oracle's f32 matmul on the bit-exact dequantized weight is the reference):
- a row sample of the output — 16 rows out of every 256-row tile, all 4096 columns, so every workgroup tile
  and XCD placement contributes — against the oracle at the precision-pass tolerance of the smaller GEMM tests;
- the whole output through a size-independent identity: column sums 1ᵀ·dX = (1ᵀ·dY)·deq(W) in float64.
"""
import numpy as np
import pytest

from oracle import binding as o

pytestmark = pytest.mark.gpu

N = 4096
Q4_K = 12
TOL = {1: 1e-3, 2: 5e-4, 3: 2e-6, 4: 5e-4}  # fp16 rounding of: both operands / weight / neither / activation


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


@pytest.fixture(scope="module")
def setup():
    from hos_amd import Gpu
    g = Gpu(0)
    rng = np.random.default_rng(2)
    w = rng.standard_normal((N, N), dtype=np.float32) * np.float32(0.02)
    raw = o.quantize(w, Q4_K)
    g.upload_quant(0xC1, raw, Q4_K, N, N)
    wd = o.dequant(raw, Q4_K, N * N).reshape(N, N)
    rows = np.concatenate([np.arange(t, t + 256, 16) + (t // 256) % 16 for t in range(0, N, 256)])
    yield g, wd, rng, rows
    g.set_gemm_passes(1)
    g.evict(0xC1)
    g.close()


def test_dequant_matches_oracle_at_full_size(setup):
    g, wd, _, _ = setup
    print("config1 dequant 4096x4096 Q4_K", flush=True)
    got = g.dequant(0xC1, N, N)
    assert np.array_equal(got.view(np.uint32), wd.view(np.uint32))


@pytest.mark.parametrize("passes", [1, 2, 3, 4])
def test_dx_4096cubed(setup, passes):
    g, wd, rng, rows = setup
    print(f"config1 dX 4096^3 Q4_K passes={passes}", flush=True)
    dy = rng.standard_normal((N, N), dtype=np.float32) * np.float32(1e-2)
    g.set_gemm_passes(passes)
    dx = g.qgemm_dx(0xC1, dy, N)
    ref, _, _ = o.op_matmul(dy[rows], wd)
    assert rel_l2(dx[rows], ref) < TOL[passes]
    colsum = dy.astype(np.float64).sum(0) @ wd.astype(np.float64)
    assert rel_l2(dx.astype(np.float64).sum(0), colsum) < max(TOL[passes], 1e-5)  # f32 vs float64 sums
    assert np.isfinite(dx).all()


@pytest.mark.parametrize("passes", [1, 3])
def test_fwd_4096cubed(setup, passes):
    g, wd, rng, rows = setup
    print(f"config1 fwd 4096^3 Q4_K passes={passes}", flush=True)
    x = rng.standard_normal((N, N), dtype=np.float32)
    g.set_gemm_passes(passes)
    y = g.qgemm_fwd(0xC1, x, N)
    ref, _, _ = o.op_matmul(x[rows], wd.T.copy())
    assert rel_l2(y[rows], ref) < TOL[passes]
    colsum = x.astype(np.float64).sum(0) @ wd.T.astype(np.float64)
    assert rel_l2(y.astype(np.float64).sum(0), colsum) < max(TOL[passes], 1e-5)


def test_lora_r16_gradient_4096(setup):
    """LoRA branch on the configs[1] shapes: x [4096, 4096], dY [4096, 4096], r 16, A/B ~N(0, 0.02), s = 2;
    u = x·A, dB = s·uᵀ·dY, du = s·dY·Bᵀ, dA = xᵀ·du (and y += s·u·B, dx += du·Aᵀ), each against the oracle's
    matmul and its VJPs (src/tensor.rs:307-391) at the f32 bar of the smaller LoRA tests."""
    g, _, rng, _ = setup
    print("config1 LoRA r16 4096x4096", flush=True)
    r, s = 16, 2.0
    x = rng.standard_normal((N, N), dtype=np.float32)
    dy = rng.standard_normal((N, N), dtype=np.float32) * np.float32(1e-2)
    A = rng.standard_normal((N, r), dtype=np.float32) * np.float32(0.02)
    B = rng.standard_normal((r, N), dtype=np.float32) * np.float32(0.02)
    u, _, _ = o.op_matmul(x, A)
    ub, du_ref, dB_ref = o.op_matmul(u, B, s * dy)
    _, _, dA_ref = o.op_matmul(x, A, du_ref)
    X, DY, AA, BB = g.to_dev(x), g.to_dev(dy), g.to_dev(A), g.to_dev(B)
    Y, DX = g.empty_dev((N, N), fill=0.0), g.empty_dev((N, N), fill=0.0)
    U, DA, DB = g.empty_dev((N, r)), g.empty_dev((N, r)), g.empty_dev((r, N))
    g.op("lora", X, DY, N, N, N, r, AA, BB, s, Y, U, DA, DB, DX)
    assert rel_l2(U.get(), u) < 1e-5
    assert rel_l2(DB.get(), dB_ref) < 1e-5
    assert rel_l2(DA.get(), dA_ref) < 1e-5
    assert rel_l2(Y.get(), s * ub) < 1e-5
    rows = np.arange(0, N, 61)
    dxl, _, _ = o.op_matmul(du_ref[rows], A.T.copy())
    assert rel_l2(DX.get()[rows], dxl) < 1e-5
    for a in (X, DY, AA, BB, Y, DX, U, DA, DB):
        a.free()


def test_exact_mode_large_q8_0_forward():
    """Precision mode 5 at a size where the launcher picks the integer-code kernel (forward, Q8_0, >= 64 GFLOP
    per launch: here 4096³): activation hi + lo against the exact codes, the 32-block scales applied in f32 —
    the mode-3 bar against the oracle's f32 matmul on the bit-exact dequantized weight (src/gguf.rs:354-367,
    src/tensor.rs:307-327), on the same row sample and column-sum identity as the Q4_K checks above."""
    from hos_amd import Gpu
    print("exact-mode forward 4096^3 Q8_0 passes=5", flush=True)
    g = Gpu(0)
    rng = np.random.default_rng(8)
    w = rng.standard_normal((N, N), dtype=np.float32) * np.float32(0.02)
    raw = o.quantize(w, 8)
    g.upload_quant(0xC5, raw, 8, N, N)
    wd = o.dequant(raw, 8, N * N).reshape(N, N)
    x = rng.standard_normal((N, N), dtype=np.float32)
    rows = np.concatenate([np.arange(t, t + 256, 16) + (t // 256) % 16 for t in range(0, N, 256)])
    g.set_gemm_passes(5)
    y = g.qgemm_fwd(0xC5, x, N)
    g.set_gemm_passes(1)
    g.evict(0xC5)
    g.close()
    ref, _, _ = o.op_matmul(x[rows], wd.T.copy())
    assert rel_l2(y[rows], ref) < TOL[3]
    colsum = x.astype(np.float64).sum(0) @ wd.T.astype(np.float64)
    assert rel_l2(y.astype(np.float64).sum(0), colsum) < 1e-5
