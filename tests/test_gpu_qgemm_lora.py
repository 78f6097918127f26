"""The frozen-base GEMM with its LoRA term fused into the epilogue (hos_hip_qgemm_lora_dev): the adapted linear
of src/peft.rs:508-512, y = x·deq(W)ᵀ + s·(x·A)·B, and its input gradient dx = dY·deq(W) + du·Aᵀ, with the
rank-r factor u / du given.

Reference: the oracle's f32 matmul (src/tensor.rs:307-391) on the bit-exact dequantized weight for the base
term, float64 numpy for the rank-r term. The rank-r term runs on bf16 hi/lo MFMA (~2^-16 relative to the
term); the test makes it as large as the base term, so a dropped or misplaced rank, row or column fails the
1e-5 bar by orders of magnitude.

Cases: ragged row counts (not a multiple of any tile), an output width that is not a multiple of the tile
(forward), ranks 16 / 20 (zero-padded to 32) / 48 / 64 / 96 (the stacked q|k|v dX, on 64×64 and, with 256 output
tiles, 128×128×64 tiles; ranks above a tile's LDS staging in chunks), L read through both stride
orders (B [r, N] rows, A [N, r] transposed), a narrow output with a long contraction (split over the contraction:
the first split's workgroups carry the term in their partial), rows whose magnitudes span 1e-20 .. 1e6 (the activation row
scale the term is divided by before it joins the accumulator), and 1 and 3 precision passes.
"""
import numpy as np
import pytest

from oracle import binding as o

pytestmark = pytest.mark.gpu

Q4_K, Q8_0 = 12, 8


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


@pytest.fixture(scope="module")
def gpu():
    from hos_amd import Gpu
    g = Gpu(0)
    yield g
    g.set_gemm_passes(1)
    g.close()


def run(g, which, key, inp, u, l_arr, slj, sln, rank, scale, nout):
    X, U, L = g.to_dev(inp), g.to_dev(u), g.to_dev(l_arr)
    OUT = g.empty_dev((inp.shape[0], nout), fill=0.0)
    g.op("qgemm_lora_dev", which, key, X, inp.shape[0], U, u.shape[1], L, slj, sln, rank, float(scale), OUT)
    out = OUT.get()
    for a in (X, U, L, OUT):
        a.free()
    return out


def weight(g, key, rows, cols, qtype, seed):
    rng = np.random.default_rng(seed)
    w = rng.standard_normal((rows, cols), dtype=np.float32) * np.float32(0.05)
    raw = o.quantize(w, qtype)
    g.upload_quant(key, raw, qtype, rows, cols)
    return o.dequant(raw, qtype, rows * cols).reshape(rows, cols)


# (which, t, rows, cols, rank, passes): forward outputs rows columns, dX outputs cols
CASES = [
    (0, 300, 320, 512, 16, 3),
    (0, 300, 320, 512, 20, 1),
    (0, 1000, 1024, 768, 32, 3),
    (1, 300, 512, 768, 16, 3),
    (1, 200, 512, 768, 48, 3),
    (1, 130, 256, 1024, 64, 1),
    (1, 2048, 2048, 2048, 48, 3),  # rank above 32 on 128x128x64 tiles (256 of them)
    (1, 2048, 2048, 2048, 64, 1),  # rank 64 in two staged chunks of 32 (one-plane 128x128x64 staging)
    (1, 300, 768, 512, 96, 3),  # rank 96 (Llama-3.2-1B's stacked q|k|v dX): chunks of 64 + 32 on 64x64 tiles
    (1, 2048, 3072, 2048, 96, 3),  # ... and on 128x128x64 tiles
    (1, 100, 544, 512, 48, 3),  # contraction not a multiple of 64: 32-deep slabs, chunks of 32 + 16
    (1, 64, 4096, 256, 16, 3),  # narrow output, long contraction: split-K
    (1, 64, 4096, 256, 32, 1),
]


@pytest.mark.parametrize("which,t,rows,cols,rank,passes", CASES)
def test_qgemm_lora_matches_oracle(gpu, which, t, rows, cols, rank, passes):
    g = gpu
    print(f"qgemm_lora which={which} t={t} W=[{rows},{cols}] r={rank} passes={passes}", flush=True)
    key = 0x1A00 + CASES.index((which, t, rows, cols, rank, passes))
    wd = weight(g, key, rows, cols, Q4_K if cols % 256 == 0 else Q8_0, seed=rank + 7 * which)
    rng = np.random.default_rng(1000 + rank + which)
    kin, nout = (cols, rows) if which == 0 else (rows, cols)
    x = rng.standard_normal((t, kin), dtype=np.float32)
    mags = np.ones(t, np.float32)
    mags[1::17] = 1e-20
    mags[2::13] = 1e6
    x *= mags[:, None]
    # rank-r factor with a leading dimension wider than the rank; its magnitude follows the row's (as x·A does)
    u = (rng.standard_normal((t, rank + 5), dtype=np.float32) * mags[:, None]).astype(np.float32)
    scale = 1.75
    if which == 0:  # L = B [rank, nout]: L(j, n) = B[j·nout + n]
        lmat = rng.standard_normal((rank, nout), dtype=np.float32) * np.float32(0.3)
        l_arr, slj, sln = lmat, nout, 1
    else:  # L = Aᵀ with A [nout, rank]: L(j, n) = A[n·rank + j]
        a = rng.standard_normal((nout, rank), dtype=np.float32) * np.float32(0.3)
        l_arr, slj, sln, lmat = a, 1, rank, a.T
    g.set_gemm_passes(passes)
    out = run(g, which, key, x, u, l_arr, slj, sln, rank, scale, nout)
    base, _, _ = o.op_matmul(x, wd.T.copy() if which == 0 else wd)
    term = scale * (u[:, :rank].astype(np.float64) @ lmat.astype(np.float64))
    ref = base.astype(np.float64) + term
    assert np.isfinite(out).all()
    tol = 1e-5 if passes == 3 else 3e-3
    # per row, so the 1e-20 rows are held to the same relative bar as the 1e6 rows
    errs = np.linalg.norm(out - ref, axis=1) / np.maximum(np.linalg.norm(ref, axis=1), 1e-300)
    assert errs.max() < tol, (errs.max(), int(errs.argmax()))
    g.evict(key)


def test_qgemm_lora_term_alone(gpu):
    """With the base weight zero the output is the rank-r term alone: bf16 hi/lo three-product bar (~2^-16)."""
    g = gpu
    rows, cols, t, rank = 256, 512, 200, 24
    g.upload_quant(0x1B00, o.quantize(np.zeros((rows, cols), np.float32), Q8_0), Q8_0, rows, cols)
    rng = np.random.default_rng(5)
    x = rng.standard_normal((t, cols), dtype=np.float32)
    u = rng.standard_normal((t, rank), dtype=np.float32)
    b = rng.standard_normal((rank, rows), dtype=np.float32)
    g.set_gemm_passes(3)
    out = run(g, 0, 0x1B00, x, u, b, rows, 1, rank, 0.5, rows)
    ref = 0.5 * (u.astype(np.float64) @ b.astype(np.float64))
    assert rel_l2(out, ref) < 3e-5
    g.evict(0x1B00)


def test_qgemm_lora_rejects_bad_rank(gpu):
    g = gpu
    g.upload_quant(0x1C00, o.quantize(np.zeros((64, 256), np.float32), Q8_0), Q8_0, 64, 256)
    X, U, L = g.to_dev(np.zeros((4, 256), np.float32)), g.to_dev(np.zeros((4, 140), np.float32)), \
        g.to_dev(np.zeros((140, 64), np.float32))
    OUT = g.empty_dev((4, 64), fill=0.0)
    for rank in (0, 129):
        with pytest.raises(Exception):
            g.op("qgemm_lora_dev", 0, 0x1C00, X, 4, U, 140, L, 64, 1, rank, 1.0, OUT)
    for a in (X, U, L, OUT):
        a.free()
    g.evict(0x1C00)
