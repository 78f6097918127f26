"""hos_hip_lora_noalloc (the LoRA branch with its scratch in a static per-GPU device array, no allocation)
against hos_hip_lora on the same inputs, through the C ABI: two calls in a row, the second smaller, so the
second runs on scratch the first left behind. Bar: the f32 bar of the LoRA op tests (rel L2 1e-5 against the
allocating entry point, which the oracle pins in test_gpu_ops.py); u, dA, dB also bit-identical (same kernels,
same splits)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def _branch(g, name, x, dy, A, B, s, y0, dx0):
    rows, inn = x.shape
    out, r = dy.shape[1], A.shape[1]
    X, DY, AA, BB = g.to_dev(x), g.to_dev(dy), g.to_dev(A), g.to_dev(B)
    Y, DX = g.to_dev(y0), g.to_dev(dx0)
    U, DA, DB = g.empty_dev((rows, r)), g.empty_dev((inn, r)), g.empty_dev((r, out))
    g.op(name, X, DY, rows, inn, out, r, AA, BB, s, Y, U, DA, DB, DX)
    res = [a.get() for a in (U, DA, DB, Y, DX)]
    for a in (X, DY, AA, BB, Y, DX, U, DA, DB):
        a.free()
    return res


def test_lora_noalloc_matches_lora():
    from hos_amd import Gpu
    g = Gpu(0)
    # the second call is smaller and splits differently, so it reads scratch regions the first one wrote
    for rows, inn, out, r in ((2048, 4096, 2048, 32), (200, 896, 128, 16)):
        print(f"lora_noalloc rows={rows} in={inn} out={out} r={r}", flush=True)
        rng = np.random.default_rng(rows + r)
        x = rng.standard_normal((rows, inn), dtype=np.float32)
        dy = rng.standard_normal((rows, out), dtype=np.float32)
        A = rng.standard_normal((inn, r), dtype=np.float32) * np.float32(0.02)
        B = rng.standard_normal((r, out), dtype=np.float32) * np.float32(0.02)
        y0 = rng.standard_normal((rows, out), dtype=np.float32)
        dx0 = rng.standard_normal((rows, inn), dtype=np.float32)
        want = _branch(g, "lora", x, dy, A, B, 2.0, y0, dx0)
        got = _branch(g, "lora_noalloc", x, dy, A, B, 2.0, y0, dx0)
        for a, b in zip(got[:3], want[:3]):
            assert np.array_equal(a, b)
        for a, b in zip(got[3:], want[3:]):
            assert rel_l2(a, b) < 1e-5
    g.close()


def test_lora_noalloc_rejects_oversize():
    from hos_amd import Gpu, HosError
    g = Gpu(0)
    big = g.empty_dev((4,))  # never touched: the size check fails before any launch
    with pytest.raises(HosError, match="maximum"):
        g.op("lora_noalloc", big, big, 1 << 20, 4096, 4096, 96, big, big, 1.0, None, big, big, big, None)
    big.free()
    g.close()
