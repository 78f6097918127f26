"""Op-level GPU parity: each fused kernel of the training path through its C-ABI entry point against the
oracle's restatement of the same reference op (src/tensor.rs), as tests/autograd.rs checks the reference's
ops one by one.

Bars: RoPE and AdamW bit-exact (same operation order, same f32 roundings, same host libm table);
RMSNorm / SwiGLU within f32 reassociation (1e-5 relative, elementwise with a small absolute floor);
cross-entropy against a float64 softmax (2e-6) and the oracle's sequential-f32 sum (its own error, doubled);
attention (bf16 hi/lo MFMA, ~2^-16 per product) within 1e-4 relative L2; LoRA factor
GEMMs (fp32 MFMA) within 1e-5 relative L2; embedding bit-exact (bit-exact dequantization).
"""
import numpy as np
import pytest

from oracle import binding as o

pytestmark = pytest.mark.gpu


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


def close(a, b, rtol=1e-5, atol=1e-7):
    return np.allclose(np.asarray(a, np.float64), np.asarray(b, np.float64), rtol=rtol, atol=atol)


@pytest.mark.parametrize("rows,d", [(37, 576), (8, 896), (3, 2048)])
def test_rmsnorm_fwd_bwd(gpu, rows, d):
    print(f"rmsnorm rows={rows} d={d}", flush=True)
    rng = np.random.default_rng(rows + d)
    x = rng.standard_normal((rows, d)).astype(np.float32)
    w = (1.0 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    g = rng.standard_normal((rows, d)).astype(np.float32)
    ref, gx_ref, _ = o.op_rmsnorm(x, w, 1e-6, gout=g)
    X, W, G = gpu.to_dev(x), gpu.to_dev(w), gpu.to_dev(g)
    Y, INV, GX = gpu.empty_dev((rows, d)), gpu.empty_dev((rows,)), gpu.empty_dev((rows, d))
    gpu.op("rmsnorm_fwd", X, W, rows, d, 1e-6, Y, INV)
    gpu.op("rmsnorm_bwd", G, X, INV, W, rows, d, GX)
    assert close(Y.get(), ref)
    assert close(GX.get(), gx_ref, atol=1e-6)
    for a in (X, W, G, Y, INV, GX):
        a.free()


@pytest.mark.parametrize("neox", [True, False])
def test_rope_bit_exact(gpu, neox):
    B, T, nh, hd, base = 3, 50, 4, 64, 1e6 if neox else 1e4
    print(f"rope neox={neox}", flush=True)
    rng = np.random.default_rng(3)
    x = rng.standard_normal((B * T, nh * hd)).astype(np.float32)
    g = rng.standard_normal((B * T, nh * hd)).astype(np.float32)
    pos = np.tile(np.arange(T), B)
    ref, dx_ref = o.op_rope(x, nh, hd, base, neox, pos, gout=g)
    X, G = gpu.to_dev(x), gpu.to_dev(g)
    gpu.op("rope", X, B * T, nh * hd, 0, nh, hd, T, base, int(neox), 0)
    gpu.op("rope", G, B * T, nh * hd, 0, nh, hd, T, base, int(neox), 1)
    assert np.array_equal(X.get(), ref)
    assert np.array_equal(G.get(), dx_ref)
    X.free()
    G.free()


def test_swiglu_fwd_bwd(gpu):
    rows, F = 29, 1536
    print("swiglu", flush=True)
    rng = np.random.default_rng(4)
    gate = (2 * rng.standard_normal((rows, F))).astype(np.float32)
    up = rng.standard_normal((rows, F)).astype(np.float32)
    dh = rng.standard_normal((rows, F)).astype(np.float32)
    h_ref, dg_ref, du_ref = o.op_swiglu(gate, up, gout=dh)
    GU, DH = gpu.to_dev(np.concatenate([gate, up], 1)), gpu.to_dev(dh)
    H, DGU = gpu.empty_dev((rows, F)), gpu.empty_dev((rows, 2 * F))
    gpu.op("swiglu_fwd", GU, rows, F, H)
    gpu.op("swiglu_bwd", GU, DH, rows, F, DGU)
    dgu = DGU.get()
    assert close(H.get(), h_ref, atol=1e-6)
    assert close(dgu[:, :F], dg_ref, atol=1e-6) and close(dgu[:, F:], du_ref, atol=1e-6)
    for a in (GU, DH, H, DGU):
        a.free()


@pytest.mark.parametrize("B,T,nh,nkv,hd", [(1, 128, 9, 3, 64), (2, 77, 14, 2, 64), (1, 64, 4, 4, 64),
                                           # OLMoE's head dim (16 heads of 128, no GQA) and a GQA case
                                           (2, 70, 4, 4, 128), (1, 97, 6, 2, 128),
                                           # one token; several 128-row workgroups with a ragged last one
                                           (1, 1, 4, 4, 64), (2, 300, 8, 2, 64), (1, 512, 14, 2, 64),
                                           # long ragged sequence: both wave groups of every workgroup busy
                                           (1, 1000, 4, 2, 64)])
def test_attention_fwd_bwd(gpu, B, T, nh, nkv, hd):
    print(f"attention B={B} T={T} heads={nh}/{nkv} hd={hd}", flush=True)
    rng = np.random.default_rng(B * T + nh)
    q = rng.standard_normal((B, T, nh * hd)).astype(np.float32)
    k = rng.standard_normal((B, T, nkv * hd)).astype(np.float32)
    v = rng.standard_normal((B, T, nkv * hd)).astype(np.float32)
    go = rng.standard_normal((B, T, nh * hd)).astype(np.float32)
    W3 = (nh + 2 * nkv) * hd
    qkv = np.concatenate([q, k, v], 2).reshape(B * T, W3)
    QKV, GO = gpu.to_dev(qkv), gpu.to_dev(go.reshape(B * T, nh * hd))
    O, LSE, D = gpu.empty_dev((B * T, nh * hd)), gpu.empty_dev((B, nh, T)), gpu.empty_dev((B * T, W3), fill=0.0)
    gpu.op("attention_fwd", QKV, W3, nh * hd, (nh + nkv) * hd, B, T, nh, nkv, hd, O, nh * hd, LSE)
    gpu.op("attention_bwd", QKV, W3, nh * hd, (nh + nkv) * hd, O, GO, nh * hd, LSE, B, T, nh, nkv, hd, D, W3)
    out, dqkv = O.get().reshape(B, T, -1), D.get().reshape(B, T, W3)
    for b in range(B):  # the reference runs one sequence at a time
        ref, dq, dk, dv = o.op_attention(q[b], k[b], v[b], nh, nkv, hd, gout=go[b])
        # dq and dk vanish at T = 1 (a single key has P = 1 and dS = dP − D = 0): measure them against dv's size
        floor = float(np.linalg.norm(dv))
        err = lambda a, r: float(np.linalg.norm(np.asarray(a, np.float64) - r)) / max(float(np.linalg.norm(r)), floor)
        assert rel_l2(out[b], ref) < 1e-4
        assert err(dqkv[b, :, :nh * hd], dq) < 1e-4
        assert err(dqkv[b, :, nh * hd:(nh + nkv) * hd], dk) < 1e-4
        assert rel_l2(dqkv[b, :, (nh + nkv) * hd:], dv) < 1e-4
    for a in (QKV, GO, O, LSE, D):
        a.free()


@pytest.mark.parametrize("rows,V", [(17, 512), (4, 49152), (3, 151936)])
def test_cross_entropy(gpu, rows, V):
    print(f"cross_entropy rows={rows} V={V}", flush=True)
    rng = np.random.default_rng(V)
    logits = (3 * rng.standard_normal((rows, V))).astype(np.float32)
    tg = rng.integers(0, V, rows).astype(np.int32)
    loss_ref, dl_ref = o.op_cross_entropy(logits, tg, gscale=1.0)
    L, TG = gpu.to_dev(logits), gpu.to_dev(tg)
    RL, DL = gpu.empty_dev((rows,)), gpu.empty_dev((rows, V))
    gpu.op("cross_entropy", L, rows, V, TG, 1.0 / rows, RL, DL)
    # float64 softmax as the exact value: the GPU reduces the exp-sum as a tree, the oracle (like the
    # reference) sequentially in f32, whose normaliser carries up to ~V·2^-24 relative rounding
    z = logits.astype(np.float64)
    p64 = np.exp(z - z.max(1, keepdims=True))
    p64 /= p64.sum(1, keepdims=True)
    d64 = p64.copy()
    d64[np.arange(rows), tg] -= 1.0
    d64 /= rows
    loss64 = float(np.mean(-np.log(p64[np.arange(rows), tg])))
    dl = DL.get()
    assert abs(float(np.mean(RL.get(), dtype=np.float64)) - loss64) <= 1e-6 * abs(loss64)
    assert abs(loss_ref - loss64) <= 1e-4 * abs(loss64)  # the oracle's own sequential-f32 rounding
    assert rel_l2(dl, d64) < 2e-6
    assert rel_l2(dl, dl_ref) < max(2e-6, 2 * rel_l2(dl_ref, d64))
    assert abs(dl.sum(1)).max() < 1e-6  # each gradient row sums to zero
    for a in (L, TG, RL, DL):
        a.free()


def test_adamw_bit_exact(gpu):
    n = 10007
    print("adamw", flush=True)
    rng = np.random.default_rng(8)
    p = rng.standard_normal(n).astype(np.float32)
    m = np.zeros(n, np.float32)
    v = np.zeros(n, np.float32)
    P, M, Vd = gpu.to_dev(p), gpu.to_dev(m), gpu.to_dev(v)
    for t in range(1, 4):
        g = rng.standard_normal(n).astype(np.float32)
        G = gpu.to_dev(g)
        gpu.op("adamw", P, G, M, Vd, n, 1e-3, 0.9, 0.95, 1e-8, 0.1, t, 1)
        p, m, v = o.adamw(p, g, m, v, t, 1e-3, 0.1, True)
        G.free()
        assert np.array_equal(P.get(), p) and np.array_equal(M.get(), m) and np.array_equal(Vd.get(), v)
    for a in (P, M, Vd):
        a.free()


@pytest.mark.parametrize("t", [8, 12])
def test_embedding_bit_exact(gpu, t):
    print(f"embedding type {t}", flush=True)
    V, d = 300, 512
    raw = o.quantize((np.random.default_rng(t).standard_normal((V, d)) * 0.02).astype(np.float32), t)
    gpu.upload_quant(500 + t, raw, t, V, d)
    ids = np.random.default_rng(1).integers(0, V, 41).astype(np.int32)
    I, OUT = gpu.to_dev(ids), gpu.empty_dev((41, d))
    gpu.op("embedding", 500 + t, I, 41, OUT)
    table = o.dequant(raw, t, V * d).reshape(V, d)
    assert np.array_equal(OUT.get().view(np.uint32), table[ids].view(np.uint32))
    I.free()
    OUT.free()
    gpu.evict(500 + t)


@pytest.mark.parametrize("rows,inn,out,r", [(96, 256, 384, 8), (200, 896, 128, 16), (64, 576, 1536, 32)])
def test_lora_branch(gpu, rows, inn, out, r):
    print(f"lora rows={rows} in={inn} out={out} r={r}", flush=True)
    rng = np.random.default_rng(rows + r)
    x = rng.standard_normal((rows, inn)).astype(np.float32)
    dy = rng.standard_normal((rows, out)).astype(np.float32)
    A = (0.02 * rng.standard_normal((inn, r))).astype(np.float32)
    Bm = (0.02 * rng.standard_normal((r, out))).astype(np.float32)
    s = 2.0
    y0 = rng.standard_normal((rows, out)).astype(np.float32)
    dx0 = rng.standard_normal((rows, inn)).astype(np.float32)
    # oracle matmuls (src/tensor.rs:307-391) for each factor product
    u, _, _ = o.op_matmul(x, A)
    ub, du_ref, dB_ref = o.op_matmul(u, Bm, s * dy)
    _, _, dA_ref = o.op_matmul(x, A, du_ref)
    dxl, _, _ = o.op_matmul(du_ref, A.T.copy())
    X, DY, AA, BB = gpu.to_dev(x), gpu.to_dev(dy), gpu.to_dev(A), gpu.to_dev(Bm)
    Y, DX = gpu.to_dev(y0), gpu.to_dev(dx0)
    U, DA, DB = gpu.empty_dev((rows, r)), gpu.empty_dev((inn, r)), gpu.empty_dev((r, out))
    gpu.op("lora", X, DY, rows, inn, out, r, AA, BB, s, Y, U, DA, DB, DX)
    assert rel_l2(U.get(), u) < 1e-5
    assert rel_l2(Y.get() - y0, s * ub) < 1e-5
    assert rel_l2(DB.get(), dB_ref) < 1e-5
    assert rel_l2(DA.get(), dA_ref) < 1e-5
    assert rel_l2(DX.get() - dx0, dxl) < 1e-5
    for a in (X, DY, AA, BB, Y, DX, U, DA, DB):
        a.free()


def test_op_errors(gpu):
    from hos_amd import HosError
    X = gpu.empty_dev((4, 64))
    with pytest.raises(HosError):
        gpu.op("rope", X, 4, 64, 0, 1, 63, 4, 1e4, 1, 0)  # odd head_dim
    with pytest.raises(HosError):
        gpu.op("embedding", 987654, X, 4, X)  # no table under that key
    X.free()
