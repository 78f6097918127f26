"""The mixture-of-experts (OLMoE) training step against the oracle (oracle/peft.cpp moe_ffn: the forward of
src/forward.rs:542-572 and :487-493, backward by the chain rule — the reference's PEFT has no MoE
backward), same quantized bytes, LoRA factors and tokens.

Bar: loss and every LoRA gradient within 1e-3 relative L2 of the f32 path. At the full OLMoE size
(B4 x T512), where the oracle would take hours, the size-independent properties of the dense configs.
"""
import numpy as np
import pytest

from test_gpu_peft import TOL, compare_grads, oracle_model, rel_l2

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def gpu():
    from hos_amd import Gpu
    g = Gpu(0)
    yield g
    g.close()


def moe_cfg(**kw):
    from hos_amd.peft import ModelConfig
    base = dict(name="moe-tiny", n_layers=2, dim=256, n_heads=4, n_kv_heads=4, head_dim=64, ffn_dim=128,
                vocab=512, rms_eps=1e-5, rope_base=10000.0, rope_neox=True, lora_rank=8, lora_alpha=16.0,
                lora_targets=("q", "k", "v", "o"), quant=8, head_quant=8, n_experts=8, n_experts_used=2,
                qk_norm=True)
    base.update(kw)
    return ModelConfig(**base)


def run(gpu, cfg, B, T, seed):
    from hos_amd import synth
    from hos_amd.peft import PeftModel, TARGETS
    tensors = synth.build_tensors(gpu, cfg, seed=seed, norm_jitter=0.2)
    lora = synth.lora_init(cfg, seed=seed + 1, b_std=0.02)
    ids, tg = synth.tokens(cfg, B, T, seed=seed + 2)
    pm = PeftModel(gpu, cfg, max_batch=B, max_seq=T)
    pm.load(tensors)
    for (l, t), (A, Bm) in lora.items():
        pm.set_lora(l, t, A, Bm)
    om = oracle_model(cfg, tensors, lora)
    lg = pm.loss_grad(ids, tg)
    lo = om.loss_grad(ids, tg)
    assert abs(lg - lo) / abs(lo) <= TOL, (lg, lo)
    worst = compare_grads(pm, om, cfg, lora, TARGETS)
    lgt, lot = pm.logits(ids[0]), om.logits(ids[0])
    assert rel_l2(lgt, lot) <= TOL
    pm.close()
    return lg, lo, worst


@pytest.mark.parametrize("hd,E,K,quant", [(64, 8, 2, 8), (128, 8, 3, 8), (64, 4, 4, 12), (64, 16, 1, 14)])
def test_moe_step_parity(gpu, hd, E, K, quant):
    cfg = moe_cfg(head_dim=hd, n_heads=256 // hd, n_kv_heads=256 // hd, n_experts=E, n_experts_used=K, quant=quant,
                  ffn_dim=256 if quant != 8 else 128)
    print(f"moe parity hd={hd} E={E} K={K} quant={quant}", flush=True)
    lg, lo, worst = run(gpu, cfg, B=2, T=40, seed=E + K)
    print(f"moe loss gpu {lg:.6f} cpu {lo:.6f} worst grad rel L2 {worst:.2e}", flush=True)


def test_moe_without_qk_norm_ragged(gpu):
    cfg = moe_cfg(qk_norm=False, n_experts=6, n_experts_used=2, n_layers=3)
    print("moe parity no qk-norm B=3 T=33", flush=True)
    run(gpu, cfg, B=3, T=33, seed=41)


@pytest.mark.timeout(600)
def test_olmoe_two_layer_parity(gpu):
    """The OLMoE layer shapes (d 2048, 16 heads of 128, 64 experts top-8 of SwiGLU 1024, vocab 50304, Q8_0)
    with 2 layers, B1 x T24, against the oracle."""
    from hos_amd import synth
    import copy
    cfg = copy.copy(synth.CONFIGS["olmoe"])
    cfg.n_layers = 2
    print("moe parity olmoe 2 layers B=1 T=24", flush=True)
    lg, lo, worst = run(gpu, cfg, B=1, T=24, seed=51)
    print(f"olmoe loss gpu {lg:.6f} cpu {lo:.6f} worst grad rel L2 {worst:.2e}", flush=True)


def test_olmoe_full_size_step_properties():
    """configs[4] at its benchmark shape (16 layers, B4 x T512): deterministic, finite, loss ≈ ln(vocab) at
    B = 0, dA exactly zero at B = 0, AdamW steps lower the loss."""
    from test_gpu_peft import test_full_size_step_properties
    test_full_size_step_properties("olmoe")


def test_moe_graph_replay_matches_eager(gpu):
    from hos_amd import synth
    from hos_amd.peft import PeftModel
    cfg = moe_cfg()
    print("moe graph replay vs eager", flush=True)
    tensors = synth.build_tensors(gpu, cfg, seed=61)
    lora = synth.lora_init(cfg, seed=62, b_std=0.02)
    ids, tg = synth.tokens(cfg, 2, 48, seed=63)
    models = []
    for graph in (False, True):
        pm = PeftModel(gpu, cfg, max_batch=2, max_seq=48)
        pm.load(tensors)
        for (l, t), (A, Bm) in lora.items():
            pm.set_lora(l, t, A, Bm)
        pm.use_graph(graph)
        models.append(pm)
    I, TG, L = gpu.to_dev(ids), gpu.to_dev(tg), gpu.empty_dev((1,))
    for step in range(4):
        out = []
        for pm in models:
            pm.step_dev(I.ptr, TG.ptr, 2, 48, 1e-3, 0.0, L.ptr)
            gpu.synchronize()
            out.append((L.get()[0], [pm.get_lora(l, t) for (l, t) in lora]))
        (la, fa), (lb, fb) = out
        assert la == lb, f"step {step}"
        for (A1, B1), (A2, B2) in zip(fa, fb):
            assert np.array_equal(A1, A2) and np.array_equal(B1, B2), f"step {step}"
    for a in (I, TG, L):
        a.free()
    for pm in models:
        pm.close()


def _route(gpu, logits, K):
    M, E = logits.shape
    L = gpu.to_dev(logits)
    P, SE, SP = gpu.empty_dev((M, E)), gpu.empty_dev((M, K), np.int32), gpu.empty_dev((M, K))
    SL, CN = gpu.empty_dev((M, K), np.int32), gpu.empty_dev((E,), np.int32)
    gpu.op("moe_route", L, M, E, K, P, SE, SP, SL, CN)
    out = tuple(a.get() for a in (P, SE, SP, SL, CN))
    for a in (L, P, SE, SP, SL, CN):
        a.free()
    return out


def _check_grouping(sel_e, slot, counts, E):
    """slot = rank of each selection among its expert's selections in (token, slot) order; counts = totals."""
    flat, sl = sel_e.ravel(), slot.ravel()
    seen = np.zeros(E, np.int64)
    for q, e in enumerate(flat):
        assert sl[q] == seen[e], f"selection {q}: slot {sl[q]} != {seen[e]}"
        seen[e] += 1
    assert np.array_equal(counts, seen)


@pytest.mark.parametrize("E,K", [(64, 8), (8, 2), (5, 5)])
def test_moe_route_matches_stable_sort(gpu, E, K):
    """The router entry point (src/forward.rs:542-552): softmax within 1e-6 of float64, and the selection equal to
    a stable descending sort of the kernel's own probabilities (ties to the lower expert), raw probabilities
    carried. Rows with forced exact ties (duplicated logits) check the tie order."""
    rng = np.random.default_rng(E * 100 + K)
    M = 300
    logits = rng.standard_normal((M, E)).astype(np.float32)
    logits[::7, 1] = logits[::7, 0]          # exact ties between experts 0 and 1
    logits[::11, :] = 0.25                   # a whole row tied: experts 0..K-1 in order
    print(f"moe_route E={E} K={K} M={M}", flush=True)
    p, sel_e, sel_p, slot, counts = _route(gpu, logits, K)
    x = logits.astype(np.float64)
    want = np.exp(x - x.max(1, keepdims=True))
    want /= want.sum(1, keepdims=True)
    assert np.abs(p - want).max() <= 1e-6
    order = np.argsort(-p, axis=1, kind="stable")[:, :K]
    assert np.array_equal(sel_e, order)
    assert np.array_equal(sel_p, np.take_along_axis(p, sel_e, 1))
    _check_grouping(sel_e, slot, counts, E)


def test_moe_route_nan_logits_give_distinct_experts(gpu):
    """Regression test of the router with diverged (NaN) logits: every row still selects K distinct experts in
    [0, E) (a NaN probability ranks below every number), the grouping stays consistent, and the NaN is carried
    in the selected probabilities rather than turned into an index."""
    E, K, M = 64, 8, 64
    rng = np.random.default_rng(5)
    logits = rng.standard_normal((M, E)).astype(np.float32)
    logits[0, :] = np.nan                    # every logit NaN
    logits[1, 3] = np.nan                    # one NaN logit: the softmax sum, so the whole row, is NaN
    logits[2, 10:40] = np.nan
    print("moe_route NaN logits", flush=True)
    p, sel_e, sel_p, slot, counts = _route(gpu, logits, K)
    for t in range(M):
        assert len(set(sel_e[t].tolist())) == K, f"row {t}: {sel_e[t]}"
        assert ((sel_e[t] >= 0) & (sel_e[t] < E)).all()
    assert np.array_equal(sel_e[0], np.arange(K))  # all NaN: ties resolve to the lowest experts
    assert np.isnan(sel_p[0]).all() and np.isnan(sel_p[1]).all()
    assert np.isfinite(sel_p[3:]).all()
    _check_grouping(sel_e, slot, counts, E)


@pytest.mark.timeout(1500)
def test_olmoe_full_depth_parity():
    """configs[4] at full depth (16 layers, d 2048, 64 experts top-8 in Q8_0, QK-norm, LoRA r16 on q/k/v/o) on one
    512-token sequence — the benchmark's sequence length, so the grouped expert GEMMs run 128-row tiles of experts
    holding up to hundreds of rows — against the oracle: loss and every LoRA gradient within 1e-3."""
    import time
    from conftest import heartbeat
    from hos_amd import Gpu, synth
    from hos_amd.peft import PeftModel, TARGETS
    g = Gpu(0)
    cfg = synth.CONFIGS["olmoe"]
    B, T = 1, 512
    print(f"moe parity olmoe 16 layers B={B} T={T}", flush=True)
    tensors = synth.build_tensors(g, cfg, seed=71)
    lora = synth.lora_init(cfg, seed=72, b_std=0.02)
    ids, tg = synth.tokens(cfg, B, T, seed=73)
    pm = PeftModel(g, cfg, max_batch=B, max_seq=T)
    pm.load(tensors)
    for (l, t), (A, Bm) in lora.items():
        pm.set_lora(l, t, A, Bm)
    lg = pm.loss_grad(ids, tg)
    print(f"gpu loss {lg:.6f}; loading the oracle", flush=True)
    t0 = time.time()
    with heartbeat("oracle olmoe B1xT512"):
        om = oracle_model(cfg, tensors, lora)
        del tensors
        lo = om.loss_grad(ids, tg)
    print(f"oracle loss {lo:.6f} in {time.time() - t0:.1f} s (with loading)", flush=True)
    assert abs(lg - lo) / abs(lo) <= TOL, (lg, lo)
    worst = compare_grads(pm, om, cfg, lora, TARGETS)
    print(f"olmoe 16 layers B1xT512: loss gpu {lg:.6f} cpu {lo:.6f}, worst LoRA grad rel L2 {worst:.2e}", flush=True)
    pm.close()
    g.close()
