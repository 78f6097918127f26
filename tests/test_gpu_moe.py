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
