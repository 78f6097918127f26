"""Whole-step parity of the device LoRA training step against the oracle's restatement of HOS's CPU path
(src/peft.rs forward + src/tensor.rs VJPs + src/main.rs:2583-2601 accumulation + AdamW), same quantized
bytes, same LoRA factors, same tokens.

Bar: loss and every LoRA gradient within relative L2 1e-3 of the CPU f32 path.
"""
import types

import numpy as np
import pytest

from oracle import binding as o

pytestmark = pytest.mark.gpu

TOL = 1e-3


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    nb = np.linalg.norm(b)
    return np.linalg.norm(a - b) / nb if nb > 0 else np.linalg.norm(a)


@pytest.fixture(scope="module")
def gpu():
    from hos_amd import Gpu
    g = Gpu(0)
    yield g
    g.close()


def oracle_model(cfg, tensors, lora):
    oc = types.SimpleNamespace(**{k: getattr(cfg, k) for k in (
        "n_layers", "dim", "n_heads", "n_kv_heads", "head_dim", "ffn_dim", "vocab", "rms_eps", "rope_base",
        "rope_neox", "attn_bias", "lora_rank", "lora_alpha", "n_experts", "n_experts_used", "qk_norm")})
    oc.lora_targets = cfg.target_mask
    m = o.OracleModel(oc)
    for name, (raw, t, rows, cols) in tensors.items():
        m.set_tensor(name, raw, t, rows, cols)
    for (l, t), (A, B) in lora.items():
        m.set_lora(l, ("q", "k", "v", "o", "gate", "up", "down").index(t), A, B)
    return m


def run_pair(gpu, cfg, B, T, b_std=0.02, seed=0):
    from hos_amd import synth
    from hos_amd.peft import PeftModel, TARGETS
    tensors = synth.build_tensors(gpu, cfg, seed=seed)
    lora = synth.lora_init(cfg, seed=seed + 1, b_std=b_std)
    ids, tg = synth.tokens(cfg, B, T, seed=seed + 2)
    pm = PeftModel(gpu, cfg, max_batch=B, max_seq=T)
    pm.load(tensors)
    for (l, t), (A, Bm) in lora.items():
        pm.set_lora(l, t, A, Bm)
    om = oracle_model(cfg, tensors, lora)
    return pm, om, ids, tg, lora, TARGETS


def compare_grads(pm, om, cfg, lora, TARGETS, tol=TOL):
    worst = 0.0
    for (l, t) in lora:
        i, ou = cfg.target_dims(t)
        gA, gB = pm.get_lora_grad(l, t)
        oA, oB = om.get_lora_grad(l, TARGETS.index(t), ((i, cfg.lora_rank), (cfg.lora_rank, ou)))
        for g, w, nm in ((gA, oA, "dA"), (gB, oB, "dB")):
            e = rel_l2(g, w)
            worst = max(worst, e)
            assert e <= tol, f"layer {l} {t} {nm}: rel L2 {e:.3e}"
    return worst


def tiny(quant, **kw):
    from hos_amd.peft import ModelConfig
    base = dict(name="tiny", n_layers=2, dim=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn_dim=512, vocab=512,
                rms_eps=1e-6, rope_base=1e6, rope_neox=True, attn_bias=True, lora_rank=8, lora_alpha=16.0,
                lora_targets=("q", "k", "v", "o", "gate", "up", "down"), quant=quant, head_quant=quant)
    base.update(kw)
    return ModelConfig(**base)


@pytest.mark.parametrize("quant", [8, 12, 14])
def test_step_grads_all_targets(gpu, quant):
    cfg = tiny(quant)
    print(f"peft tiny quant={quant} B=2 T=96", flush=True)
    pm, om, ids, tg, lora, TARGETS = run_pair(gpu, cfg, B=2, T=96)
    lg = pm.loss_grad(ids, tg)
    lo = om.loss_grad(ids, tg)
    assert abs(lg - lo) / abs(lo) <= TOL
    compare_grads(pm, om, cfg, lora, TARGETS)


def test_step_llama_layout_ragged(gpu):
    """Interleaved RoPE, no bias, GQA group 3, T not a multiple of the 64-row tiles, B=3."""
    cfg = tiny(8, n_heads=6, n_kv_heads=2, rope_neox=False, attn_bias=False, rope_base=10000.0, dim=192,
               ffn_dim=384, vocab=320, n_layers=3)
    print("peft llama-layout B=3 T=50", flush=True)
    pm, om, ids, tg, lora, TARGETS = run_pair(gpu, cfg, B=3, T=50, seed=5)
    lg = pm.loss_grad(ids, tg)
    lo = om.loss_grad(ids, tg)
    assert abs(lg - lo) / abs(lo) <= TOL
    compare_grads(pm, om, cfg, lora, TARGETS)


@pytest.mark.timeout(600)
@pytest.mark.parametrize("rank", [16, 32])
def test_step_many_rows(gpu, rank):
    """M = 8192 token rows, as in Llama-3.2-1B's B8×T1024 step: the fp16 LoRA rows products then take two 16-row
    tiles per workgroup wherever their width allows (r16: q|k|v 48, gate|up 32, o and down 16 columns; r32: gate|up
    64, o and down 32 — q|k|v at 96 stays at one tile), which the smaller steps above never reach."""
    cfg = tiny(12, lora_rank=rank, lora_alpha=2.0 * rank, n_layers=2)
    print(f"peft tiny Q4_K r{rank} B=16 T=512", flush=True)
    pm, om, ids, tg, lora, TARGETS = run_pair(gpu, cfg, B=16, T=512, seed=11)
    lg = pm.loss_grad(ids, tg)
    lo = om.loss_grad(ids, tg)
    assert abs(lg - lo) / abs(lo) <= TOL
    compare_grads(pm, om, cfg, lora, TARGETS)


def test_reference_faithful_qv_b_zero(gpu):
    """The reference's own setting: LoRA on q and v only, B = 0 (src/peft.rs:187-199). dA must be exactly 0,
    and the adapted logits equal the base (the init-parity check of src/main.rs:2497-2534)."""
    cfg = tiny(8, lora_targets=("q", "v"), attn_bias=False)
    print("peft reference-faithful q,v B=0", flush=True)
    pm, om, ids, tg, lora, TARGETS = run_pair(gpu, cfg, B=1, T=64, b_std=0.0, seed=9)
    lg = pm.loss_grad(ids, tg)
    lo = om.loss_grad(ids, tg)
    assert abs(lg - lo) / abs(lo) <= TOL
    for (l, t) in lora:
        gA, gB = pm.get_lora_grad(l, t)
        assert not gA.any()
        i, ou = cfg.target_dims(t)
        _, oB = om.get_lora_grad(l, TARGETS.index(t), ((i, cfg.lora_rank), (cfg.lora_rank, ou)))
        assert rel_l2(gB, oB) <= TOL
    lgt = pm.logits(ids[0])
    lot = om.logits(ids[0])
    assert rel_l2(lgt, lot) <= TOL


def test_adamw_steps_track_oracle(gpu):
    """Three optimizer steps. At every step the loss and every LoRA gradient (A and B) are checked at the 1e-3
    bar at identical parameters (the GPU model is re-synced to the oracle's parameters after each update), and
    the AdamW update itself is checked for both factors. AdamW's first steps move each element by about ±lr
    whatever the gradient's size (m̂/√v̂ ≈ sign(g)), so a gradient entry within its rounding of zero can flip a
    whole ±lr move: after the update B (which starts small) is held to 5e-3, A to the 1e-3 bar. The update
    arithmetic alone is bit-exact (test_gpu_ops.py::test_adamw_bit_exact)."""
    cfg = tiny(12, n_layers=1, gemm_passes=3)
    print("peft adamw 3 steps", flush=True)
    pm, om, ids, tg, lora, TARGETS = run_pair(gpu, cfg, B=2, T=64, seed=11)
    shapes = {t: ((cfg.target_dims(t)[0], cfg.lora_rank), (cfg.lora_rank, cfg.target_dims(t)[1]))
              for (_, t) in lora}
    for step in range(3):
        lg = pm.loss_grad(ids, tg)
        lo = om.loss_grad(ids, tg)
        assert abs(lg - lo) / abs(lo) <= TOL, f"step {step}"
        for (l, t) in lora:
            gA, gB = pm.get_lora_grad(l, t)
            oA, oB = om.get_lora_grad(l, TARGETS.index(t), shapes[t])
            assert rel_l2(gA, oA) <= TOL and rel_l2(gB, oB) <= TOL, f"step {step} {t} grads"
        pm.adamw(1e-3)
        om.adamw(1e-3, 0.0)
        for (l, t) in lora:
            gA, gB = pm.get_lora(l, t)
            oA, oB = om.get_lora(l, TARGETS.index(t), shapes[t])
            assert rel_l2(gA, oA) <= TOL and rel_l2(gB, oB) <= 5e-3, f"step {step} {t} params"
            pm.set_lora(l, t, oA, oB)


def test_errors_are_reported(gpu):
    from hos_amd import HosError
    from hos_amd.peft import PeftModel
    cfg = tiny(8, n_layers=1)
    pm = PeftModel(gpu, cfg, max_batch=1, max_seq=32)
    ids = np.zeros((1, 32), np.int32)
    with pytest.raises(HosError, match="missing tensor"):
        pm.loss_grad(ids, ids)
    with pytest.raises(HosError):
        pm.set_tensor("blk.0.attn_q.weight", np.zeros(10, np.uint8), 8, 256, 256)
    with pytest.raises(HosError):
        pm.set_tensor("blk.7.attn_q.weight", np.zeros(10, np.uint8), 8, 256, 256)


def test_smollm2_135m_one_step(gpu):
    """configs[0] exactly: SmolLM2-135M architecture, Q8_0, LoRA r=8 (alpha 16) on q/k/v/o, A ~ N(0,0.02),
    one step on 1 x 128. B is drawn ~N(0, 0.02) so every dA is non-zero."""
    from hos_amd.synth import CONFIGS
    cfg = CONFIGS["smollm2-135m"]
    print("peft smollm2-135m B=1 T=128", flush=True)
    pm, om, ids, tg, lora, TARGETS = run_pair(gpu, cfg, B=1, T=128, seed=3)
    lg = pm.loss_grad(ids, tg)
    lo = om.loss_grad(ids, tg)
    assert abs(lg - lo) / abs(lo) <= TOL
    worst = compare_grads(pm, om, cfg, lora, TARGETS)
    print(f"smollm2 loss gpu {lg:.6f} cpu {lo:.6f} worst grad rel L2 {worst:.2e}")


def test_qwen25_05b_config_parity():
    """configs[2] (the benchmark model: Qwen2.5-0.5B architecture, Q4_K with the Q8_0 fallback for 896-wide
    rows, QKV bias, NEOX RoPE 1e6, LoRA r=16 on all seven projections) against the oracle, B=2 x T=48."""
    from hos_amd import Gpu
    from hos_amd.synth import CONFIGS
    g = Gpu(0)
    cfg = CONFIGS["qwen2.5-0.5b"]
    print("peft qwen2.5-0.5b B=2 T=48", flush=True)
    pm, om, ids, tg, lora, TARGETS = run_pair(g, cfg, B=2, T=48, seed=21)
    lg = pm.loss_grad(ids, tg)
    lo = om.loss_grad(ids, tg)
    assert abs(lg - lo) / abs(lo) <= TOL
    worst = compare_grads(pm, om, cfg, lora, TARGETS)
    print(f"qwen loss gpu {lg:.6f} cpu {lo:.6f} worst grad rel L2 {worst:.2e}")
    pm.close()
    g.close()


@pytest.mark.timeout(600)  # the CPU oracle of a 1.2 B-parameter model takes minutes on a loaded host
def test_llama32_1b_config_parity():
    """configs[3] architecture (Llama-3.2-1B: 16 layers, d 2048, 32/8 heads, SwiGLU 8192, vocab 128256,
    tied Q4_K embeddings, interleaved RoPE 5e5) with LoRA r=32 on all projections, B=1 x T=24."""
    from hos_amd import Gpu
    from hos_amd.synth import CONFIGS
    g = Gpu(0)
    cfg = CONFIGS["llama3.2-1b"]
    print("peft llama3.2-1b B=1 T=24", flush=True)
    pm, om, ids, tg, lora, TARGETS = run_pair(g, cfg, B=1, T=24, seed=31)
    lg = pm.loss_grad(ids, tg)
    lo = om.loss_grad(ids, tg)
    assert abs(lg - lo) / abs(lo) <= TOL
    worst = compare_grads(pm, om, cfg, lora, TARGETS)
    print(f"llama loss gpu {lg:.6f} cpu {lo:.6f} worst grad rel L2 {worst:.2e}")
    pm.close()
    g.close()


@pytest.mark.parametrize("name", ["qwen2.5-0.5b", "llama3.2-1b"])
def test_full_size_step_properties(name):
    """The benchmark shapes themselves (B4 x T512 for Qwen2.5-0.5B, B8 x T1024 for Llama-3.2-1B), where the
    oracle would take hours: the step is deterministic (bit-identical loss and gradients on a repeat), every
    gradient is finite, the initial loss of near-uniform logits is close to ln(vocab), B = 0 makes every dA
    exactly zero, and a few AdamW steps on one batch lower its loss."""
    from hos_amd import Gpu, synth
    from hos_amd.peft import PeftModel
    g = Gpu(0)
    cfg = synth.CONFIGS[name]
    B, T = cfg.batch, cfg.seq
    print(f"peft full-size properties {name} B={B} T={T}", flush=True)
    tensors = synth.build_tensors(g, cfg, seed=1)
    lora = synth.lora_init(cfg, seed=2, b_std=0.0)
    ids, tg = synth.tokens(cfg, B, T, seed=3)
    pm = PeftModel(g, cfg, max_batch=B, max_seq=T)
    pm.load(tensors)
    for (l, t), (A, Bm) in lora.items():
        pm.set_lora(l, t, A, Bm)
    l1 = pm.loss_grad(ids, tg)
    grads1 = {k: pm.get_lora_grad(*k) for k in list(lora)[:6]}
    l2 = pm.loss_grad(ids, tg)
    grads2 = {k: pm.get_lora_grad(*k) for k in grads1}
    assert l1 == l2
    for k in grads1:
        dA, dB = grads1[k]
        assert np.array_equal(dA, grads2[k][0]) and np.array_equal(dB, grads2[k][1])
        assert np.isfinite(dB).all() and np.abs(dB).sum() > 0
        assert not dA.any()  # B = 0: the gradient reaching A is exactly zero
    assert abs(l1 - np.log(cfg.vocab)) < 0.5
    losses = [pm.step(ids, tg, lr=1e-3) for _ in range(4)]
    print(f"{name} losses {losses}", flush=True)
    assert losses[-1] < losses[0]
    pm.close()
    g.close()


def test_graph_replay_matches_eager(gpu):
    """hos_peft_step_dev replays a captured graph of the step after its first call. Two identical models,
    one eager and one replaying: after every step (with host synchronisation and eager reads in between)
    the loss and every LoRA factor are bit-identical, including after an lr change between replays."""
    from hos_amd import synth
    from hos_amd.peft import PeftModel
    cfg = tiny(12, n_layers=2)
    print("peft graph replay vs eager", flush=True)
    tensors = synth.build_tensors(gpu, cfg, seed=4)
    lora = synth.lora_init(cfg, seed=5, b_std=0.02)
    ids, tg = synth.tokens(cfg, 2, 64, seed=6)
    models = []
    for graph in (False, True):
        pm = PeftModel(gpu, cfg, max_batch=2, max_seq=64)
        pm.load(tensors)
        for (l, t), (A, Bm) in lora.items():
            pm.set_lora(l, t, A, Bm)
        pm.use_graph(graph)
        models.append(pm)
    I, TG, L = gpu.to_dev(ids), gpu.to_dev(tg), gpu.empty_dev((1,))
    for step, lr in enumerate((1e-3, 1e-3, 3e-3, 1e-3, 1e-3)):
        out = []
        for pm in models:
            pm.step_dev(I.ptr, TG.ptr, 2, 64, lr, 0.01, L.ptr)
            gpu.synchronize()
            out.append((L.get()[0], [pm.get_lora(l, t) for (l, t) in lora]))
        (la, fa), (lb, fb) = out
        assert la == lb, f"step {step}: loss {la} vs {lb}"
        for (A1, B1), (A2, B2) in zip(fa, fb):
            assert np.array_equal(A1, A2) and np.array_equal(B1, B2), f"step {step}"
    for a in (I, TG, L):
        a.free()
    for pm in models:
        pm.close()


def _bench_shape_parity(name, B, T, seed):
    """The whole training step at a shape the benchmark times, against the oracle on the same seeded inputs, with the
    default per-site precision policy: the loss and every LoRA dA / dB (every layer, every target) within 1e-3
    relative L2. At these row counts the tile rule picks the kernels the benchmark runs (the 256-row head tiles
    with the fused softmax statistics, split contractions whose first split carries the rank-r term, the 64-deep
    two-plane slabs), which the small-shape parity tests above never reach."""
    import time
    from conftest import heartbeat
    from hos_amd import Gpu
    from hos_amd.synth import CONFIGS
    g = Gpu(0)
    cfg = CONFIGS[name]
    print(f"peft bench-shape parity {name} B={B} T={T}", flush=True)
    pm, om, ids, tg, lora, TARGETS = run_pair(g, cfg, B=B, T=T, seed=seed)
    lg = pm.loss_grad(ids, tg)
    print(f"gpu loss {lg:.6f}; running the oracle on the host", flush=True)
    t0 = time.time()
    with heartbeat(f"oracle {name} B{B}xT{T}"):
        lo = om.loss_grad(ids, tg)
    print(f"oracle loss {lo:.6f} in {time.time() - t0:.1f} s", flush=True)
    assert abs(lg - lo) / abs(lo) <= TOL
    worst = compare_grads(pm, om, cfg, lora, TARGETS)
    print(f"{name} B{B}xT{T}: loss gpu {lg:.6f} cpu {lo:.6f}, worst LoRA grad rel L2 {worst:.2e} "
          f"over {2 * len(lora)} gradients", flush=True)
    pm.close()
    g.close()


@pytest.mark.timeout(1200)  # the oracle's 4 x 512-token step takes minutes on the host
def test_qwen25_05b_bench_shape_parity():
    """configs[2] at the benchmark's own batch: Qwen2.5-0.5B architecture, B4 x T512 (M = 2048 rows)."""
    _bench_shape_parity("qwen2.5-0.5b", 4, 512, seed=41)


@pytest.mark.timeout(1200)
def test_llama32_1b_long_sequence_parity():
    """configs[3] architecture with LoRA r32 on all projections at T = 1024 (the benchmark's sequence length;
    M = 1024 rows, causal attention over the full sequence), B1."""
    _bench_shape_parity("llama3.2-1b", 1, 1024, seed=43)
