"""RGA adapters (Regulatory Genome Adapters, src/peft.rs:61-96, 200-215, 491-499, 565-584) on the device
training step, against the oracle's restatement on the same quantized bytes, adapter values and tokens.

Bar (as for LoRA): loss and every adapter gradient within relative L2 1e-3 of the CPU f32 path.

* gradients of every RGA tensor (genome, wg, each layer's wr, downs, ups) with the gate sparsity term on;
* up = 0 (the reference's init) leaves the model exactly the base model (logits bit-identical);
* AdamW steps track the oracle; a captured-graph replay is bit-identical to eager steps;
* the .hos checkpoint carries the reference's adapter tensor names (genome.0, wg, rga.{l}.wr / down.{k} /
  up.{k}) and the optimizer state in parameter order, and resuming from it continues bit-identically.
"""
import json
import types

import numpy as np
import pytest

from oracle import binding as o
from oracle import hos_format as hf

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


def cfg_rga(**kw):
    from hos_amd.peft import ModelConfig
    base = dict(name="rga-tiny", n_layers=2, dim=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn_dim=512,
                vocab=512, rms_eps=1e-6, rope_base=1e6, rope_neox=True, attn_bias=True, lora_rank=8,
                lora_alpha=16.0, lora_targets=(), quant=8, head_quant=8, rga_genes=4, rga_bottleneck=4,
                rga_lambda=0.05)
    base.update(kw)
    return ModelConfig(**base)


def oracle_model(cfg, tensors, params):
    oc = types.SimpleNamespace(**{k: getattr(cfg, k) for k in (
        "n_layers", "dim", "n_heads", "n_kv_heads", "head_dim", "ffn_dim", "vocab", "rms_eps", "rope_base",
        "rope_neox", "attn_bias", "lora_rank", "lora_alpha", "rga_genes", "rga_bottleneck", "rga_lambda")})
    oc.lora_targets = cfg.target_mask
    m = o.OracleModel(oc)
    for name, (raw, t, rows, cols) in tensors.items():
        m.set_tensor(name, raw, t, rows, cols)
    for name, v in params.items():
        m.set_rga(name, v)
    return m


def device_model(gpu, cfg, tensors, params, B, T):
    from hos_amd.peft import PeftModel
    pm = PeftModel(gpu, cfg, max_batch=B, max_seq=T)
    pm.load(tensors)
    for name, v in params.items():
        pm.set_rga(name, v)
    return pm


def run_pair(gpu, cfg, B, T, seed=0, up_std=0.02, std=0.02):
    from hos_amd import synth
    tensors = synth.build_tensors(gpu, cfg, seed=seed)
    params = synth.rga_init(cfg, seed=seed + 1, std=std, up_std=up_std)
    ids, tg = synth.tokens(cfg, B, T, seed=seed + 2)
    return device_model(gpu, cfg, tensors, params, B, T), oracle_model(cfg, tensors, params), ids, tg, tensors, \
        params


@pytest.mark.parametrize("quant", [8, 12])
def test_gradients_match_oracle(gpu, quant):
    cfg = cfg_rga(quant=quant, head_quant=quant)
    print(f"rga tiny quant={quant} B=2 T=80", flush=True)
    pm, om, ids, tg, _, params = run_pair(gpu, cfg, 2, 80, seed=3, std=0.05)
    lg, lo = pm.loss_grad(ids, tg), om.loss_grad(ids, tg)
    assert abs(lg - lo) / abs(lo) <= TOL
    worst = 0.0
    for name, shape in cfg.rga_shapes().items():
        _, g = pm.get_rga(name)
        _, w = om.get_rga(name, shape)
        e = rel_l2(g, w)
        worst = max(worst, e)
        assert e <= TOL, f"{name}: rel L2 {e:.3e}"
    print(f"worst rel L2 {worst:.2e}", flush=True)


def test_smollm2_shapes_with_rga(gpu):
    """SmolLM2-135M layer shapes (d 576, 9/3 heads, FFN 1536), 4 genes of bottleneck 4, λ = 1e-3 (cmd_peft's
    defaults, src/main.rs:1017, 2559-2562), three layers."""
    cfg = cfg_rga(dim=576, n_heads=9, n_kv_heads=3, ffn_dim=1536, vocab=2048, n_layers=3, rope_base=10000.0,
                  rope_neox=False, attn_bias=False, rga_lambda=1e-3)
    print("rga smollm2 shapes B=1 T=64", flush=True)
    pm, om, ids, tg, _, _ = run_pair(gpu, cfg, 1, 64, seed=21, up_std=0.02)
    lg, lo = pm.loss_grad(ids, tg), om.loss_grad(ids, tg)
    assert abs(lg - lo) / abs(lo) <= TOL
    for name, shape in cfg.rga_shapes().items():
        _, g = pm.get_rga(name)
        _, w = om.get_rga(name, shape)
        assert rel_l2(g, w) <= TOL, name


def test_up_zero_is_the_base_model(gpu):
    from hos_amd import synth
    from hos_amd.peft import PeftModel
    cfg = cfg_rga()
    print("rga up=0 init parity", flush=True)
    tensors = synth.build_tensors(gpu, cfg, seed=7)
    params = synth.rga_init(cfg, seed=8)  # ups = 0, as the reference initializes them
    pm = device_model(gpu, cfg, tensors, params, 1, 40)
    base_cfg = cfg_rga(rga_genes=0, lora_targets=("q",))
    bm = PeftModel(gpu, base_cfg, max_batch=1, max_seq=40)
    bm.load(tensors)  # LoRA B = 0 (never set): the base model
    ids, _ = synth.tokens(cfg, 1, 40, seed=9)
    assert np.array_equal(pm.logits(ids[0]), bm.logits(ids[0]))


def test_adamw_steps_track_oracle(gpu):
    cfg = cfg_rga(n_layers=1, gemm_passes=3)
    print("rga adamw 3 steps", flush=True)
    pm, om, ids, tg, _, _ = run_pair(gpu, cfg, 2, 48, seed=31, std=0.05, up_std=0.05)
    for step in range(3):
        lg = pm.step(ids, tg, lr=1e-3)
        lo = om.loss_grad(ids, tg)
        om.adamw(1e-3, 0.0)
        assert abs(lg - lo) / abs(lo) <= TOL, f"step {step}"
    for name, shape in cfg.rga_shapes().items():
        v, _ = pm.get_rga(name)
        w, _ = om.get_rga(name, shape)
        assert rel_l2(v, w) <= 5e-3, name


def test_graph_replay_matches_eager(gpu):
    from hos_amd import synth
    cfg = cfg_rga()
    print("rga graph replay vs eager", flush=True)
    tensors = synth.build_tensors(gpu, cfg, seed=41)
    params = synth.rga_init(cfg, seed=42, up_std=0.02)
    ids, tg = synth.tokens(cfg, 2, 32, seed=43)
    models = []
    for graph in (False, True):
        pm = device_model(gpu, cfg, tensors, params, 2, 32)
        pm.use_graph(graph)
        models.append(pm)
    I, TG, L = gpu.to_dev(ids), gpu.to_dev(tg), gpu.empty_dev((1,))
    for step, lr in enumerate((1e-3, 1e-3, 3e-3, 1e-3)):
        out = []
        for pm in models:
            pm.step_dev(I.ptr, TG.ptr, 2, 32, lr, 0.0, L.ptr)
            gpu.synchronize()
            out.append((L.get()[0], [pm.get_rga(n)[0] for n in cfg.rga_shapes()]))
        (la, fa), (lb, fb) = out
        assert la == lb, f"step {step}: loss {la} vs {lb}"
        for a, b in zip(fa, fb):
            assert np.array_equal(a, b), f"step {step}"
    for a in (I, TG, L):
        a.free()
    for pm in models:
        pm.close()


def test_checkpoint_names_and_resume(gpu, tmp_path):
    from hos_amd import synth
    cfg = cfg_rga(rga_genes=2, rga_bottleneck=3)
    print("rga checkpoint resume", flush=True)
    tensors = synth.build_tensors(gpu, cfg, seed=51)
    params = synth.rga_init(cfg, seed=52, up_std=0.02)
    ids, tg = synth.tokens(cfg, 1, 32, seed=53)
    pm = device_model(gpu, cfg, tensors, params, 1, 32)
    for _ in range(2):
        pm.step(ids, tg, lr=1e-3)
    path = tmp_path / "rga.hos"
    pm.save_hos(str(path), optimizer=True)
    ver, card, ts, ok = hf.read(path.read_bytes())
    assert ok and ver == 2
    names = [t[0] for t in ts]
    want = ["genome.0", "wg"]
    for l in range(cfg.n_layers):  # PeftModel::adapter_tensors order (src/peft.rs:741-760)
        want.append(f"rga.{l}.wr")
        for k in range(cfg.rga_genes):
            want += [f"rga.{l}.down.{k}", f"rga.{l}.up.{k}"]
    assert names[:len(want)] == want
    n_params = len(cfg.rga_shapes())
    assert sum(1 for n in names if n.startswith("opt.m.")) == n_params
    byname = {t[0]: t for t in ts}
    for name, shape in cfg.rga_shapes().items():
        v, _ = pm.get_rga(name)
        _, _, _, sh, _, raw = byname[name]
        assert list(sh) == list(shape)
        assert np.array_equal(np.frombuffer(raw, np.float32).reshape(shape), v), name
    # opt.m.{k} follows the parameter order (PeftModel::params, src/peft.rs:283-311): k = 0 is wg
    assert byname["opt.m.0"][3] == [8 * cfg.rga_genes]
    assert json.loads(card)["arch"]["method"] == "rga"
    fresh = device_model(gpu, cfg, tensors, synth.rga_init(cfg, seed=99), 1, 32)
    fresh.load_hos(str(path), optimizer=True)
    la, lb = pm.step(ids, tg, lr=1e-3), fresh.step(ids, tg, lr=1e-3)
    assert la == lb
    for name in cfg.rga_shapes():
        assert np.array_equal(pm.get_rga(name)[0], fresh.get_rga(name)[0]), name


def test_full_size_step_properties():
    """The benchmark shapes (Qwen2.5-0.5B architecture, B4 x T512) with RGA at cmd_peft's defaults (4 genes,
    bottleneck 4, λ 1e-3), where the oracle would take hours: the step is deterministic (bit-identical loss and
    gradients on a repeat), every gradient is finite, up = 0 makes every down gradient exactly zero (dG = dx·Upᵀ
    vanishes) while wr still moves through the sparsity term, the initial loss is ln(vocab) plus about
    λ·mean(gate), and a few AdamW steps on one batch lower the loss."""
    import dataclasses

    from hos_amd import Gpu, synth
    g = Gpu(0)
    cfg = dataclasses.replace(synth.CONFIGS["qwen2.5-0.5b"], lora_targets=(), rga_genes=4, rga_bottleneck=4,
                              rga_lambda=1e-3)
    B, T = cfg.batch, cfg.seq
    print(f"rga full-size properties B={B} T={T}", flush=True)
    tensors = synth.build_tensors(g, cfg, seed=1)
    params = synth.rga_init(cfg, seed=2)  # ups = 0
    ids, tg = synth.tokens(cfg, B, T, seed=3)
    pm = device_model(g, cfg, tensors, params, B, T)
    l1 = pm.loss_grad(ids, tg)
    names = ["genome.0", "wg", "rga.0.wr", "rga.0.down.1", "rga.23.up.3", "rga.11.down.0"]
    g1 = {n: pm.get_rga(n)[1] for n in names}
    l2 = pm.loss_grad(ids, tg)
    g2 = {n: pm.get_rga(n)[1] for n in names}
    assert l1 == l2
    for n in names:
        assert np.array_equal(g1[n], g2[n]), n
        assert np.isfinite(g1[n]).all(), n
    assert not g1["rga.0.down.1"].any() and not g1["rga.11.down.0"].any()
    assert np.abs(g1["rga.0.wr"]).sum() > 0 and np.abs(g1["rga.23.up.3"]).sum() > 0
    assert abs(l1 - np.log(cfg.vocab)) < 0.5
    losses = [pm.step(ids, tg, lr=1e-3) for _ in range(4)]
    print(f"rga losses {losses}", flush=True)
    assert losses[-1] < losses[0]
    pm.close()
    g.close()
