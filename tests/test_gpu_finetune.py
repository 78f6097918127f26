"""Full-parameter finetune step (hos_ft_*, FtModel of src/finetune.rs) against the oracle's FtModel
restatement (oracle/peft.cpp with every weight trainable), same bytes, same tokens.

Bar: loss and every parameter's gradient within 1e-3 relative L2 of the f32 CPU path; AdamW steps track
the oracle's parameters; the step is deterministic.
"""
import numpy as np
import pytest

from oracle import binding as o
from test_gpu_peft import TOL, rel_l2

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def gpu():
    from hos_amd import Gpu
    g = Gpu(0)
    yield g
    g.close()


def ft_cfg(**kw):
    from hos_amd.peft import ModelConfig
    base = dict(name="ft-tiny", n_layers=2, dim=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn_dim=512, vocab=384,
                rms_eps=1e-6, rope_base=1e6, rope_neox=True, attn_bias=True, lora_rank=8, lora_alpha=16.0,
                lora_targets=(), quant=12, head_quant=8)
    base.update(kw)
    return ModelConfig(**base)


def names_shapes(cfg):
    from hos_amd import synth
    out = []
    for name, rows, cols, kind in synth.tensor_list(cfg):
        out.append((name, (rows, cols) if kind not in ("norm", "bias") else (cols,)))
    if not any(n == "output.weight" for n, _ in out):
        out.append(("output.weight", (cfg.vocab, cfg.dim)))
    return out


def pair(gpu, cfg, B, T, seed):
    from hos_amd import synth
    from hos_amd.finetune import FtModel
    tensors = synth.build_tensors(gpu, cfg, seed=seed, norm_jitter=0.2)
    ft = FtModel(gpu, cfg, max_batch=B, max_seq=T)
    ft.load(tensors)
    om = o.OracleFt(cfg)
    for name, (raw, t, rows, cols) in tensors.items():
        om.set_tensor(name, raw, t, rows, cols)
    ids, tg = synth.tokens(cfg, B, T, seed=seed + 1)
    return ft, om, ids, tg


# T 40: 80 tokens, the f32 weight-gradient GEMM; T 48: 96 tokens, a multiple of 32, the fp16-MFMA one over dYᵀ
@pytest.mark.parametrize("T", [40, 48])
@pytest.mark.parametrize("kw", [{}, dict(attn_bias=False, rope_neox=False, n_heads=6, n_kv_heads=3, dim=384,
                                        quant=8, head_quant=8, vocab=320)])
def test_finetune_grads_match_oracle(gpu, kw, T):
    cfg = ft_cfg(**kw)
    print(f"finetune parity {kw} T={T}", flush=True)
    ft, om, ids, tg = pair(gpu, cfg, B=2, T=T, seed=3)
    lg, lo = ft.loss_grad(ids, tg), om.loss_grad(ids, tg)
    assert abs(lg - lo) / abs(lo) <= TOL, (lg, lo)
    worst = 0.0
    for name, shape in names_shapes(cfg):
        gv, gg = ft.get(name, shape)
        ov, og = om.get(name, shape)
        assert np.array_equal(gv, ov), name  # same dequantized values
        e = rel_l2(gg, og)
        worst = max(worst, e)
        assert e <= TOL, f"{name}: grad rel L2 {e:.3e}"
    print(f"finetune loss gpu {lg:.6f} cpu {lo:.6f} worst grad rel L2 {worst:.2e}", flush=True)
    ft.close()


def test_finetune_adamw_tracks_oracle_and_is_deterministic(gpu):
    cfg = ft_cfg(n_layers=1)
    print("finetune adamw + determinism", flush=True)
    ft, om, ids, tg = pair(gpu, cfg, B=1, T=32, seed=7)
    l1 = ft.loss_grad(ids, tg)
    g1 = ft.get("blk.0.attn_q.weight", (256, 256))[1]
    l2 = ft.loss_grad(ids, tg)
    assert l1 == l2 and np.array_equal(g1, ft.get("blk.0.attn_q.weight", (256, 256))[1])
    for step in range(3):
        ft.step(ids, tg, lr=1e-3)
        om.loss_grad(ids, tg)
        om.adamw(1e-3, 0.0)
    # AdamW's first steps move every element by about ±lr whatever its gradient's size, so elements whose
    # gradient is near zero can step apart; the parameters still agree to a small fraction of the updates
    # (3 steps of lr 1e-3 on weights ~0.02 move them by ~10%).
    # The k bias is left out: adding a constant to every key shifts each query's scores by a constant,
    # which the softmax ignores, so its gradient is ~0 (RoPE only) and Adam's normalised step is noise.
    for name, shape in names_shapes(cfg):
        if name.endswith("attn_k.bias"):
            continue
        gv, _ = ft.get(name, shape)
        ov, _ = om.get(name, shape)
        assert rel_l2(gv, ov) < 5e-4, name
    ft.close()


def test_finetune_untied_head(gpu):
    cfg = ft_cfg(n_layers=1)
    print("finetune untied head", flush=True)
    ft, om, ids, tg = pair(gpu, cfg, B=1, T=24, seed=11)
    e0 = ft.get("token_embd.weight", (cfg.vocab, cfg.dim))[0]
    h0 = ft.get("output.weight", (cfg.vocab, cfg.dim))[0]
    assert np.array_equal(e0, h0)
    ft.step(ids, tg, lr=1e-3)
    e1 = ft.get("token_embd.weight", (cfg.vocab, cfg.dim))[0]
    h1 = ft.get("output.weight", (cfg.vocab, cfg.dim))[0]
    assert not np.array_equal(e1, h1)
    unused = np.setdiff1d(np.arange(cfg.vocab), ids.ravel())
    assert np.array_equal(e1[unused], e0[unused])  # embedding rows of unseen tokens: zero gradient, no step
    ft.close()


def test_finetune_qwen_full_width_properties(gpu):
    """Qwen2.5-0.5B architecture at B1 x T256 (all 494 M weights trainable in f32 on the device):
    deterministic, finite gradients, loss near ln(vocab), AdamW steps lower the loss."""
    from hos_amd import synth
    from hos_amd.finetune import FtModel
    cfg = synth.CONFIGS["qwen2.5-0.5b"]
    print("finetune qwen2.5-0.5b B=1 T=256", flush=True)
    tensors = synth.build_tensors(gpu, cfg, seed=1)
    ft = FtModel(gpu, cfg, max_batch=1, max_seq=256)
    ft.load(tensors)
    ids, tg = synth.tokens(cfg, 1, 256, seed=2)
    l1 = ft.loss_grad(ids, tg)
    g1 = ft.get("blk.3.ffn_down.weight", (cfg.dim, cfg.ffn_dim))[1]
    assert np.isfinite(g1).all() and np.abs(g1).sum() > 0
    assert l1 == ft.loss_grad(ids, tg)
    assert abs(l1 - np.log(cfg.vocab)) < 0.5
    losses = [ft.step(ids, tg, lr=1e-4) for _ in range(3)]
    print(f"finetune qwen losses {losses}", flush=True)
    assert losses[-1] < losses[0]
    ft.close()
