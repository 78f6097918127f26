"""Pins the oracle's full-parameter finetune model (FtModel, src/finetune.rs: every weight trainable,
untied head copy, AdamW over FtModel::params with decay on 2-D tensors):

* the loss equals the LoRA model's at B = 0 (same forward), and weight gradients match central
  differences of the loss for matrices, norms, biases, the embedding and the head;
* the head starts as an exact copy of the tied embedding but is a separate parameter: its gradient is the
  head's alone, and an AdamW step moves the two apart.
"""
import types

import numpy as np

from oracle import binding as o


def _cfg():
    from hos_amd.peft import ModelConfig
    return ModelConfig("ft-tiny", n_layers=2, dim=64, n_heads=2, n_kv_heads=1, head_dim=32, ffn_dim=96, vocab=80,
                       rms_eps=1e-5, rope_base=10000.0, rope_neox=True, attn_bias=True, lora_rank=4, lora_alpha=8.0,
                       lora_targets=("q", "v"), quant=8, head_quant=8)


def _tensors(cfg, seed):
    from hos_amd import synth
    return synth.build_tensors(None, cfg, seed=seed, quantize=lambda w, t: o.quantize(w, t), norm_jitter=0.2)


def _ft(cfg, tensors):
    m = o.OracleFt(cfg)
    for name, (raw, t, rows, cols) in tensors.items():
        m.set_tensor(name, raw, t, rows, cols)
    return m


def _shape(tensors, name):
    _, _, rows, cols = tensors.get(name, tensors["token_embd.weight"] if name == "output.weight" else None)
    return (rows, cols) if rows > 1 else (cols,)


def test_loss_equals_frozen_lora_model_at_b_zero():
    cfg = _cfg()
    tensors = _tensors(cfg, 1)
    ids = np.random.default_rng(2).integers(0, cfg.vocab, size=(2, 11)).astype(np.int32)
    tg = np.roll(ids, -1, axis=1)
    ft = _ft(cfg, tensors)
    oc = types.SimpleNamespace(**{k: getattr(cfg, k) for k in (
        "n_layers", "dim", "n_heads", "n_kv_heads", "head_dim", "ffn_dim", "vocab", "rms_eps", "rope_base",
        "rope_neox", "attn_bias", "lora_rank", "lora_alpha")})
    oc.lora_targets = cfg.target_mask
    lm = o.OracleModel(oc)
    for name, (raw, t, rows, cols) in tensors.items():
        lm.set_tensor(name, raw, t, rows, cols)
    assert ft.loss_grad(ids, tg) == lm.loss_grad(ids, tg)


def test_weight_gradients_match_finite_differences():
    cfg = _cfg()
    tensors = _tensors(cfg, 3)
    ids = np.random.default_rng(4).integers(0, cfg.vocab, size=(1, 9)).astype(np.int32)
    tg = np.roll(ids, -1, axis=1)
    ft = _ft(cfg, tensors)
    ft.loss_grad(ids, tg)
    hshape = _shape(tensors, "output.weight")
    hv, _ = ft.get("output.weight", hshape)
    _, _, vr, vc = tensors["token_embd.weight"]
    base = dict(tensors)  # the head explicitly (F32): perturbing the embedding must not move it
    base["output.weight"] = (hv.astype(np.float32).view(np.uint8).ravel(), 0, vr, vc)
    names = ["token_embd.weight", "output.weight", "output_norm.weight", "blk.0.attn_q.weight",
             "blk.0.attn_k.bias", "blk.1.attn_output.weight", "blk.1.ffn_norm.weight", "blk.0.ffn_down.weight",
             "blk.1.ffn_gate.weight"]
    rng = np.random.default_rng(5)
    for name in names:
        shape = _shape(tensors, name)
        v, g = ft.get(name, shape)
        picks = list(np.argsort(-np.abs(g).ravel())[:2]) + list(rng.integers(0, g.size, 1))
        for flat in picks:
            eps = np.float32(1e-2 * max(1.0, abs(v.ravel()[flat])))
            vals = []
            for sgn in (1, -1):
                t2 = dict(base)
                w = v.copy().ravel()
                w[flat] += sgn * eps
                w = w.reshape(shape)
                raw, t, rows, cols = base[name]
                t2[name] = (w.astype(np.float32).view(np.uint8).ravel(), 0, rows, cols)  # as F32
                m = _ft(cfg, t2)
                vals.append(m.loss_grad(ids, tg))
            num = (vals[0] - vals[1]) / (2 * eps)
            ana = g.ravel()[flat]
            assert abs(num - ana) <= 3e-3 + 5e-2 * abs(ana), f"{name}[{flat}]: numeric {num} analytic {ana}"


def test_head_is_an_untied_copy():
    cfg = _cfg()
    tensors = _tensors(cfg, 6)
    ids = np.random.default_rng(7).integers(0, cfg.vocab, size=(1, 9)).astype(np.int32)
    tg = np.roll(ids, -1, axis=1)
    ft = _ft(cfg, tensors)
    shape = _shape(tensors, "token_embd.weight")
    e0, _ = ft.get("token_embd.weight", shape)
    h0, _ = ft.get("output.weight", shape)
    assert np.array_equal(e0, h0)
    ft.loss_grad(ids, tg)
    _, ge = ft.get("token_embd.weight", shape)
    _, gh = ft.get("output.weight", shape)
    assert not np.array_equal(ge, gh)
    assert np.count_nonzero(np.abs(ge).sum(1)) <= len(set(ids[0].tolist()))  # rows of the input tokens only
    ft.adamw(1e-3, 0.0)
    e1, _ = ft.get("token_embd.weight", shape)
    h1, _ = ft.get("output.weight", shape)
    assert not np.array_equal(e1, h1)
