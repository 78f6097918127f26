"""Pins the oracle's mixture-of-experts FFN and QK-norm (oracle/peft.cpp moe_ffn, restating
src/forward.rs:487-493 and :542-572 for the training path; the reference's PEFT has no MoE backward, so
these checks fix what the mathematics does):

* E = 1, top-1: the router's softmax is exactly 1, so the MoE model equals the dense model with the same
  expert weights — logits and every LoRA gradient bit-identical;
* a zero router: every probability is exactly 1/E, the stable sort picks experts 0 .. k-1, and the raw
  (not renormalised) probabilities weight them — with experts 0 and 1 equal to a dense FFN and k = 2 of
  E = 4 this is exactly the dense model with its down projection halved (bit-identical);
* central differences of the loss against the LoRA gradients through a random router, top-2 of 4
  experts and QK-norm;
* relabelling the experts (router rows and expert blocks permuted together) changes nothing beyond the
  softmax's summation order.
"""
import copy

import numpy as np
import pytest

from oracle import binding as o

Q8 = 8


def _cfg(**kw):
    from hos_amd.peft import ModelConfig
    base = dict(name="moe-tiny", n_layers=2, dim=64, n_heads=2, n_kv_heads=2, head_dim=32, ffn_dim=64, vocab=96,
                rms_eps=1e-5, rope_base=10000.0, rope_neox=True, lora_rank=4, lora_alpha=8.0,
                lora_targets=("q", "k", "v", "o"), quant=Q8, head_quant=Q8, n_experts=4, n_experts_used=2,
                qk_norm=True)
    base.update(kw)
    return ModelConfig(**base)


def _tensors(cfg, seed):
    from hos_amd import synth
    return synth.build_tensors(None, cfg, seed=seed, quantize=lambda w, t: o.quantize(w, t), norm_jitter=0.2)


def _model(cfg, tensors, lora):
    import types
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


def _lora(cfg, seed):
    from hos_amd import synth
    return synth.lora_init(cfg, seed=seed, b_std=0.05)


def _grads(m, cfg, lora):
    out = {}
    for (l, t) in lora:
        i, ou = cfg.target_dims(t)
        out[(l, t)] = m.get_lora_grad(l, ("q", "k", "v", "o").index(t), ((i, cfg.lora_rank), (cfg.lora_rank, ou)))
    return out


def _dense_from_moe(tensors, cfg, expert=0, down_scale=1.0):
    """The dense model whose FFN is expert `expert` of the MoE tensors (Q8_0 rows re-quantized from their
    dequantized values, with the down projection scaled by a power of two)."""
    out = {}
    f, d = cfg.ffn_dim, cfg.dim
    for name, (raw, t, rows, cols) in tensors.items():
        if name.endswith("ffn_gate_inp.weight"):
            continue
        for k, per in (("gate", f), ("up", f), ("down", d)):
            if name.endswith(f"ffn_{k}_exps.weight"):
                w = o.dequant(raw, t, rows * cols).reshape(rows, cols)[expert * per:(expert + 1) * per]
                if k == "down":
                    w = w * np.float32(down_scale)
                q = o.quantize(np.ascontiguousarray(w, np.float32), t)
                assert np.array_equal(o.dequant(q, t, w.size).reshape(w.shape), w)  # exact round trip
                out[name.replace(f"ffn_{k}_exps", f"ffn_{k}")] = (q, t, per, cols)
                break
        else:
            out[name] = (raw, t, rows, cols)
    return out


def test_single_expert_equals_dense():
    cfg = _cfg(n_experts=1, n_experts_used=1)
    tensors = _tensors(cfg, 1)
    dcfg = copy.copy(cfg)
    dcfg.n_experts = dcfg.n_experts_used = 0
    lora = _lora(cfg, 2)
    mm, md = _model(cfg, tensors, lora), _model(dcfg, _dense_from_moe(tensors, cfg), lora)
    ids = np.random.default_rng(3).integers(0, cfg.vocab, size=(2, 17)).astype(np.int32)
    tg = np.roll(ids, -1, axis=1)
    assert np.array_equal(mm.logits(ids[0]), md.logits(ids[0]))
    assert mm.loss_grad(ids, tg) == md.loss_grad(ids, tg)
    gm, gd = _grads(mm, cfg, lora), _grads(md, cfg, lora)
    for k in gm:
        for a, b in zip(gm[k], gd[k]):
            assert np.array_equal(a, b), k


def test_zero_router_is_first_experts_with_raw_probabilities():
    cfg = _cfg(n_experts=4, n_experts_used=2)
    tensors = _tensors(cfg, 4)
    for l in range(cfg.n_layers):  # zero router; expert 1 := expert 0
        name = f"blk.{l}.ffn_gate_inp.weight"
        raw, t, rows, cols = tensors[name]
        tensors[name] = (np.zeros(rows * cols, np.float32).view(np.uint8), t, rows, cols)
        for k, per in (("gate", cfg.ffn_dim), ("up", cfg.ffn_dim), ("down", cfg.dim)):
            name = f"blk.{l}.ffn_{k}_exps.weight"
            raw, t, rows, cols = tensors[name]
            b = np.frombuffer(np.ascontiguousarray(raw).tobytes(), np.uint8).copy()
            eb = o.bytes_for(t, per * cols)
            b[eb:2 * eb] = b[:eb]
            tensors[name] = (b, t, rows, cols)
    dcfg = copy.copy(cfg)
    dcfg.n_experts = dcfg.n_experts_used = 0
    lora = _lora(cfg, 5)
    mm, md = _model(cfg, tensors, lora), _model(dcfg, _dense_from_moe(tensors, cfg, 0, 0.5), lora)
    ids = np.random.default_rng(6).integers(0, cfg.vocab, size=(1, 21)).astype(np.int32)
    tg = np.roll(ids, -1, axis=1)
    assert np.array_equal(mm.logits(ids[0]), md.logits(ids[0]))
    assert mm.loss_grad(ids, tg) == md.loss_grad(ids, tg)
    gm, gd = _grads(mm, cfg, lora), _grads(md, cfg, lora)
    for k in gm:
        for a, b in zip(gm[k], gd[k]):
            assert np.array_equal(a, b), k


def test_expert_relabelling_invariant():
    cfg = _cfg()
    tensors = _tensors(cfg, 7)
    perm = np.array([2, 0, 3, 1])
    pt = dict(tensors)
    for l in range(cfg.n_layers):
        name = f"blk.{l}.ffn_gate_inp.weight"
        raw, t, rows, cols = tensors[name]
        r = np.frombuffer(np.ascontiguousarray(raw).tobytes(), np.float32).reshape(rows, cols)[perm]
        pt[name] = (np.ascontiguousarray(r).view(np.uint8).ravel(), t, rows, cols)
        for k, per in (("gate", cfg.ffn_dim), ("up", cfg.ffn_dim), ("down", cfg.dim)):
            name = f"blk.{l}.ffn_{k}_exps.weight"
            raw, t, rows, cols = tensors[name]
            b = np.frombuffer(np.ascontiguousarray(raw).tobytes(), np.uint8)
            eb = o.bytes_for(t, per * cols)
            pt[name] = (np.concatenate([b[e * eb:(e + 1) * eb] for e in perm]), t, rows, cols)
    lora = _lora(cfg, 8)
    ma, mb = _model(cfg, tensors, lora), _model(cfg, pt, lora)
    ids = np.random.default_rng(9).integers(0, cfg.vocab, size=(1, 19)).astype(np.int32)
    tg = np.roll(ids, -1, axis=1)
    # (equal up to the softmax's summation order over the experts)
    np.testing.assert_allclose(ma.logits(ids[0]), mb.logits(ids[0]), rtol=1e-5, atol=1e-6)
    assert abs(ma.loss_grad(ids, tg) - mb.loss_grad(ids, tg)) < 1e-5


def test_finite_differences_through_router_and_qk_norm():
    cfg = _cfg()
    tensors = _tensors(cfg, 10)
    lora = _lora(cfg, 11)
    ids = np.random.default_rng(12).integers(0, cfg.vocab, size=(1, 13)).astype(np.int32)
    tg = np.roll(ids, -1, axis=1)
    m = _model(cfg, tensors, lora)
    m.loss_grad(ids, tg)
    g = _grads(m, cfg, lora)
    rng = np.random.default_rng(13)
    checked = 0
    for (l, t) in [(0, "q"), (0, "k"), (1, "v"), (0, "o")]:
        A, B = lora[(l, t)]
        gA = g[(l, t)][0]
        for flat in np.argsort(-np.abs(gA).ravel())[:3].tolist() + rng.integers(0, gA.size, 2).tolist():
            eps = np.float32(2e-3)
            vals = []
            for sgn in (1, -1):
                A2 = A.copy().ravel()
                A2[flat] += sgn * eps
                lo = dict(lora)
                lo[(l, t)] = (A2.reshape(A.shape), B)
                vals.append(_model(cfg, tensors, lo).loss_grad(ids, tg))
            num = (vals[0] - vals[1]) / (2 * eps)
            ana = gA.ravel()[flat]
            assert abs(num - ana) <= 2e-3 + 3e-2 * abs(ana), f"{l} {t} A[{flat}]: numeric {num} analytic {ana}"
            checked += 1
    assert checked == 20
