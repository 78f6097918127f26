"""Model loading from a GGUF file (hos_peft_create_from_gguf: src/gguf.rs:225-286 + Model::load,
src/model.rs:713-921) gives the same model as loading the same tensors one by one: identical loss and
LoRA gradients, and an unsupported linear-weight encoding is refused by name."""
import numpy as np
import pytest

from gguf_writer import gguf_bytes, model_meta, model_tensors

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def gpu():
    from hos_amd import Gpu
    g = Gpu(0)
    yield g
    g.close()


def _tiny(**kw):
    from hos_amd.peft import ModelConfig
    base = dict(name="tiny", n_layers=2, dim=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn_dim=512, vocab=512,
                rms_eps=1e-6, rope_base=1e6, rope_neox=True, attn_bias=True, lora_rank=8, lora_alpha=16.0,
                lora_targets=("q", "k", "v", "o", "gate", "up", "down"), quant=12, head_quant=14)
    base.update(kw)
    return ModelConfig(**base)


def _f16_round(tensors):
    """1-D tensors rounded through f16, so a file that stores them as F16 holds the same values."""
    out = {}
    for n, (raw, t, rows, cols) in tensors.items():
        if rows == 1 and t == 0:
            v = np.frombuffer(np.ascontiguousarray(raw).tobytes(), np.float32).astype(np.float16).astype(np.float32)
            raw = v.view(np.uint8)
        out[n] = (raw, t, rows, cols)
    return out


@pytest.mark.parametrize("arch,alignment,norm_type,tied", [("qwen2", 32, 1, True), ("llama", 64, 0, False)])
def test_gguf_load_matches_tensor_load(gpu, tmp_path, arch, alignment, norm_type, tied):
    from hos_amd import synth
    from hos_amd.peft import PeftModel
    neox = arch == "qwen2"
    cfg = _tiny(rope_neox=neox, attn_bias=neox, tied=tied, rope_base=1e6 if neox else 5e5)
    print(f"gguf load arch={arch} align={alignment} norm_type={norm_type} tied={tied}", flush=True)
    tensors = synth.build_tensors(gpu, cfg, seed=11)
    if norm_type == 1:
        tensors = _f16_round(tensors)
    path = tmp_path / "tiny.gguf"
    path.write_bytes(gguf_bytes(model_meta(cfg, arch), model_tensors(tensors, norm_type), alignment=alignment))

    B, T = 2, 40
    train = dict(lora_rank=cfg.lora_rank, lora_alpha=cfg.lora_alpha, lora_targets=cfg.lora_targets)
    pg = PeftModel.from_gguf(gpu, path, max_batch=B, max_seq=T, **train)
    for k in ("n_layers", "dim", "n_heads", "n_kv_heads", "head_dim", "ffn_dim", "vocab", "rope_neox", "attn_bias"):
        assert getattr(pg.cfg, k) == getattr(cfg, k), k
    assert pg.cfg.rms_eps == np.float32(cfg.rms_eps) and pg.cfg.rope_base == np.float32(cfg.rope_base)
    pd = PeftModel(gpu, cfg, max_batch=B, max_seq=T)
    pd.load(tensors)
    lora = synth.lora_init(cfg, seed=12, b_std=0.02)
    for (l, t), (A, Bm) in lora.items():
        pg.set_lora(l, t, A, Bm)
        pd.set_lora(l, t, A, Bm)
    ids, tg = synth.tokens(cfg, B, T, seed=13)
    assert pg.loss_grad(ids, tg) == pd.loss_grad(ids, tg)
    for (l, t) in lora:
        for a, b in zip(pg.get_lora_grad(l, t), pd.get_lora_grad(l, t)):
            np.testing.assert_array_equal(a, b)
    pg.close()
    pd.close()


def test_gguf_unsupported_quant_refused(gpu, tmp_path):
    from hos_amd import synth
    from hos_amd.hip_be import HosError
    from hos_amd.peft import PeftModel
    cfg = _tiny(n_layers=1)
    print("gguf unsupported quant", flush=True)
    tensors = model_tensors(synth.build_tensors(gpu, cfg, seed=3))
    raw, _, dims = tensors["blk.0.ffn_up.weight"]
    tensors["blk.0.ffn_up.weight"] = (np.zeros(dims[0] * dims[1] // 32 * 20, np.uint8), 3, dims)  # Q4_1
    path = tmp_path / "q41.gguf"
    path.write_bytes(gguf_bytes(model_meta(cfg, "qwen2"), tensors))
    with pytest.raises(HosError) as e:
        PeftModel.from_gguf(gpu, path, lora_rank=8, lora_targets=("q", "v"))
    assert e.value.code == 4


def test_gguf_mixed_encodings_match_oracle(gpu, tmp_path):
    """A GGUF file whose linear weights use every encoding the reference decodes (a Q4_K_M-style mix:
    Q4_0, Q5_0, Q5_K, Q6_K, Q8_0, Q4_K, F16, BF16, F32; F16 norms), loaded by the library, against the oracle
    loaded from the same bytes: loss and every LoRA gradient within 1e-3 relative L2,
    the loss also to 1e-5 relative."""
    import types

    from hos_amd import synth
    from hos_amd.peft import PeftModel
    from oracle import binding as o
    cfg = _tiny()
    print("gguf mixed encodings vs oracle", flush=True)
    enc = {0: {"attn_q": 2, "attn_k": 6, "attn_v": 13, "attn_output": 1, "ffn_gate": 30, "ffn_up": 12,
               "ffn_down": 14},
           1: {"attn_q": 13, "attn_k": 0, "attn_v": 8, "attn_output": 2, "ffn_gate": 6, "ffn_up": 1,
               "ffn_down": 13}}
    rng = np.random.default_rng(21)
    tensors = _f16_round(synth.build_tensors(gpu, cfg, seed=20, quantize=o.quantize))
    for name, (raw, t, rows, cols) in list(tensors.items()):
        parts = name.split(".")
        if len(parts) == 4 and parts[3] == "weight" and parts[2] in enc.get(int(parts[1]) if parts[0] == "blk" else -1, {}):
            t2 = enc[int(parts[1])][parts[2]]
            w = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
            if t2 == 0:
                raw2 = w.view(np.uint8).ravel()
            elif t2 == 30:
                raw2 = (w.view(np.uint32) >> 16).astype(np.uint16).view(np.uint8).ravel()
            else:
                raw2 = o.quantize(w, t2)
            tensors[name] = (raw2, t2, rows, cols)
    path = tmp_path / "mixed.gguf"
    path.write_bytes(gguf_bytes(model_meta(cfg, "qwen2"), model_tensors(tensors, norm_type=1)))
    B, T = 2, 32
    pg = PeftModel.from_gguf(gpu, path, max_batch=B, max_seq=T, lora_rank=cfg.lora_rank,
                             lora_alpha=cfg.lora_alpha, lora_targets=cfg.lora_targets)
    oc = types.SimpleNamespace(**{k: getattr(cfg, k) for k in (
        "n_layers", "dim", "n_heads", "n_kv_heads", "head_dim", "ffn_dim", "vocab", "rms_eps", "rope_base",
        "rope_neox", "attn_bias", "lora_rank", "lora_alpha")})
    oc.lora_targets = cfg.target_mask
    om = o.OracleModel(oc)
    for name, (raw, t, rows, cols) in tensors.items():
        om.set_tensor(name, raw, t, rows, cols)
    lora = synth.lora_init(cfg, seed=22, b_std=0.02)
    for (l, t), (A, Bm) in lora.items():
        pg.set_lora(l, t, A, Bm)
        om.set_lora(l, synth.ALL.index(t), A, Bm)
    ids, tg = synth.tokens(cfg, B, T, seed=23)
    loss, want = pg.loss_grad(ids, tg), om.loss_grad(ids, tg)
    assert abs(loss - want) <= 1e-5 * abs(want), (loss, want)
    worst = 0.0
    for (l, t) in lora:
        i, ou = cfg.target_dims(t)
        got = pg.get_lora_grad(l, t)
        ref = om.get_lora_grad(l, synth.ALL.index(t), ((i, cfg.lora_rank), (cfg.lora_rank, ou)))
        for a, b in zip(got, ref):
            worst = max(worst, float(np.linalg.norm(a - b) / np.linalg.norm(b)))
    print(f"worst LoRA grad rel L2 {worst:.2e}", flush=True)
    assert worst <= 1e-3
    pg.close()
