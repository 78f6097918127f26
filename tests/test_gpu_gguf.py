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
    tensors["blk.0.ffn_up.weight"] = (np.zeros(dims[0] * dims[1] // 32 * 18, np.uint8), 2, dims)  # Q4_0
    path = tmp_path / "q40.gguf"
    path.write_bytes(gguf_bytes(model_meta(cfg, "qwen2"), tensors))
    with pytest.raises(HosError) as e:
        PeftModel.from_gguf(gpu, path, lora_rank=8, lora_targets=("q", "v"))
    assert e.value.code == 4
