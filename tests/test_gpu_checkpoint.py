"""Adapter / optimizer checkpoints in the .hos layout (hos_peft_save_hos / hos_peft_load_hos), checked
with the oracle's reader and writer (oracle/hos_format.py, src/format.rs).

* what is written: tensor names / order / roles / shapes of PeftModel::adapter_tensors (q|v model:
  lora.{l}.{aq,bq,av,bv}, src/peft.rs:731-740), bit-exact factors, the optimizer tensors and scalars of
  src/main.rs:6276-6307, valid per-tensor and file checksums, a card whose id is model_id of the adapter;
* resume: train, save, load into a fresh model, continue -> bit-identical to continuing the original
  (the reload / resume check of src/main.rs:6330-6370);
* files the oracle writes (v1 and v2) load; bad files are refused with the right status and leave the
  model unchanged.
"""
import json

import numpy as np
import pytest

from oracle import binding as o
from oracle import hos_format as hf

pytestmark = pytest.mark.gpu

TARGETS = ("q", "k", "v", "o", "gate", "up", "down")


@pytest.fixture(scope="module")
def gpu():
    from hos_amd import Gpu
    g = Gpu(0)
    yield g
    g.close()


def _cfg(**kw):
    from hos_amd.peft import ModelConfig
    base = dict(name="tiny", n_layers=2, dim=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn_dim=512, vocab=512,
                rms_eps=1e-6, rope_base=1e6, rope_neox=True, attn_bias=True, lora_rank=8, lora_alpha=16.0,
                lora_targets=TARGETS, quant=8, head_quant=8, gemm_passes=3)
    base.update(kw)
    return ModelConfig(**base)


def _model(gpu, cfg, tensors, B=2, T=32, lora_seed=4):
    from hos_amd import synth
    from hos_amd.peft import PeftModel
    pm = PeftModel(gpu, cfg, max_batch=B, max_seq=T)
    pm.load(tensors)
    if lora_seed is not None:
        for (l, t), (A, Bm) in synth.lora_init(cfg, seed=lora_seed, b_std=0.02).items():
            pm.set_lora(l, t, A, Bm)
    return pm


def _factors(pm, cfg):
    return {(l, t): pm.get_lora(l, t) for l in range(cfg.n_layers) for t in cfg.lora_targets}


def test_written_capsule(gpu, tmp_path):
    from hos_amd import synth
    cfg = _cfg(lora_targets=("q", "v"))
    print("checkpoint written capsule q|v", flush=True)
    tensors = synth.build_tensors(gpu, cfg, seed=1)
    pm = _model(gpu, cfg, tensors)
    ids, tg = synth.tokens(cfg, 2, 32, seed=2)
    for _ in range(2):
        pm.step(ids, tg, 1e-3, 0.01)
    path = tmp_path / "a.hos"
    pm.save_hos(path, optimizer=True)
    ver, card, out, file_ok = hf.read(path.read_bytes())
    assert ver == 2 and file_ok
    names = [x[0] for x in out]
    want = [f"lora.{l}.{n}" for l in range(cfg.n_layers) for n in ("aq", "bq", "av", "bv")]
    nparam = len(want)
    want += [f"opt.{mv}.{k}" for k in range(nparam) for mv in ("m", "v")]
    want += ["opt.step", "opt.lr", "opt.beta1", "opt.beta2", "opt.wd"]
    assert names == want
    by = {x[0]: x for x in out}
    adapter = []
    for l in range(cfg.n_layers):
        for t in ("q", "v"):
            A, Bm = pm.get_lora(l, t)
            for nm, arr in ((f"lora.{l}.a{t}", A), (f"lora.{l}.b{t}", Bm)):
                _, role, dtype, shape, nf, raw = by[nm]
                assert (role, dtype, shape, nf) == (hf.ROLE_WEIGHT, hf.DTYPE_F32, list(arr.shape), arr.size)
                assert raw == np.ascontiguousarray(arr, "<f4").tobytes()
                adapter.append((nm, role, shape, arr))
    for k in range(nparam):
        for mv in ("m", "v"):
            _, role, _, shape, nf, raw = by[f"opt.{mv}.{k}"]
            assert role == hf.ROLE_OPT_STATE and shape == [nf] and nf == adapter[k][3].size
            assert np.isfinite(np.frombuffer(raw, "<f4")).all()
        assert np.frombuffer(by[f"opt.v.{k}"][5], "<f4").min() >= 0
    sc = {n: np.frombuffer(by[n][5], "<f4")[0] for n in ("opt.step", "opt.lr", "opt.beta1", "opt.beta2", "opt.wd")}
    assert sc == {"opt.step": 2.0, "opt.lr": np.float32(1e-3), "opt.beta1": np.float32(0.9),
                  "opt.beta2": np.float32(0.95), "opt.wd": np.float32(0.01)}
    assert all(by[n][1] == hf.ROLE_SCALAR and by[n][3] == [1] for n in sc)
    c = json.loads(card)
    assert c["format"] == "hos" and c["mode"] == "adapter" and c["resume"]["step"] == 2
    assert c["id"] == hf.model_id(adapter) == pm.adapter_id()
    # base id: FNV-1a over the dequantized f32 token embedding (src/main.rs:2641-2646)
    raw, t, rows, cols = tensors["token_embd.weight"]
    emb = o.dequant(raw, t, rows * cols)
    assert pm.base_id() == f"{hf.fnv1a64(np.ascontiguousarray(emb, '<f4').tobytes()):016x}"
    # save_adapter's card, passed through verbatim
    card2 = pm.adapter_card("tiny-lora", "tiny.gguf", end_loss=1.5, steps=2, lr=1e-3)
    pm.save_hos(tmp_path / "b.hos", card=card2, optimizer=False)
    _, text, out2, ok2 = hf.read((tmp_path / "b.hos").read_bytes())
    assert ok2 and text == card2 and [x[0] for x in out2] == want[:nparam]
    from hos_amd.peft import read_card
    c2 = read_card(tmp_path / "b.hos")
    assert c2["lineage"] == [pm.base_id()] == [c2["provenance"]["dataset_hash"]]
    assert c2["history"][0]["lr"] == 0.001 and c2["id"] == c["id"]
    pm.close()


def test_resume_is_bit_identical(gpu, tmp_path):
    from hos_amd import synth
    cfg = _cfg()
    print("checkpoint resume all targets", flush=True)
    tensors = synth.build_tensors(gpu, cfg, seed=5)
    a = _model(gpu, cfg, tensors)
    batches = [synth.tokens(cfg, 2, 32, seed=10 + i) for i in range(3)]
    for ids, tg in batches[:2]:
        a.step(ids, tg, 2e-3, 0.0)
    path = tmp_path / "r.hos"
    a.save_hos(path, optimizer=True)
    b = _model(gpu, cfg, tensors, lora_seed=77)  # different factors; overwritten by the load
    b.load_hos(path, optimizer=True)
    fa, fb = _factors(a, cfg), _factors(b, cfg)
    for k in fa:
        for x, y in zip(fa[k], fb[k]):
            np.testing.assert_array_equal(x, y)
    c = _model(gpu, cfg, tensors, lora_seed=77)
    c.load_hos(path, optimizer=False)  # factors only: fresh AdamW
    ids, tg = batches[2]
    la, lb, lc = a.step(ids, tg, 2e-3, 0.0), b.step(ids, tg, 2e-3, 0.0), c.step(ids, tg, 2e-3, 0.0)
    assert la == lb == lc  # same factors before the step -> same loss
    fa, fb, fc = _factors(a, cfg), _factors(b, cfg), _factors(c, cfg)
    diff_c = 0
    for k in fa:
        for x, y, z in zip(fa[k], fb[k], fc[k]):
            np.testing.assert_array_equal(x, y)
            diff_c += int(not np.array_equal(x, z))
    assert diff_c > 0  # without the moments and step count the update differs
    for m in (a, b, c):
        m.close()


def _oracle_adapter(cfg, seed, names=None):
    rng = np.random.default_rng(seed)
    out = []
    for l in range(cfg.n_layers):
        for t in cfg.lora_targets:
            i, ou = cfg.target_dims(t)
            for ab, shape in (("a", [i, cfg.lora_rank]), ("b", [cfg.lora_rank, ou])):
                out.append((f"lora.{l}.{ab}{t}", hf.ROLE_WEIGHT, shape,
                            rng.standard_normal(shape).astype(np.float32)))
    return out


@pytest.mark.parametrize("version", [1, 2])
def test_loads_oracle_written(gpu, tmp_path, version):
    from hos_amd import synth
    cfg = _cfg(lora_targets=("q", "v", "down"), n_layers=1)
    print(f"checkpoint load oracle v{version}", flush=True)
    tensors = synth.build_tensors(gpu, cfg, seed=6)
    pm = _model(gpu, cfg, tensors)
    ad = _oracle_adapter(cfg, seed=version)
    extra = [("grow.0.gate", hf.ROLE_WEIGHT, [3], np.ones(3, np.float32))]  # unknown tensors are ignored
    path = tmp_path / "o.hos"
    path.write_bytes(hf.write(extra + ad[::-1], '{"format":"hos"}', version=version))
    pm.load_hos(path, optimizer=False)
    by = {n: d for n, _, _, d in ad}
    for t in cfg.lora_targets:
        A, Bm = pm.get_lora(0, t)
        np.testing.assert_array_equal(A, by[f"lora.0.a{t}"])
        np.testing.assert_array_equal(Bm, by[f"lora.0.b{t}"])
    pm.close()


def test_bad_files_refused(gpu, tmp_path):
    from hos_amd import synth
    from hos_amd.hip_be import HosError
    cfg = _cfg(lora_targets=("q", "v"), n_layers=1)
    print("checkpoint bad files", flush=True)
    tensors = synth.build_tensors(gpu, cfg, seed=7)
    pm = _model(gpu, cfg, tensors)
    before = _factors(pm, cfg)
    ad = _oracle_adapter(cfg, seed=3)
    cases = {
        "missing": (hf.write(ad[:-1], "{}"), 3),
        "shape": (hf.write([(n, r, s[::-1], d) if n.endswith("aq") else (n, r, s, d) for n, r, s, d in ad], "{}"), 2),
        "quant": (hf.write(ad, "{}", stored={ad[0][0]: (hf.DTYPE_Q8_0, b"\0" * 34)}), 4),
        "magic": (b"not a hos file at all", 2),
        "no_opt": (hf.write(ad, "{}"), 3),  # load with optimizer=True but no opt.* tensors
    }
    good = bytearray(hf.write(ad, "{}"))
    good[len(good) // 2] ^= 0xFF
    cases["corrupt"] = (bytes(good), 2)
    for name, (data, code) in cases.items():
        p = tmp_path / f"{name}.hos"
        p.write_bytes(data)
        with pytest.raises(HosError) as e:
            pm.load_hos(p, optimizer=(name == "no_opt"))
        assert e.value.code == code, name
    after = _factors(pm, cfg)
    for k in before:
        for x, y in zip(before[k], after[k]):
            np.testing.assert_array_equal(x, y)
    pm.close()
