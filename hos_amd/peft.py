"""Host-side mirror of HOS's LoRA training API (src/peft.rs PeftModel, src/tensor.rs AdamW) over the C ABI.

``PeftModel.loss_grad(ids, targets)`` is one optimizer step's gradient (zero_grad, then B sequences with
``loss·(1/B)`` backward, src/main.rs:2583-2596); ``adamw(lr, wd)`` is ``AdamW::step``; ``step`` does both.
The model lives on one device; the host only enqueues.
"""
import ctypes
import json
from dataclasses import dataclass, field

import numpy as np

from ._lib import PeftCfg, lib
from .hip_be import Gpu, HosError

TARGETS = ("q", "k", "v", "o", "gate", "up", "down")
TARGET_BITS = {t: 1 << i for i, t in enumerate(TARGETS)}


@dataclass
class ModelConfig:
    """src/model.rs:622-644 (Config) + src/peft.rs:121-126 (PeftCfg) + the batch shape."""
    name: str
    n_layers: int
    dim: int
    n_heads: int
    n_kv_heads: int
    head_dim: int
    ffn_dim: int
    vocab: int
    rms_eps: float = 1e-5
    rope_base: float = 10000.0
    rope_neox: bool = False
    attn_bias: bool = False
    tied: bool = True
    lora_rank: int = 8
    lora_alpha: float = 16.0
    lora_targets: tuple = ("q", "v")
    quant: int = 8            # GGUF type of the linear weights
    head_quant: int = 8       # GGUF type of token_embd / output
    batch: int = 1
    seq: int = 128
    lr: float = 1e-3
    gemm_passes: int = 0      # qGEMM precision passes (0 = library default)
    n_experts: int = 0        # mixture-of-experts FFN (0 = dense), src/model.rs:642-643
    n_experts_used: int = 0
    qk_norm: bool = False     # OLMoE RMSNorm of the q / k projections before RoPE
    # RGA adapters instead of LoRA (src/peft.rs:61-96): genes per layer, gene bottleneck, gate sparsity weight
    rga_genes: int = 0
    rga_bottleneck: int = 4
    rga_lambda: float = 1e-3
    extra: dict = field(default_factory=dict)

    @property
    def is_rga(self):
        return self.rga_genes > 0

    def rga_shapes(self):
        """Adapter tensor name -> shape, in PeftModel::params order (src/peft.rs:283-311; genome last)."""
        k, b, d = self.rga_genes, self.rga_bottleneck, self.dim
        out = {"wg": (8, k)}
        for l in range(self.n_layers):
            out[f"rga.{l}.wr"] = (d, k)
            for kk in range(k):
                out[f"rga.{l}.down.{kk}"] = (d, b)
            for kk in range(k):
                out[f"rga.{l}.up.{kk}"] = (b, d)
        out["genome.0"] = (1, 8)
        return out

    @property
    def target_mask(self):
        m = 0
        for t in self.lora_targets:
            m |= TARGET_BITS[t]
        return m

    def target_dims(self, t):
        """(in, out) of the projection adapted by target t."""
        d, qd, kvd, f = self.dim, self.n_heads * self.head_dim, self.n_kv_heads * self.head_dim, self.ffn_dim
        return {"q": (d, qd), "k": (d, kvd), "v": (d, kvd), "o": (qd, d), "gate": (d, f), "up": (d, f),
                "down": (f, d)}[t]


def _cstruct(cfg, max_batch=None, max_seq=None):
    return PeftCfg(cfg.n_layers, cfg.dim, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim, cfg.ffn_dim, cfg.vocab,
                   cfg.rms_eps, cfg.rope_base, int(cfg.rope_neox), int(cfg.attn_bias), cfg.lora_rank,
                   cfg.lora_alpha, cfg.target_mask, max_batch or cfg.batch, max_seq or cfg.seq, cfg.gemm_passes,
                   cfg.n_experts, cfg.n_experts_used, int(cfg.qk_norm), cfg.rga_genes, cfg.rga_bottleneck,
                   cfg.rga_lambda)


def _from_cstruct(c, name, **train):
    return ModelConfig(name=name, n_layers=c.n_layers, dim=c.dim, n_heads=c.n_heads, n_kv_heads=c.n_kv_heads,
                       head_dim=c.head_dim, ffn_dim=c.ffn_dim, vocab=c.vocab, rms_eps=c.rms_eps,
                       rope_base=c.rope_base, rope_neox=bool(c.rope_neox), attn_bias=bool(c.attn_bias),
                       n_experts=c.n_experts, n_experts_used=c.n_experts_used, qk_norm=bool(c.qk_norm), **train)


def gguf_config(path, **train):
    """The model config a GGUF file declares (Model::load's metadata mapping, src/model.rs:713-771),
    parsed by the library (no device work). ``train`` sets the ModelConfig training fields."""
    tmp = ModelConfig(name="gguf", n_layers=0, dim=0, n_heads=0, n_kv_heads=0, head_dim=0, ffn_dim=0, vocab=0,
                      **train)
    c = _cstruct(tmp)
    err = ctypes.create_string_buffer(512)
    rc = lib().hos_gguf_config(str(path).encode(), ctypes.byref(c), err, len(err))
    if rc:
        raise HosError(rc, err.value.decode())
    return _from_cstruct(c, str(path), **train)


class PeftModel:
    def __init__(self, gpu: Gpu, cfg: ModelConfig, max_batch=None, max_seq=None, _handle=None):
        self.gpu, self.cfg = gpu, cfg
        if _handle is not None:
            self.h = _handle
            gpu.adopt(self)
            return
        c = _cstruct(cfg, max_batch, max_seq)
        h = ctypes.c_void_p()
        rc = lib().hos_peft_create(gpu.h, ctypes.byref(c), ctypes.byref(h))
        if rc:
            raise HosError(rc, "hos_peft_create failed (see stderr)")
        self.h = h
        gpu.adopt(self)

    @classmethod
    def from_gguf(cls, gpu: Gpu, path, max_batch=1, max_seq=128, **train):
        """Load a GGUF base model (Model::load, src/model.rs:713-921) and wrap it with LoRA adapters as
        ``train`` (lora_rank, lora_alpha, lora_targets, gemm_passes, lr, ...) describes."""
        tmp = ModelConfig(name="gguf", n_layers=0, dim=0, n_heads=0, n_kv_heads=0, head_dim=0, ffn_dim=0,
                          vocab=0, batch=max_batch, seq=max_seq, **train)
        c, out = _cstruct(tmp), PeftCfg()
        h = ctypes.c_void_p()
        rc = lib().hos_peft_create_from_gguf(gpu.h, str(path).encode(), ctypes.byref(c), ctypes.byref(h),
                                             ctypes.byref(out))
        if rc:
            raise HosError(rc, f"hos_peft_create_from_gguf({path}) failed (see stderr)")
        return cls(gpu, _from_cstruct(out, str(path), batch=max_batch, seq=max_seq, **train), _handle=h)

    def close(self):
        if getattr(self, "h", None):
            lib().hos_peft_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def _chk(self, rc):
        if rc:
            raise HosError(rc, lib().hos_peft_last_error(self.h).decode())

    def set_tensor(self, name, raw, ggml_type, rows, cols):
        raw = np.ascontiguousarray(raw).view(np.uint8).ravel()
        self._chk(lib().hos_peft_set_tensor(self.h, name.encode(), raw.ctypes.data, raw.size, ggml_type, rows, cols))

    def load(self, tensors):
        for name, (raw, t, rows, cols) in tensors.items():
            self.set_tensor(name, raw, t, rows, cols)

    def set_lora(self, layer, target, A, B):
        ti = TARGETS.index(target) if isinstance(target, str) else target
        A = np.ascontiguousarray(A, np.float32)
        B = np.ascontiguousarray(B, np.float32)
        self._chk(lib().hos_peft_set_lora(self.h, layer, ti, A.ctypes.data, B.ctypes.data))

    def _pair(self, fn, layer, target):
        t = TARGETS[target] if isinstance(target, int) else target
        i, o = self.cfg.target_dims(t)
        A = np.empty((i, self.cfg.lora_rank), np.float32)
        B = np.empty((self.cfg.lora_rank, o), np.float32)
        self._chk(fn(self.h, layer, TARGETS.index(t), A.ctypes.data, B.ctypes.data))
        return A, B

    def get_lora(self, layer, target):
        return self._pair(lib().hos_peft_get_lora, layer, target)

    def get_lora_grad(self, layer, target):
        return self._pair(lib().hos_peft_get_lora_grad, layer, target)

    def set_rga(self, name, value):
        """An RGA parameter by its adapter tensor name (genome.0, wg, rga.{l}.wr / down.{k} / up.{k}),
        reference layout (PeftModel::adapter_tensors, src/peft.rs:741-760)."""
        v = np.ascontiguousarray(value, np.float32)
        self._chk(lib().hos_peft_set_adapter(self.h, name.encode(), v.ctypes.data, v.size))

    def get_rga(self, name):
        """(value, gradient) of an RGA parameter, reference layout."""
        shape = self.cfg.rga_shapes()[name]
        v = np.empty(shape, np.float32)
        g = np.empty(shape, np.float32)
        self._chk(lib().hos_peft_get_adapter(self.h, name.encode(), v.ctypes.data, g.ctypes.data, v.size))
        return v, g

    def loss_grad(self, ids, targets):
        ids = np.ascontiguousarray(ids, np.int32)
        tg = np.ascontiguousarray(targets, np.int32)
        B, T = ids.shape
        loss = ctypes.c_float()
        self._chk(lib().hos_peft_loss_grad(self.h, ids.ctypes.data, tg.ctypes.data, B, T, ctypes.byref(loss)))
        return loss.value

    def adamw(self, lr, wd=0.0):
        self._chk(lib().hos_peft_adamw(self.h, lr, wd))

    def step(self, ids, targets, lr, wd=0.0):
        loss = self.loss_grad(ids, targets)
        self.adamw(lr, wd)
        return loss

    def step_dev(self, ids_dev, tgt_dev, B, T, lr, wd=0.0, loss_dev=None):
        self._chk(lib().hos_peft_step_dev(self.h, ids_dev, tgt_dev, B, T, lr, wd, loss_dev))

    def use_graph(self, on):
        """Replay a captured graph of the whole step in step_dev (default on)."""
        self._chk(lib().hos_peft_use_graph(self.h, int(on)))

    def logits(self, ids):
        ids = np.ascontiguousarray(ids, np.int32).ravel()
        out = np.empty((ids.size, self.cfg.vocab), np.float32)
        self._chk(lib().hos_peft_logits(self.h, ids.ctypes.data, ids.size, out.ctypes.data))
        return out

    def profile(self, on, only=None):
        """Time kernel classes with HIP events (`only`: restrict to one class)."""
        self._chk(lib().hos_peft_profile_only(self.h, (only or "").encode()))
        self._chk(lib().hos_peft_profile(self.h, int(on)))

    def kernel_stats(self, cls):
        n = ctypes.c_longlong()
        ms, fl, by = ctypes.c_double(), ctypes.c_double(), ctypes.c_double()
        self._chk(lib().hos_peft_kernel_stats(self.h, cls.encode(), ctypes.byref(n), ctypes.byref(ms),
                                              ctypes.byref(fl), ctypes.byref(by)))
        return {"launches": n.value, "ms": ms.value, "flops": fl.value, "bytes": by.value}

    # ---------------- checkpoints (.hos capsule) ----------------
    def adapter_id(self):
        """model_id of the adapter tensors (src/format.rs:100-111)."""
        buf = ctypes.create_string_buffer(17)
        self._chk(lib().hos_peft_adapter_id(self.h, buf))
        return buf.value.decode()

    def base_id(self):
        """The base model's id as save_adapter records it (src/main.rs:2641-2646)."""
        buf = ctypes.create_string_buffer(17)
        self._chk(lib().hos_peft_base_id(self.h, buf))
        return buf.value.decode()

    def adapter_card(self, name, base_path="", end_loss=0.0, steps=0, lr=0.0, method="lora",
                     base_arch="Llama"):
        """The card save_adapter writes (src/main.rs:2614-2688), as JSON text with serde's field order."""
        f32 = lambda x: float(str(np.float32(x)))  # noqa: E731  shortest f32 digits
        base = self.base_id()
        card = {
            "format": "hos", "spec": 1, "name": name, "id": self.adapter_id(), "mode": "adapter",
            "arch": {"base_architecture": base_arch, "block_count": self.cfg.n_layers, "method": method,
                     "source_format": "hos-peft"},
            "provenance": {"created": "", "engine": "hos-peft", "dataset": f"{method} adapter on {base_path}",
                           "dataset_hash": base},
            "resume": {"seed": 0, "step": 0, "rng_state": 0},
            "history": [{"steps": int(steps), "final_loss": f32(end_loss), "optimizer": "adamw", "lr": f32(lr)}],
            "lineage": [base],
        }
        return json.dumps(card, separators=(",", ":"))

    def save_hos(self, path, card=None, optimizer=True):
        """Write the adapters (and AdamW state) as a .hos capsule; card: JSON text or dict (None = default)."""
        if isinstance(card, dict):
            card = json.dumps(card, separators=(",", ":"))
        self._chk(lib().hos_peft_save_hos(self.h, str(path).encode(), card.encode() if card else None,
                                          int(optimizer)))

    def load_hos(self, path, optimizer=True):
        """Restore adapters (and AdamW state) from a .hos capsule."""
        self._chk(lib().hos_peft_load_hos(self.h, str(path).encode(), int(optimizer)))


def read_card(path):
    """The card of a .hos file as a dict (read_card, src/format.rs:270-285)."""
    need = ctypes.c_size_t()
    buf = ctypes.create_string_buffer(4096)
    rc = lib().hos_format_card(str(path).encode(), buf, len(buf), ctypes.byref(need))
    if rc:
        raise HosError(rc, buf.value.decode(errors="replace"))
    if need.value > len(buf):
        buf = ctypes.create_string_buffer(need.value)
        rc = lib().hos_format_card(str(path).encode(), buf, len(buf), ctypes.byref(need))
        if rc:
            raise HosError(rc, buf.value.decode(errors="replace"))
    return json.loads(buf.value.decode())
