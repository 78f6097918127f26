"""Benchmark configurations and their synthetic frozen bases.

Weights are random-init ~N(0, 0.02) (norm weights 1.0, biases ~N(0, 0.02)) drawn with numpy's PCG64 from a
fixed seed and quantized on the device by the byte-exact port of HOS's own quantizers (src/gguf_write.rs).
Linear weights whose row length is not a multiple of the type's block (e.g. 896-wide rows for Q4_K's
256-element super-blocks) fall back to Q8_0, the per-tensor gate of src/model.rs:225-228 and
src/gguf_write.rs:103 applied the way GGUF converters do.
"""
import numpy as np

from .hip_be import BLOCK, GGML_F32, GGML_Q4_K, GGML_Q6_K, GGML_Q8_0
from .peft import ModelConfig

ALL = ("q", "k", "v", "o", "gate", "up", "down")

CONFIGS = {
    # SmolLM2-135M, Q8_0, LoRA r=8 on q/k/v/o, one step on 1 x 128
    "smollm2-135m": ModelConfig("smollm2-135m", n_layers=30, dim=576, n_heads=9, n_kv_heads=3, head_dim=64,
                                ffn_dim=1536, vocab=49152, rms_eps=1e-5, rope_base=10000.0, rope_neox=False,
                                lora_rank=8, lora_alpha=16.0, lora_targets=("q", "k", "v", "o"),
                                quant=GGML_Q8_0, head_quant=GGML_Q8_0, batch=1, seq=128, lr=1e-3),
    # Qwen2.5-0.5B, Q4_K (Q6_K head/embedding), LoRA r=16 on all 7, 4 x 512, AdamW lr 1e-4
    "qwen2.5-0.5b": ModelConfig("qwen2.5-0.5b", n_layers=24, dim=896, n_heads=14, n_kv_heads=2, head_dim=64,
                                ffn_dim=4864, vocab=151936, rms_eps=1e-6, rope_base=1e6, rope_neox=True,
                                attn_bias=True, lora_rank=16, lora_alpha=16.0, lora_targets=ALL,
                                quant=GGML_Q4_K, head_quant=GGML_Q6_K, batch=4, seq=512, lr=1e-4),
    # Llama-3.2-1B, Q4_K, LoRA r=32 on all 7, 8 x 1024
    "llama3.2-1b": ModelConfig("llama3.2-1b", n_layers=16, dim=2048, n_heads=32, n_kv_heads=8, head_dim=64,
                               ffn_dim=8192, vocab=128256, rms_eps=1e-5, rope_base=5e5, rope_neox=False,
                               lora_rank=32, lora_alpha=16.0, lora_targets=ALL, quant=GGML_Q4_K,
                               head_quant=GGML_Q4_K, batch=8, seq=1024, lr=1e-4),
    # OLMoE architecture, 64 experts top-8 (SwiGLU 1024) kept in Q8_0, QK-norm, head_dim 128,
    # LoRA r=16 on the attention projections, 4 x 512
    "olmoe": ModelConfig("olmoe", n_layers=16, dim=2048, n_heads=16, n_kv_heads=16, head_dim=128, ffn_dim=1024,
                         vocab=50304, rms_eps=1e-5, rope_base=10000.0, rope_neox=True, lora_rank=16,
                         lora_alpha=16.0, lora_targets=("q", "k", "v", "o"), quant=GGML_Q8_0,
                         head_quant=GGML_Q8_0, batch=4, seq=512, lr=1e-4, n_experts=64, n_experts_used=8,
                         qk_norm=True),
}


def storage_type(want, cols):
    """The type a [rows, cols] tensor is stored in: `want` if cols is block-aligned, else Q8_0."""
    return want if cols % BLOCK[want] == 0 else GGML_Q8_0


def tensor_list(cfg):
    """(name, rows, cols, kind) in GGUF naming (src/model.rs:713-921); kind: 'lin' | 'head' | 'norm' | 'bias'."""
    d, qd, kvd, f = cfg.dim, cfg.n_heads * cfg.head_dim, cfg.n_kv_heads * cfg.head_dim, cfg.ffn_dim
    out = [("token_embd.weight", cfg.vocab, d, "head")]
    if not cfg.tied:
        out.append(("output.weight", cfg.vocab, d, "head"))
    out.append(("output_norm.weight", 1, d, "norm"))
    E = cfg.n_experts
    for l in range(cfg.n_layers):
        p = f"blk.{l}."
        out += [(p + "attn_norm.weight", 1, d, "norm"), (p + "attn_q.weight", qd, d, "lin"),
                (p + "attn_k.weight", kvd, d, "lin"), (p + "attn_v.weight", kvd, d, "lin"),
                (p + "attn_output.weight", d, qd, "lin"), (p + "ffn_norm.weight", 1, d, "norm")]
        if E:  # MoE (src/model.rs:815-838): f32 router [E, d], stacked experts [E·rows, cols]
            out += [(p + "ffn_gate_inp.weight", E, d, "router"), (p + "ffn_gate_exps.weight", E * f, d, "lin"),
                    (p + "ffn_up_exps.weight", E * f, d, "lin"), (p + "ffn_down_exps.weight", E * d, f, "lin")]
        else:
            out += [(p + "ffn_gate.weight", f, d, "lin"), (p + "ffn_up.weight", f, d, "lin"),
                    (p + "ffn_down.weight", d, f, "lin")]
        if cfg.qk_norm:
            out += [(p + "attn_q_norm.weight", 1, qd, "norm"), (p + "attn_k_norm.weight", 1, kvd, "norm")]
        if cfg.attn_bias:
            out += [(p + "attn_q.bias", 1, qd, "bias"), (p + "attn_k.bias", 1, kvd, "bias"),
                    (p + "attn_v.bias", 1, kvd, "bias")]
    return out


def build_tensors(gpu, cfg, seed=1234, quantize=None, norm_jitter=0.0):
    """name -> (raw bytes, ggml_type, rows, cols), quantized on the device (or with `quantize(w, type)`).
    Norm weights are 1.0 (+ U(-norm_jitter, norm_jitter)); the MoE router is f32 ~N(0, 0.02) like the other
    weights (cfg.extra["router_std"] overrides)."""
    device = quantize is None
    quantize = quantize or gpu.quantize
    rng = np.random.default_rng(seed)
    tensors = {}
    for idx, (name, rows, cols, kind) in enumerate(tensor_list(cfg)):
        if device and "_exps" in name:
            # MoE expert stacks (billions of values at OLMoE size): drawn and quantized on the device
            t = storage_type(cfg.quant, cols)
            tensors[name] = (gpu.random_quantized(rows, cols, t, seed=seed * 4096 + idx), t, rows, cols)
            continue
        if kind == "norm":
            v = np.ones(cols, np.float32)
            if norm_jitter:
                v += rng.uniform(-norm_jitter, norm_jitter, cols).astype(np.float32)
            tensors[name] = (v.view(np.uint8), GGML_F32, 1, cols)
            continue
        std = np.float32(cfg.extra.get("router_std", 0.02) if kind == "router" else 0.02)
        w = (rng.standard_normal((rows, cols), dtype=np.float32) * std).astype(np.float32)
        if kind in ("bias", "router"):
            tensors[name] = (w.ravel().view(np.uint8), GGML_F32, rows, cols)
            continue
        t = storage_type(cfg.head_quant if kind == "head" else cfg.quant, cols)
        tensors[name] = (quantize(w, t), t, rows, cols)
    return tensors


def lora_init(cfg, seed=99, b_std=0.0):
    """LoRA factors per (layer, target): A ~ N(0, 0.02), B = 0 (or ~N(0, b_std) for gradient checks)."""
    rng = np.random.default_rng(seed)
    out = {}
    for l in range(cfg.n_layers):
        for t in cfg.lora_targets:
            i, o = cfg.target_dims(t)
            A = (rng.standard_normal((i, cfg.lora_rank), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
            B = (rng.standard_normal((cfg.lora_rank, o), dtype=np.float32) * np.float32(b_std)).astype(np.float32)
            out[(l, t)] = (A, B)
    return out


def rga_init(cfg, seed=99, std=0.02, up_std=0.0):
    """RGA parameters by adapter tensor name: genome, wg, wr and the gene downs ~N(0, std), ups = 0 as the
    reference initializes them (src/peft.rs:200-215), or ~N(0, up_std) for gradient checks."""
    rng = np.random.default_rng(seed)
    out = {}
    for name, shape in cfg.rga_shapes().items():
        s = up_std if ".up." in name else std
        out[name] = (rng.standard_normal(shape, dtype=np.float32) * np.float32(s)).astype(np.float32)
    return out


def tokens(cfg, batch, seq, seed=7):
    """Uniform token ids over the vocab; targets are the next-token shift."""
    rng = np.random.default_rng(seed)
    w = rng.integers(0, cfg.vocab, size=(batch, seq + 1), dtype=np.int64).astype(np.int32)
    return np.ascontiguousarray(w[:, :seq]), np.ascontiguousarray(w[:, 1:])


def algorithmic_flops_per_token(cfg, seq):
    """F_tok = 4·P_base + 6·P_lora + 6·L·T·q_dim, causal attention counted once (the reference's
    baseline formula)."""
    d, qd, kvd, f, v = cfg.dim, cfg.n_heads * cfg.head_dim, cfg.n_kv_heads * cfg.head_dim, cfg.ffn_dim, cfg.vocab
    # a mixture of experts counts the active parameters: the K routed experts and the router
    ffn = (cfg.n_experts_used * 3 * d * f + d * cfg.n_experts) if cfg.n_experts else 3 * d * f
    p_base = cfg.n_layers * (d * qd + 2 * d * kvd + qd * d + ffn) + d * v
    p_lora = cfg.n_layers * sum(cfg.lora_rank * sum(cfg.target_dims(t)) for t in cfg.lora_targets)
    if cfg.rga_genes:  # RGA: gate weights + each gene's down and up per layer (the genome terms are per step)
        p_lora += cfg.n_layers * cfg.rga_genes * d * (1 + 2 * cfg.rga_bottleneck)
    return 4 * p_base + 6 * p_lora + 6 * cfg.n_layers * seq * qd
