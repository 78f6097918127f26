"""GGUF reader + Model::load config mapping of the C-ABI library (hos_gguf_config), on the CPU.

Covers src/gguf.rs:225-286 (header, typed metadata incl. arrays, tensor infos, alignment, error on
bad magic / version / truncation) and src/model.rs:713-771 (metadata -> config, defaults, head_dim
fallbacks, vocab from token_embd, QKV-bias detection, NEOX RoPE for qwen2), plus the robustness cases
of tests/fuzz_gguf.rs (random bytes, GGUF magic + garbage, truncated and byte-flipped files must return
an error, never crash). No device work: the config call parses only.
"""
import os
import struct

import numpy as np
import pytest

from gguf_writer import ARR, F32, F64, STR, U32, U64, I32, gguf_bytes, model_meta

LIB = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "hos_amd", "libhos_hip.so")
pytestmark = pytest.mark.skipif(not os.path.exists(LIB), reason="libhos_hip.so not built")

HOS_E_IO, HOS_E_FORMAT, HOS_E_MISSING_TENSOR, HOS_E_UNSUPPORTED_ARCH, HOS_E_MISSING_META = 1, 2, 3, 5, 6


class Cfg:
    n_layers, dim, n_heads, n_kv_heads, head_dim, ffn_dim = 2, 128, 4, 2, 32, 256
    rms_eps, rope_base, vocab = 1e-6, 1e6, 96


def _tensors(cfg, bias=True, output=False, embd=True):
    t = {}
    if embd:
        t["token_embd.weight"] = (np.zeros(cfg.vocab * cfg.dim // 32 * 34, np.uint8), 8, [cfg.dim, cfg.vocab])
    if output:
        t["output.weight"] = (np.zeros(cfg.vocab * cfg.dim // 32 * 34, np.uint8), 8, [cfg.dim, cfg.vocab])
    t["output_norm.weight"] = (np.ones(cfg.dim, np.float32), 0, [cfg.dim])
    if bias:
        t["blk.0.attn_q.bias"] = (np.zeros(cfg.n_heads * cfg.head_dim, np.float32), 0, [cfg.n_heads * cfg.head_dim])
    return t


def _write(tmp_path, data, name="m.gguf"):
    p = tmp_path / name
    p.write_bytes(data)
    return p


def _config(path):
    from hos_amd._lib import PeftCfg, lib
    import ctypes
    c = PeftCfg()
    c.lora_rank, c.max_batch = 7, 3
    err = ctypes.create_string_buffer(256)
    rc = lib().hos_gguf_config(str(path).encode(), ctypes.byref(c), err, len(err))
    return rc, c, err.value.decode()


def test_qwen2_mapping(tmp_path):
    cfg = Cfg()
    p = _write(tmp_path, gguf_bytes(model_meta(cfg, "qwen2"), _tensors(cfg)))
    rc, c, err = _config(p)
    assert rc == 0, err
    assert (c.n_layers, c.dim, c.n_heads, c.n_kv_heads, c.head_dim, c.ffn_dim, c.vocab) == (2, 128, 4, 2, 32, 256, 96)
    assert c.rms_eps == np.float32(1e-6) and c.rope_base == np.float32(1e6)
    assert c.rope_neox == 1 and c.attn_bias == 1
    assert (c.lora_rank, c.max_batch) == (7, 3)  # training fields pass through


def test_llama_defaults(tmp_path):
    """head_count_kv absent -> n_heads; eps -> 1e-5; freq_base -> 10000; head_dim -> dim / n_heads
    (src/model.rs:733-765); no attn_q.bias -> no bias; llama keeps interleaved RoPE."""
    cfg = Cfg()
    meta = model_meta(cfg, "llama", omit=("{arch}.attention.head_count_kv", "{arch}.attention.layer_norm_rms_epsilon",
                                          "{arch}.rope.freq_base", "{arch}.attention.key_length"))
    p = _write(tmp_path, gguf_bytes(meta, _tensors(cfg, bias=False)))
    rc, c, err = _config(p)
    assert rc == 0, err
    assert c.n_kv_heads == 4 and c.head_dim == 32 and c.rms_eps == np.float32(1e-5) and c.rope_base == 10000.0
    assert c.rope_neox == 0 and c.attn_bias == 0


def test_head_dim_from_rope_dimension_count(tmp_path):
    cfg = Cfg()
    meta = model_meta(cfg, "llama", omit=("{arch}.attention.key_length",),
                      extra={"llama.rope.dimension_count": (U32, 48)})
    rc, c, err = _config(_write(tmp_path, gguf_bytes(meta, _tensors(cfg))))
    assert rc == 0, err
    assert c.head_dim == 48


def test_general_architecture_defaults_to_llama(tmp_path):
    cfg = Cfg()
    meta = model_meta(cfg, "llama", omit=("general.architecture",))
    rc, c, err = _config(_write(tmp_path, gguf_bytes(meta, _tensors(cfg))))
    assert rc == 0, err
    assert c.dim == 128


def test_value_widths(tmp_path):
    """Integer keys as U64 / I32 and float keys as F64 are read like their narrower forms."""
    cfg = Cfg()
    meta = model_meta(cfg, "qwen2", extra={
        "qwen2.block_count": (U64, 5), "qwen2.feed_forward_length": (I32, 384),
        "qwen2.attention.layer_norm_rms_epsilon": (F64, 1e-5), "qwen2.rope.freq_base": (U32, 500000),
        "general.nested": (ARR, (ARR, [(U32, [1, 2]), (U32, [])])),
    })
    rc, c, err = _config(_write(tmp_path, gguf_bytes(meta, _tensors(cfg))))
    assert rc == 0, err
    assert c.n_layers == 5 and c.ffn_dim == 384 and c.rms_eps == np.float32(1e-5) and c.rope_base == 500000.0


@pytest.mark.parametrize("alignment", [32, 64, 256])
def test_alignment_and_version2(tmp_path, alignment):
    cfg = Cfg()
    meta = model_meta(cfg, "qwen2", extra={"general.alignment": (U32, alignment)})
    rc, c, err = _config(_write(tmp_path, gguf_bytes(meta, _tensors(cfg), alignment=alignment, version=2)))
    assert rc == 0, err


def test_errors(tmp_path):
    cfg = Cfg()
    good = gguf_bytes(model_meta(cfg, "qwen2"), _tensors(cfg))
    assert _config(tmp_path / "absent.gguf")[0] == HOS_E_IO
    assert _config(_write(tmp_path, b"GGML" + good[4:], "magic.gguf"))[0] == HOS_E_FORMAT
    assert _config(_write(tmp_path, good[:4] + struct.pack("<I", 1) + good[8:], "v1.gguf"))[0] == HOS_E_FORMAT
    assert _config(_write(tmp_path, good[:40], "trunc.gguf"))[0] == HOS_E_FORMAT
    meta = model_meta(cfg, "qwen2", omit=("{arch}.embedding_length",))
    rc, _, err = _config(_write(tmp_path, gguf_bytes(meta, _tensors(cfg)), "nometa.gguf"))
    assert rc == HOS_E_MISSING_META and "embedding_length" in err
    rc, _, err = _config(_write(tmp_path, gguf_bytes(model_meta(cfg, "qwen2"), _tensors(cfg, embd=False)), "noemb.gguf"))
    assert rc == HOS_E_MISSING_TENSOR and "token_embd" in err
    rc, _, err = _config(_write(tmp_path, gguf_bytes(model_meta(cfg, "mamba"), _tensors(cfg)), "arch.gguf"))
    assert rc == HOS_E_UNSUPPORTED_ARCH and "mamba" in err
    bad = gguf_bytes({"general.architecture": (STR, "qwen2"), "x": (U32, 1)}, {})
    i = bad.index(b"x") + 1
    bad = bad[:i] + struct.pack("<I", 99) + bad[i + 4:]
    assert _config(_write(tmp_path, bad, "vtype.gguf"))[0] == HOS_E_FORMAT


class _XorShift:
    """The xorshift64 stream of the reference's fuzz test (tests/fuzz_gguf.rs:22-35)."""
    def __init__(self, s):
        self.s = s

    def next(self):
        x = self.s
        x ^= (x << 13) & 0xFFFFFFFFFFFFFFFF
        x ^= x >> 7
        x ^= (x << 17) & 0xFFFFFFFFFFFFFFFF
        self.s = x
        return x

    def byte(self):
        return (self.next() >> 24) & 0xFF


def test_fuzz_never_crashes(tmp_path):
    """Random bytes, GGUF magic + garbage, truncations and byte flips of a valid file: every call
    returns (0 or an error code); a crash would take the test process down."""
    r = _XorShift(0x9E3779B97F4A7C15)
    p = tmp_path / "fz.gguf"
    n = 0
    for ln in (0, 1, 4, 8, 24, 64, 200, 4096):
        for _ in range(10):
            p.write_bytes(bytes(r.byte() for _ in range(ln)))
            assert _config(p)[0] != 0
            n += 1
    for _ in range(100):
        p.write_bytes(b"GGUF" + bytes(r.byte() for _ in range(r.next() % 512)))
        assert _config(p)[0] in (HOS_E_FORMAT, HOS_E_MISSING_META, HOS_E_MISSING_TENSOR, HOS_E_UNSUPPORTED_ARCH)
    cfg = Cfg()
    full = gguf_bytes(model_meta(cfg, "qwen2"), _tensors(cfg, output=True))
    for _ in range(60):
        p.write_bytes(full[: r.next() % len(full)])
        _config(p)
    for _ in range(120):
        b = bytearray(full)
        for _ in range(1 + r.next() % 2):
            b[r.next() % len(b)] ^= r.byte()
        p.write_bytes(bytes(b))
        _config(p)


def test_olmoe_mapping(tmp_path):
    """OLMoE (src/model.rs:792-795, 872-873): expert_count / expert_used_count with the stacked expert
    tensors present make a mixture-of-experts FFN; attn_q_norm turns on QK-norm; NEOX RoPE."""
    cfg = Cfg()
    meta = model_meta(cfg, "olmoe", extra={"olmoe.expert_count": (U32, 8), "olmoe.expert_used_count": (U32, 2)})
    t = _tensors(cfg, bias=False)
    t["blk.0.ffn_gate_exps.weight"] = (np.zeros(8 * 256 * 128 // 32 * 34, np.uint8), 8, [128, 256, 8])
    t["blk.0.attn_q_norm.weight"] = (np.ones(128, np.float32), 0, [128])
    rc, c, err = _config(_write(tmp_path, gguf_bytes(meta, t)))
    assert rc == 0, err
    assert (c.n_experts, c.n_experts_used, c.qk_norm, c.rope_neox) == (8, 2, 1, 1)
    del t["blk.0.ffn_gate_exps.weight"]  # expert_count without expert tensors: dense (src/model.rs:795)
    rc, c, err = _config(_write(tmp_path, gguf_bytes(meta, t), "dense.gguf"))
    assert rc == 0 and c.n_experts == 0


def test_qwen2moe_mapping(tmp_path):
    """qwen2moe is the Qwen2 family (Arch::detect, src/model.rs:35): keys under `qwen2moe.`, NEOX RoPE, QKV
    bias detection, experts from expert_count / expert_used_count with the stacked expert tensors present."""
    cfg = Cfg()
    meta = model_meta(cfg, "qwen2moe", extra={"qwen2moe.expert_count": (U32, 4), "qwen2moe.expert_used_count": (U32, 2)})
    t = _tensors(cfg, bias=True)
    t["blk.0.ffn_gate_exps.weight"] = (np.zeros(4 * 256 * 128 // 32 * 34, np.uint8), 8, [128, 256, 4])
    rc, c, err = _config(_write(tmp_path, gguf_bytes(meta, t)))
    assert rc == 0, err
    assert (c.dim, c.n_layers, c.n_heads, c.n_kv_heads) == (cfg.dim, cfg.n_layers, cfg.n_heads, cfg.n_kv_heads)
    assert (c.rope_neox, c.attn_bias, c.n_experts, c.n_experts_used) == (1, 1, 4, 2)


def test_oversized_tensor_dims_refused(tmp_path):
    """Tensor dims whose byte count would overflow are a format error from the config call, not a wrapped
    size (the data bounds are checked before any byte is read)."""
    cfg = Cfg()
    t = _tensors(cfg)
    t["blk.0.attn_q.weight"] = (np.zeros(64, np.uint8), 0, [1 << 31, 1 << 31])
    rc, _, err = _config(_write(tmp_path, gguf_bytes(model_meta(cfg, "qwen2"), t)))
    assert rc == HOS_E_FORMAT, err
