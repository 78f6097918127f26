"""ORACLE — test infrastructure only.

ctypes binding of ``liboracle.so``, the CPU restatement of HOS's CPU training path
(GGUF codec from src/gguf.rs + src/gguf_write.rs, autograd ops from src/tensor.rs,
LoRA model from src/peft.rs). Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this module; the product path
(``hos_amd``) never does.
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

F32P = ctypes.POINTER(ctypes.c_float)
I32P = ctypes.POINTER(ctypes.c_int32)
U8P = ctypes.POINTER(ctypes.c_uint8)


class OrcCfg(ctypes.Structure):
    _fields_ = [
        ("n_layers", ctypes.c_int), ("dim", ctypes.c_int), ("n_heads", ctypes.c_int),
        ("n_kv_heads", ctypes.c_int), ("head_dim", ctypes.c_int), ("ffn_dim", ctypes.c_int),
        ("vocab", ctypes.c_int), ("rms_eps", ctypes.c_float), ("rope_base", ctypes.c_float),
        ("rope_neox", ctypes.c_int), ("attn_bias", ctypes.c_int), ("lora_rank", ctypes.c_int),
        ("lora_alpha", ctypes.c_float), ("lora_targets", ctypes.c_uint32),
        ("n_experts", ctypes.c_int), ("n_experts_used", ctypes.c_int), ("qk_norm", ctypes.c_int),
        ("rga_genes", ctypes.c_int), ("rga_bottleneck", ctypes.c_int), ("rga_lambda", ctypes.c_float),
    ]


def build():
    """Compile liboracle.so from oracle/*.cpp (g++, OpenMP)."""
    subprocess.check_call(["make", "-s", "-C", _HERE])


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.orc_f16_to_f32.restype = ctypes.c_float
        L.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.orc_f32_to_f16.restype = ctypes.c_uint16
        L.orc_f32_to_f16.argtypes = [ctypes.c_float]
        L.orc_set_threads.restype = ctypes.c_int
        L.orc_set_threads.argtypes = [ctypes.c_int]
        L.orc_bytes_for.restype = ctypes.c_size_t
        L.orc_bytes_for.argtypes = [ctypes.c_uint32, ctypes.c_size_t]
        L.orc_dequant.argtypes = [ctypes.c_void_p, ctypes.c_uint32, ctypes.c_size_t, ctypes.c_void_p]
        L.orc_quantize.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_uint32, ctypes.c_void_p]
        L.orc_qkx_scale_min.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, F32P, F32P]
        L.orc_pack_scales_mins.argtypes = [ctypes.c_void_p] * 3
        sz = ctypes.c_size_t
        vp = ctypes.c_void_p
        L.orc_op_matmul.argtypes = [vp, sz, sz, vp, sz, vp, vp, vp, vp]
        L.orc_op_rmsnorm.argtypes = [vp, vp, sz, sz, ctypes.c_float, vp, vp, vp, vp]
        L.orc_op_rope.argtypes = [vp, sz, sz, sz, ctypes.c_float, ctypes.c_int, vp, vp, vp, vp]
        L.orc_op_swiglu.argtypes = [vp, vp, sz, vp, vp, vp, vp]
        L.orc_op_softmax_rows.argtypes = [vp, sz, sz, vp, vp, vp]
        L.orc_op_cross_entropy.argtypes = [vp, sz, sz, vp, ctypes.c_float, F32P, vp]
        L.orc_op_attention.argtypes = [vp, vp, vp, sz, sz, sz, sz, vp, vp, vp, vp, vp]
        L.orc_adamw.argtypes = [vp, vp, vp, vp, sz, ctypes.c_uint64, ctypes.c_float, ctypes.c_float, ctypes.c_int]
        L.orc_randn_uniform.argtypes = [sz, sz, ctypes.POINTER(ctypes.c_uint64), vp]
        L.orc_case.argtypes = [ctypes.c_char_p, ctypes.c_int, ctypes.POINTER(ctypes.c_void_p), vp, vp, F32P,
                               ctypes.POINTER(ctypes.c_void_p)]
        L.orc_model_create.restype = vp
        L.orc_model_create.argtypes = [ctypes.POINTER(OrcCfg)]
        L.orc_model_destroy.argtypes = [vp]
        L.orc_model_set_tensor.argtypes = [vp, ctypes.c_char_p, vp, ctypes.c_uint32, sz, sz]
        L.orc_model_set_lora.argtypes = [vp, ctypes.c_int, ctypes.c_int, vp, vp]
        L.orc_model_get_lora.argtypes = [vp, ctypes.c_int, ctypes.c_int, vp, vp]
        L.orc_model_get_lora_grad.argtypes = [vp, ctypes.c_int, ctypes.c_int, vp, vp]
        L.orc_model_rga_tensor.argtypes = [vp, ctypes.c_char_p, vp, vp, sz, ctypes.c_int]
        L.orc_model_loss_grad.restype = ctypes.c_float
        L.orc_model_loss_grad.argtypes = [vp, vp, vp, ctypes.c_int, ctypes.c_int]
        L.orc_model_adamw.argtypes = [vp, ctypes.c_float, ctypes.c_float]
        L.orc_model_logits.argtypes = [vp, vp, ctypes.c_int, vp]
        L.orc_ft_create.restype = vp
        L.orc_ft_create.argtypes = [ctypes.POINTER(OrcCfg)]
        L.orc_ft_get.argtypes = [vp, ctypes.c_char_p, vp, vp]
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


# ---- codec ----

def set_threads(n=0):
    """OpenMP threads the oracle uses from now on (n <= 0: unchanged); returns the count in effect."""
    return lib().orc_set_threads(n)


def bytes_for(ggml_type, n):
    return lib().orc_bytes_for(ggml_type, n)


def dequant(raw, ggml_type, n):
    raw = np.ascontiguousarray(np.frombuffer(bytes(raw), dtype=np.uint8) if not isinstance(raw, np.ndarray) else raw,
                               dtype=np.uint8)
    out = np.empty(n, np.float32)
    rc = lib().orc_dequant(_p(raw), ggml_type, n, _p(out))
    if rc:
        raise ValueError(f"dequant: unsupported type {ggml_type}")
    return out


def quantize(x, ggml_type):
    x = _f32(x).ravel()
    out = np.zeros(bytes_for(ggml_type, x.size), np.uint8)
    rc = lib().orc_quantize(_p(x), x.size, ggml_type, _p(out))
    if rc:
        raise ValueError(f"quantize: rc={rc}")
    return out


def f32_to_f16_bits(v):
    return lib().orc_f32_to_f16(float(v))


def f16_bits_to_f32(h):
    return lib().orc_f16_to_f32(int(h))


def qkx_scale_min(x, nmax):
    x = _f32(x)
    s, m = ctypes.c_float(), ctypes.c_float()
    lib().orc_qkx_scale_min(_p(x), x.size, nmax, ctypes.byref(s), ctypes.byref(m))
    return s.value, m.value


# ---- single ops (forward + backward with upstream grad) ----

def op_matmul(a, b, gout=None):
    a, b = _f32(a), _f32(b)
    m, k = a.shape
    n = b.shape[1]
    out = np.empty((m, n), np.float32)
    da = np.empty_like(a) if gout is not None else None
    db = np.empty_like(b) if gout is not None else None
    lib().orc_op_matmul(_p(a), m, k, _p(b), n, _p(None if gout is None else _f32(gout)), _p(out), _p(da), _p(db))
    return out, da, db


def op_rmsnorm(x, w, eps, gout=None):
    x, w = _f32(x), _f32(w)
    r, d = x.shape
    out = np.empty_like(x)
    gx = np.empty_like(x) if gout is not None else None
    gw = np.empty_like(w) if gout is not None else None
    g = None if gout is None else _f32(gout)
    lib().orc_op_rmsnorm(_p(x), _p(w), r, d, eps, _p(g), _p(out), _p(gx), _p(gw))
    return out, gx, gw


def op_rope(x, n_heads, head_dim, base, neox, pos, gout=None):
    x = _f32(x)
    pos = np.ascontiguousarray(pos, dtype=np.int32)
    out = np.empty_like(x)
    dx = np.empty_like(x) if gout is not None else None
    g = None if gout is None else _f32(gout)
    lib().orc_op_rope(_p(x), x.shape[0], n_heads, head_dim, base, int(neox), _p(pos), _p(g), _p(out), _p(dx))
    return out, dx


def op_swiglu(g, u, gout=None):
    g, u = _f32(g), _f32(u)
    out = np.empty_like(g)
    dg = np.empty_like(g) if gout is not None else None
    du = np.empty_like(u) if gout is not None else None
    go = None if gout is None else _f32(gout)
    lib().orc_op_swiglu(_p(g), _p(u), g.size, _p(go), _p(out), _p(dg), _p(du))
    return out, dg, du


def op_cross_entropy(logits, targets, gscale=1.0, want_grad=True):
    logits = _f32(logits)
    n, v = logits.shape
    t = np.ascontiguousarray(targets, dtype=np.int32)
    loss = ctypes.c_float()
    dl = np.empty_like(logits) if want_grad else None
    lib().orc_op_cross_entropy(_p(logits), n, v, _p(t), gscale, ctypes.byref(loss), _p(dl))
    return loss.value, dl


def op_attention(q, k, v, n_heads, n_kv, head_dim, gout=None):
    q, k, v = _f32(q), _f32(k), _f32(v)
    t = q.shape[0]
    out = np.empty_like(q)
    dq = np.empty_like(q) if gout is not None else None
    dk = np.empty_like(k) if gout is not None else None
    dv = np.empty_like(v) if gout is not None else None
    g = None if gout is None else _f32(gout)
    lib().orc_op_attention(_p(q), _p(k), _p(v), t, n_heads, n_kv, head_dim, _p(g), _p(out), _p(dq), _p(dk), _p(dv))
    return out, dq, dk, dv


def adamw(p, g, m, v, t, lr, wd, decay):
    """One AdamW step (in place on copies); returns (p, m, v)."""
    p, m, v = _f32(p).copy(), _f32(m).copy(), _f32(v).copy()
    g = _f32(g)
    lib().orc_adamw(_p(p), _p(g), _p(m), _p(v), p.size, t, lr, wd, int(decay))
    return p, m, v


def randn_uniform(rows, cols, seed):
    s = ctypes.c_uint64(seed)
    out = np.empty((rows, cols), np.float32)
    lib().orc_randn_uniform(rows, cols, ctypes.byref(s), _p(out))
    return out, s.value


def case(name, inputs):
    """Evaluate a tests/autograd.rs closure; returns (loss, [grads])."""
    arrs = [_f32(a) for a, _ in inputs]
    dims = np.array([d for _, sh in inputs for d in sh], dtype=np.int64)
    nd = np.array([len(sh) for _, sh in inputs], dtype=np.int32)
    grads = [np.zeros(a.size, np.float32) for a in arrs]
    dp = (ctypes.c_void_p * len(arrs))(*[a.ctypes.data for a in arrs])
    gp = (ctypes.c_void_p * len(arrs))(*[g.ctypes.data for g in grads])
    loss = ctypes.c_float()
    rc = lib().orc_case(name.encode(), len(arrs), dp, _p(dims), _p(nd), ctypes.byref(loss), gp)
    if rc:
        raise ValueError(name)
    return loss.value, grads


# ---- whole model ----

class OracleModel:
    """PeftModel (LoRA) restatement: set GGUF tensors, LoRA factors; loss+grad; AdamW."""

    def __init__(self, cfg):
        self.cfg = cfg
        c = OrcCfg(cfg.n_layers, cfg.dim, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim, cfg.ffn_dim, cfg.vocab,
                   cfg.rms_eps, cfg.rope_base, int(cfg.rope_neox), int(cfg.attn_bias), cfg.lora_rank,
                   cfg.lora_alpha, cfg.lora_targets, int(getattr(cfg, "n_experts", 0)),
                   int(getattr(cfg, "n_experts_used", 0)), int(getattr(cfg, "qk_norm", 0)),
                   int(getattr(cfg, "rga_genes", 0)), int(getattr(cfg, "rga_bottleneck", 0)),
                   float(getattr(cfg, "rga_lambda", 0.0)))
        self._c = c
        self.h = lib().orc_model_create(ctypes.byref(c))

    def __del__(self):
        if getattr(self, "h", None):
            lib().orc_model_destroy(self.h)
            self.h = None

    def set_tensor(self, name, raw, ggml_type, rows, cols):
        raw = np.ascontiguousarray(raw, dtype=np.uint8) if isinstance(raw, np.ndarray) and raw.dtype == np.uint8 \
            else np.ascontiguousarray(np.frombuffer(np.ascontiguousarray(raw).tobytes(), np.uint8))
        rc = lib().orc_model_set_tensor(self.h, name.encode(), _p(raw), ggml_type, rows, cols)
        if rc:
            raise ValueError(f"set_tensor {name}: rc={rc}")

    def set_lora(self, layer, target, A, B):
        A, B = _f32(A), _f32(B)
        if lib().orc_model_set_lora(self.h, layer, target, _p(A), _p(B)):
            raise ValueError("set_lora")

    def get_lora(self, layer, target, shapes):
        A = np.empty(shapes[0], np.float32)
        B = np.empty(shapes[1], np.float32)
        lib().orc_model_get_lora(self.h, layer, target, _p(A), _p(B))
        return A, B

    def get_lora_grad(self, layer, target, shapes):
        A = np.empty(shapes[0], np.float32)
        B = np.empty(shapes[1], np.float32)
        lib().orc_model_get_lora_grad(self.h, layer, target, _p(A), _p(B))
        return A, B

    def set_rga(self, name, value):
        """Set an RGA parameter by its adapter tensor name (genome.0, wg, rga.{l}.wr / down.{k} / up.{k})."""
        v = _f32(value)
        if lib().orc_model_rga_tensor(self.h, name.encode(), _p(v), None, v.size, 1):
            raise ValueError(f"set_rga {name}")

    def get_rga(self, name, shape):
        """(value, gradient) of an RGA parameter in the reference layout."""
        v = np.empty(shape, np.float32)
        g = np.empty(shape, np.float32)
        if lib().orc_model_rga_tensor(self.h, name.encode(), _p(v), _p(g), v.size, 0):
            raise ValueError(f"get_rga {name}")
        return v, g

    def loss_grad(self, ids, targets):
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        tg = np.ascontiguousarray(targets, dtype=np.int32)
        B, T = ids.shape
        return lib().orc_model_loss_grad(self.h, _p(ids), _p(tg), B, T)

    def adamw(self, lr, wd=0.0):
        lib().orc_model_adamw(self.h, lr, wd)

    def logits(self, ids):
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        out = np.empty((ids.size, self.cfg.vocab), np.float32)
        lib().orc_model_logits(self.h, _p(ids), ids.size, _p(out))
        return out


class OracleFt(OracleModel):
    """FtModel (src/finetune.rs) restatement: every weight trainable; same set_tensor / loss_grad / adamw."""

    def __init__(self, cfg):
        c = OrcCfg(cfg.n_layers, cfg.dim, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim, cfg.ffn_dim, cfg.vocab,
                   cfg.rms_eps, cfg.rope_base, int(cfg.rope_neox), int(cfg.attn_bias), cfg.lora_rank or 1,
                   cfg.lora_alpha, 0, 0, 0, 0)
        self.cfg = cfg
        self._c = c
        self.h = lib().orc_ft_create(ctypes.byref(c))

    def get(self, name, shape):
        """(value, gradient) of a parameter by GGUF name, GGUF layout."""
        v = np.empty(shape, np.float32)
        g = np.empty(shape, np.float32)
        if lib().orc_ft_get(self.h, name.encode(), _p(v), _p(g)):
            raise ValueError(name)
        return v, g
