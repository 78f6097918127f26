"""ctypes loader for libhos_hip.so (the C ABI of include/hos_hip.h).

Loading fails loudly when the library has not been built: there is no CPU fallback.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("HOS_HIP_LIB") or os.path.join(HERE, "libhos_hip.so")

vp, sz, u32, u64, i32 = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_int


class PeftCfg(ctypes.Structure):
    _fields_ = [
        ("n_layers", i32), ("dim", i32), ("n_heads", i32), ("n_kv_heads", i32), ("head_dim", i32),
        ("ffn_dim", i32), ("vocab", i32), ("rms_eps", ctypes.c_float), ("rope_base", ctypes.c_float),
        ("rope_neox", i32), ("attn_bias", i32), ("lora_rank", i32), ("lora_alpha", ctypes.c_float),
        ("lora_targets", u32), ("max_batch", i32), ("max_seq", i32), ("gemm_passes", i32),
        ("n_experts", i32), ("n_experts_used", i32), ("qk_norm", i32),
        ("rga_genes", i32), ("rga_bottleneck", i32), ("rga_lambda", ctypes.c_float),
    ]


# name -> (restype, argtypes); every symbol include/hos_hip.h declares.
SIGNATURES = {
    "hos_hip_create": (i32, [i32, ctypes.POINTER(vp)]),
    "hos_hip_destroy": (None, [vp]),
    "hos_hip_last_error": (ctypes.c_char_p, [vp]),
    "hos_hip_synchronize": (i32, [vp]),
    "hos_hip_device_arch": (i32, [vp, ctypes.c_char_p, sz]),
    "hos_hip_matmul_f32_keyed": (i32, [vp, vp, sz, sz, vp, sz, u64, vp]),
    "hos_hip_matmul_abt_keyed": (i32, [vp, vp, sz, sz, vp, sz, u64, vp]),
    "hos_hip_matmul_atb_keyed": (i32, [vp, vp, sz, sz, vp, sz, u64, vp]),
    "hos_hip_evict": (i32, [vp, u64]),
    "hos_hip_clear_cache": (i32, [vp]),
    "hos_hip_upload_quant": (i32, [vp, u64, vp, sz, u32, sz, sz]),
    "hos_hip_dequant": (i32, [vp, u64, vp]),
    "hos_hip_qgemm_fwd": (i32, [vp, u64, vp, sz, vp]),
    "hos_hip_qgemm_dx": (i32, [vp, u64, vp, sz, vp]),
    "hos_hip_qgemm_fwd_dev": (i32, [vp, u64, vp, sz, vp]),
    "hos_hip_qgemm_dx_dev": (i32, [vp, u64, vp, sz, vp]),
    "hos_hip_qgemm_lora_dev": (i32, [vp, i32, u64, vp, sz, vp, sz, vp, sz, sz, i32, ctypes.c_float, vp]),
    "hos_hip_time_qgemm": (i32, [vp, i32, u64, vp, sz, vp, i32, ctypes.POINTER(ctypes.c_float)]),
    "hos_hip_timer_begin": (i32, [vp]),
    "hos_hip_timer_end": (i32, [vp, ctypes.POINTER(ctypes.c_float)]),
    "hos_hip_quantize": (i32, [vp, vp, sz, u32, vp]),
    "hos_hip_bytes_for": (sz, [u32, sz]),
    "hos_hip_quantize_dev": (i32, [vp, vp, sz, u32, vp]),
    "hos_hip_randn_dev": (i32, [vp, vp, sz, u64, ctypes.c_float]),
    "hos_hip_set_gemm_passes": (i32, [vp, i32]),
    "hos_hip_dev_alloc": (i32, [vp, sz, ctypes.POINTER(vp)]),
    "hos_hip_dev_free": (i32, [vp, vp]),
    "hos_hip_h2d": (i32, [vp, vp, vp, sz]),
    "hos_hip_d2h": (i32, [vp, vp, vp, sz]),
    "hos_peft_create": (i32, [vp, ctypes.POINTER(PeftCfg), ctypes.POINTER(vp)]),
    "hos_peft_destroy": (None, [vp]),
    "hos_ft_create": (i32, [vp, ctypes.POINTER(PeftCfg), ctypes.POINTER(vp)]),
    "hos_ft_destroy": (None, [vp]),
    "hos_ft_last_error": (ctypes.c_char_p, [vp]),
    "hos_ft_set_tensor": (i32, [vp, ctypes.c_char_p, vp, sz, u32, sz, sz]),
    "hos_ft_get": (i32, [vp, ctypes.c_char_p, vp, vp]),
    "hos_ft_loss_grad": (i32, [vp, vp, vp, i32, i32, ctypes.POINTER(ctypes.c_float)]),
    "hos_ft_adamw": (i32, [vp, ctypes.c_float, ctypes.c_float]),
    "hos_ft_step_dev": (i32, [vp, vp, vp, i32, i32, ctypes.c_float, ctypes.c_float, vp]),
    "hos_peft_save_hos": (i32, [vp, ctypes.c_char_p, ctypes.c_char_p, i32]),
    "hos_peft_load_hos": (i32, [vp, ctypes.c_char_p, i32]),
    "hos_peft_adapter_id": (i32, [vp, ctypes.c_char_p]),
    "hos_peft_base_id": (i32, [vp, ctypes.c_char_p]),
    "hos_format_card": (i32, [ctypes.c_char_p, ctypes.c_char_p, sz, ctypes.POINTER(sz)]),
    "hos_format_verify": (i32, [ctypes.c_char_p, ctypes.POINTER(sz), ctypes.c_char_p, sz]),
    "hos_gguf_config": (i32, [ctypes.c_char_p, ctypes.POINTER(PeftCfg), ctypes.c_char_p, sz]),
    "hos_peft_create_from_gguf": (i32, [vp, ctypes.c_char_p, ctypes.POINTER(PeftCfg), ctypes.POINTER(vp),
                                        ctypes.POINTER(PeftCfg)]),
    "hos_peft_last_error": (ctypes.c_char_p, [vp]),
    "hos_peft_set_tensor": (i32, [vp, ctypes.c_char_p, vp, sz, u32, sz, sz]),
    "hos_peft_set_lora": (i32, [vp, i32, i32, vp, vp]),
    "hos_peft_get_lora": (i32, [vp, i32, i32, vp, vp]),
    "hos_peft_get_lora_grad": (i32, [vp, i32, i32, vp, vp]),
    "hos_peft_set_adapter": (i32, [vp, ctypes.c_char_p, vp, ctypes.c_size_t]),
    "hos_peft_get_adapter": (i32, [vp, ctypes.c_char_p, vp, vp, ctypes.c_size_t]),
    "hos_peft_loss_grad": (i32, [vp, vp, vp, i32, i32, ctypes.POINTER(ctypes.c_float)]),
    "hos_peft_adamw": (i32, [vp, ctypes.c_float, ctypes.c_float]),
    "hos_peft_step_dev": (i32, [vp, vp, vp, i32, i32, ctypes.c_float, ctypes.c_float, vp]),
    "hos_peft_logits": (i32, [vp, vp, i32, vp]),
    "hos_hip_embedding": (i32, [vp, u64, vp, sz, vp]),
    "hos_hip_rmsnorm_fwd": (i32, [vp, vp, vp, sz, sz, ctypes.c_float, vp, vp]),
    "hos_hip_rmsnorm_bwd": (i32, [vp, vp, vp, vp, vp, sz, sz, vp]),
    "hos_hip_rope": (i32, [vp, vp, sz, sz, sz, i32, i32, i32, ctypes.c_float, i32, i32]),
    "hos_hip_swiglu_fwd": (i32, [vp, vp, sz, sz, vp]),
    "hos_hip_swiglu_bwd": (i32, [vp, vp, vp, sz, sz, vp]),
    "hos_hip_attention_fwd": (i32, [vp, vp, sz, sz, sz, i32, i32, i32, i32, i32, vp, sz, vp]),
    "hos_hip_attention_bwd": (i32, [vp, vp, sz, sz, sz, vp, vp, sz, vp, i32, i32, i32, i32, i32, vp, sz]),
    "hos_hip_cross_entropy": (i32, [vp, vp, sz, sz, vp, ctypes.c_float, vp, vp]),
    "hos_hip_moe_route": (i32, [vp, vp, sz, i32, i32, vp, vp, vp, vp, vp]),
    "hos_hip_adamw": (i32, [vp, vp, vp, vp, vp, sz, ctypes.c_float, ctypes.c_float, ctypes.c_float,
                            ctypes.c_float, ctypes.c_float, i32, i32]),
    "hos_hip_lora": (i32, [vp, vp, vp, sz, sz, sz, i32, vp, vp, ctypes.c_float, vp, vp, vp, vp, vp]),
    "hos_hip_lora_noalloc": (i32, [vp, vp, vp, sz, sz, sz, i32, vp, vp, ctypes.c_float, vp, vp, vp, vp, vp]),
    "hos_peft_profile": (i32, [vp, i32]),
    "hos_peft_use_graph": (i32, [vp, i32]),
    "hos_peft_profile_only": (i32, [vp, ctypes.c_char_p]),
    "hos_peft_kernel_stats": (i32, [vp, ctypes.c_char_p, ctypes.POINTER(ctypes.c_longlong),
                                    ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double),
                                    ctypes.POINTER(ctypes.c_double)]),
}

_lib = None


def lib():
    """Load libhos_hip.so; raises if it is missing (build with hos_amd.build.build())."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built: run `python -m hos_amd.build` "
                               "(the HIP backend has no CPU fallback)")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib
