//! HIP backend for MI355X (gfx950): the `Gpu` surface of `src/metal_be_stub.rs` over libhos_hip's C ABI
//! (`include/hos_hip.h`). Drop-in sibling of `metal_be.rs` / `metal_be_stub.rs`, selected on Linux by the `hip`
//! feature (`src/lib.rs:43-47` module swap):
//!
//! ```text
//! #[cfg(all(not(target_os = "macos"), feature = "hip"))]
//! #[path = "hip_be.rs"]
//! pub mod metal_be;
//! ```
//!
//! Conventions kept from the reference's `Gpu`: host slices in, owned `Vec<f32>` out, frozen operands cached by
//! their never-reused tensor id (`Option<u64>`, `None` = not cached → key 0), and a panic on failure (the
//! reference's `Gpu` has no `Result` at this boundary). The training path reaches it through the thread-local
//! `GPU` of `src/tensor.rs:30-97` (`gmm`, `gmm_abt`, `gmm_atb`). The whole-step fast path (`PeftStep`) replaces
//! the body of the `cmd_peft` loop (`src/main.rs:2583-2601`) with one library call per optimizer step.
//! Inference-only methods (`matvec*`, the K-quant prefill / 2-token matmuls, conv3d, `GpuRunner`) keep the
//! stub's `unreachable!`: the inference path is not part of this backend, and `Weight::Gpu` is never built off
//! macOS.
//!
//! Link: `build.rs` adds `cargo:rustc-link-lib=dylib=hos_hip` and the directory of `libhos_hip.so`
//! (`python -m hos_amd.build`).
#![allow(non_snake_case, clippy::too_many_arguments, clippy::new_without_default)]

use std::ffi::{CStr, CString};
use std::os::raw::{c_char, c_int, c_void};
use std::sync::atomic::{AtomicU64, Ordering};

use crate::model::Model;

const NOT_HERE: &str = "the HIP backend implements the training path only (no inference kernels)";

#[repr(C)]
pub struct HosCtx {
    _p: [u8; 0],
}
#[repr(C)]
pub struct HosPeft {
    _p: [u8; 0],
}
#[repr(C)]
pub struct HosFt {
    _p: [u8; 0],
}

/// Field for field the C `hos_peft_cfg` of include/hos_hip.h (23 fields, same order and types;
/// tests/test_integration_doc.py checks this struct against the header and the ctypes mirror).
#[repr(C)]
#[derive(Default, Clone, Copy, Debug)]
pub struct HosPeftCfg {
    pub n_layers: c_int,
    pub dim: c_int,
    pub n_heads: c_int,
    pub n_kv_heads: c_int,
    pub head_dim: c_int,
    pub ffn_dim: c_int,
    pub vocab: c_int,
    pub rms_eps: f32,
    pub rope_base: f32,
    pub rope_neox: c_int,
    pub attn_bias: c_int,
    pub lora_rank: c_int,
    pub lora_alpha: f32,
    pub lora_targets: u32,
    pub max_batch: c_int,
    pub max_seq: c_int,
    pub gemm_passes: c_int,
    pub n_experts: c_int,
    pub n_experts_used: c_int,
    pub qk_norm: c_int,
    pub rga_genes: c_int,
    pub rga_bottleneck: c_int,
    pub rga_lambda: f32,
}

/// Every entry point of include/hos_hip.h, argument for argument (names and C types; `in` is `in_`).
#[link(name = "hos_hip")]
extern "C" {
    pub fn hos_hip_create(device: c_int, out: *mut *mut HosCtx) -> c_int;
    pub fn hos_hip_destroy(ctx: *mut HosCtx);
    pub fn hos_hip_last_error(ctx: *const HosCtx) -> *const c_char;
    pub fn hos_hip_synchronize(ctx: *mut HosCtx) -> c_int;
    pub fn hos_hip_device_arch(ctx: *mut HosCtx, buf: *mut c_char, len: usize) -> c_int;
    pub fn hos_hip_matmul_f32_keyed(ctx: *mut HosCtx, a: *const f32, m: usize, k: usize, b: *const f32, n: usize,
                                    b_key: u64, out: *mut f32) -> c_int;
    pub fn hos_hip_matmul_abt_keyed(ctx: *mut HosCtx, a: *const f32, m: usize, n: usize, b: *const f32, k: usize,
                                    b_key: u64, out: *mut f32) -> c_int;
    pub fn hos_hip_matmul_atb_keyed(ctx: *mut HosCtx, a: *const f32, k: usize, m: usize, b: *const f32, n: usize,
                                    a_key: u64, out: *mut f32) -> c_int;
    pub fn hos_hip_evict(ctx: *mut HosCtx, key: u64) -> c_int;
    pub fn hos_hip_clear_cache(ctx: *mut HosCtx) -> c_int;
    pub fn hos_hip_upload_quant(ctx: *mut HosCtx, key: u64, bytes: *const u8, nbytes: usize, ggml_type: u32,
                                rows: usize, cols: usize) -> c_int;
    pub fn hos_hip_dequant(ctx: *mut HosCtx, key: u64, out: *mut f32) -> c_int;
    pub fn hos_hip_qgemm_fwd(ctx: *mut HosCtx, key: u64, x: *const f32, t: usize, y: *mut f32) -> c_int;
    pub fn hos_hip_qgemm_dx(ctx: *mut HosCtx, key: u64, dy: *const f32, t: usize, dx: *mut f32) -> c_int;
    pub fn hos_hip_qgemm_fwd_dev(ctx: *mut HosCtx, key: u64, x_dev: *const f32, t: usize, y_dev: *mut f32) -> c_int;
    pub fn hos_hip_qgemm_dx_dev(ctx: *mut HosCtx, key: u64, dy_dev: *const f32, t: usize,
                                dx_dev: *mut f32) -> c_int;
    pub fn hos_hip_qgemm_lora_dev(ctx: *mut HosCtx, which: c_int, key: u64, in_dev: *const f32, t: usize,
                                  u_dev: *const f32, ldu: usize, l_dev: *const f32, slj: usize, sln: usize,
                                  rank: c_int, scale: f32, out_dev: *mut f32) -> c_int;
    pub fn hos_hip_time_qgemm(ctx: *mut HosCtx, which: c_int, key: u64, in_dev: *const f32, t: usize,
                              out_dev: *mut f32, iters: c_int, avg_ms: *mut f32) -> c_int;
    pub fn hos_hip_timer_begin(ctx: *mut HosCtx) -> c_int;
    pub fn hos_hip_timer_end(ctx: *mut HosCtx, ms: *mut f32) -> c_int;
    pub fn hos_hip_quantize(ctx: *mut HosCtx, x: *const f32, n: usize, ggml_type: u32, out: *mut u8) -> c_int;
    pub fn hos_hip_quantize_dev(ctx: *mut HosCtx, x_dev: *const f32, n: usize, ggml_type: u32,
                                out_dev: *mut u8) -> c_int;
    pub fn hos_hip_randn_dev(ctx: *mut HosCtx, out_dev: *mut f32, n: usize, seed: u64, stddev: f32) -> c_int;
    pub fn hos_hip_set_gemm_passes(ctx: *mut HosCtx, passes: c_int) -> c_int;
    pub fn hos_hip_bytes_for(ggml_type: u32, n: usize) -> usize;
    pub fn hos_hip_embedding(ctx: *mut HosCtx, key: u64, ids_dev: *const i32, rows: usize,
                             out_dev: *mut f32) -> c_int;
    pub fn hos_hip_rmsnorm_fwd(ctx: *mut HosCtx, x: *const f32, w: *const f32, rows: usize, d: usize, eps: f32,
                               y: *mut f32, inv: *mut f32) -> c_int;
    pub fn hos_hip_rmsnorm_bwd(ctx: *mut HosCtx, g: *const f32, x: *const f32, inv: *const f32, w: *const f32,
                               rows: usize, d: usize, gx: *mut f32) -> c_int;
    pub fn hos_hip_rope(ctx: *mut HosCtx, x: *mut f32, rows: usize, ld: usize, col0: usize, n_heads: c_int,
                        head_dim: c_int, seq_len: c_int, base: f32, neox: c_int, inverse: c_int) -> c_int;
    pub fn hos_hip_swiglu_fwd(ctx: *mut HosCtx, gu: *const f32, rows: usize, F: usize, h: *mut f32) -> c_int;
    pub fn hos_hip_swiglu_bwd(ctx: *mut HosCtx, gu: *const f32, dh: *const f32, rows: usize, F: usize,
                              dgu: *mut f32) -> c_int;
    pub fn hos_hip_attention_fwd(ctx: *mut HosCtx, qkv: *const f32, ld: usize, kcol: usize, vcol: usize, B: c_int,
                                 T: c_int, n_heads: c_int, n_kv_heads: c_int, head_dim: c_int, o: *mut f32,
                                 ldo: usize, lse: *mut f32) -> c_int;
    pub fn hos_hip_attention_bwd(ctx: *mut HosCtx, qkv: *const f32, ld: usize, kcol: usize, vcol: usize,
                                 o: *const f32, dout: *const f32, ldo: usize, lse: *const f32, B: c_int, T: c_int,
                                 n_heads: c_int, n_kv_heads: c_int, head_dim: c_int, dqkv: *mut f32,
                                 ldd: usize) -> c_int;
    pub fn hos_hip_cross_entropy(ctx: *mut HosCtx, logits: *const f32, rows: usize, V: usize, targets: *const i32,
                                 gscale: f32, row_loss: *mut f32, dlogits: *mut f32) -> c_int;
    pub fn hos_hip_moe_route(ctx: *mut HosCtx, logits: *const f32, rows: usize, E: c_int, K: c_int, pfull: *mut f32,
                             sel_e: *mut i32, sel_p: *mut f32, slot: *mut i32, counts: *mut i32) -> c_int;
    pub fn hos_hip_adamw(ctx: *mut HosCtx, p: *mut f32, g: *const f32, m: *mut f32, v: *mut f32, n: usize, lr: f32,
                         beta1: f32, beta2: f32, eps: f32, wd: f32, step: c_int, decay: c_int) -> c_int;
    pub fn hos_hip_lora(ctx: *mut HosCtx, x: *const f32, dy: *const f32, rows: usize, in_: usize, out: usize,
                        r: c_int, A: *const f32, B: *const f32, scale: f32, y: *mut f32, u: *mut f32, dA: *mut f32,
                        dB: *mut f32, dx: *mut f32) -> c_int;
    pub fn hos_hip_lora_noalloc(ctx: *mut HosCtx, x: *const f32, dy: *const f32, rows: usize, in_: usize, out: usize,
                                r: c_int, A: *const f32, B: *const f32, scale: f32, y: *mut f32, u: *mut f32,
                                dA: *mut f32, dB: *mut f32, dx: *mut f32) -> c_int;
    pub fn hos_hip_dev_alloc(ctx: *mut HosCtx, nbytes: usize, dptr: *mut *mut c_void) -> c_int;
    pub fn hos_hip_dev_free(ctx: *mut HosCtx, dptr: *mut c_void) -> c_int;
    pub fn hos_hip_h2d(ctx: *mut HosCtx, dst_dev: *mut c_void, src_host: *const c_void, nbytes: usize) -> c_int;
    pub fn hos_hip_d2h(ctx: *mut HosCtx, dst_host: *mut c_void, src_dev: *const c_void, nbytes: usize) -> c_int;
    pub fn hos_peft_create(ctx: *mut HosCtx, cfg: *const HosPeftCfg, out: *mut *mut HosPeft) -> c_int;
    pub fn hos_peft_destroy(p: *mut HosPeft);
    pub fn hos_peft_last_error(p: *const HosPeft) -> *const c_char;
    pub fn hos_peft_set_tensor(p: *mut HosPeft, name: *const c_char, bytes: *const u8, nbytes: usize, ggml_type: u32,
                               rows: usize, cols: usize) -> c_int;
    pub fn hos_gguf_config(path: *const c_char, cfg: *mut HosPeftCfg, err: *mut c_char, err_len: usize) -> c_int;
    pub fn hos_peft_create_from_gguf(ctx: *mut HosCtx, path: *const c_char, train: *const HosPeftCfg,
                                     out: *mut *mut HosPeft, out_cfg: *mut HosPeftCfg) -> c_int;
    pub fn hos_peft_set_lora(p: *mut HosPeft, layer: c_int, target: c_int, A: *const f32, B: *const f32) -> c_int;
    pub fn hos_peft_get_lora(p: *mut HosPeft, layer: c_int, target: c_int, A: *mut f32, B: *mut f32) -> c_int;
    pub fn hos_peft_get_lora_grad(p: *mut HosPeft, layer: c_int, target: c_int, dA: *mut f32,
                                  dB: *mut f32) -> c_int;
    pub fn hos_peft_set_adapter(p: *mut HosPeft, name: *const c_char, data: *const f32, n: usize) -> c_int;
    pub fn hos_peft_get_adapter(p: *mut HosPeft, name: *const c_char, value: *mut f32, grad: *mut f32,
                                n: usize) -> c_int;
    pub fn hos_peft_loss_grad(p: *mut HosPeft, ids: *const i32, targets: *const i32, B: c_int, T: c_int,
                              loss: *mut f32) -> c_int;
    pub fn hos_peft_adamw(p: *mut HosPeft, lr: f32, wd: f32) -> c_int;
    pub fn hos_peft_step_dev(p: *mut HosPeft, ids_dev: *const i32, targets_dev: *const i32, B: c_int, T: c_int,
                             lr: f32, wd: f32, loss_dev: *mut f32) -> c_int;
    pub fn hos_peft_use_graph(p: *mut HosPeft, enable: c_int) -> c_int;
    pub fn hos_peft_save_hos(p: *mut HosPeft, path: *const c_char, card_json: *const c_char,
                             with_optimizer: c_int) -> c_int;
    pub fn hos_peft_load_hos(p: *mut HosPeft, path: *const c_char, with_optimizer: c_int) -> c_int;
    pub fn hos_peft_adapter_id(p: *mut HosPeft, out17: *mut c_char) -> c_int;
    pub fn hos_peft_base_id(p: *mut HosPeft, out17: *mut c_char) -> c_int;
    pub fn hos_format_card(path: *const c_char, out: *mut c_char, len: usize, needed: *mut usize) -> c_int;
    pub fn hos_format_verify(path: *const c_char, n_tensors: *mut usize, err: *mut c_char, err_len: usize) -> c_int;
    pub fn hos_ft_create(ctx: *mut HosCtx, cfg: *const HosPeftCfg, out: *mut *mut HosFt) -> c_int;
    pub fn hos_ft_destroy(p: *mut HosFt);
    pub fn hos_ft_last_error(p: *const HosFt) -> *const c_char;
    pub fn hos_ft_set_tensor(p: *mut HosFt, name: *const c_char, bytes: *const u8, nbytes: usize, ggml_type: u32,
                             rows: usize, cols: usize) -> c_int;
    pub fn hos_ft_get(p: *mut HosFt, name: *const c_char, value: *mut f32, grad: *mut f32) -> c_int;
    pub fn hos_ft_loss_grad(p: *mut HosFt, ids: *const i32, targets: *const i32, B: c_int, T: c_int,
                            loss: *mut f32) -> c_int;
    pub fn hos_ft_adamw(p: *mut HosFt, lr: f32, wd: f32) -> c_int;
    pub fn hos_ft_step_dev(p: *mut HosFt, ids_dev: *const i32, targets_dev: *const i32, B: c_int, T: c_int, lr: f32,
                           wd: f32, loss_dev: *mut f32) -> c_int;
    pub fn hos_peft_logits(p: *mut HosPeft, ids: *const i32, T: c_int, out: *mut f32) -> c_int;
    pub fn hos_peft_profile(p: *mut HosPeft, enable: c_int) -> c_int;
    pub fn hos_peft_profile_only(p: *mut HosPeft, cls: *const c_char) -> c_int;
    pub fn hos_peft_kernel_stats(p: *mut HosPeft, cls: *const c_char, launches: *mut i64, total_ms: *mut f64,
                                 flops: *mut f64, bytes: *mut f64) -> c_int;
}

/// The reference's `Gpu` (`src/metal_be_stub.rs:33-208`), one per thread.
pub struct Gpu {
    ctx: *mut HosCtx,
}

/// A device-resident f32 buffer (`src/metal_be_stub.rs:13-15` `GpuBuf`): the allocation and the context that owns
/// it. `Tensor` keeps one as its resident copy (`src/tensor.rs:194`).
pub struct GpuBuf {
    ctx: *mut HosCtx,
    ptr: *mut c_void,
    bytes: usize,
}

/// `src/metal_be_stub.rs:17-20`: copy the first `n` floats of a resident buffer back to the host.
pub fn download_buf(buf: &GpuBuf, n: usize) -> Vec<f32> {
    assert!(n * 4 <= buf.bytes, "download_buf: {n} floats from a {}-byte buffer", buf.bytes);
    let mut out = vec![0.0f32; n];
    let rc = unsafe { hos_hip_d2h(buf.ctx, out.as_mut_ptr() as *mut c_void, buf.ptr, n * 4) };
    assert!(rc == 0, "hos_hip_d2h failed ({rc})");
    out
}

impl Drop for GpuBuf {
    fn drop(&mut self) {
        unsafe { hos_hip_dev_free(self.ctx, self.ptr) };
    }
}

/// A frozen weight kept quantized on the device (`src/metal_be_stub.rs:22-28` `GpuMatrix`), uploaded under a
/// library key that no tensor id uses (the top bit set) and evicted when dropped.
#[derive(Default)]
pub struct GpuMatrix {
    pub n_rows: usize,
    pub in_dim: usize,
    pub ggml_type: u32,
    key: u64,
    ctx: usize, // *mut HosCtx of the owning Gpu (0 = empty)
}

impl Drop for GpuMatrix {
    fn drop(&mut self) {
        if self.ctx != 0 {
            unsafe { hos_hip_evict(self.ctx as *mut HosCtx, self.key) };
        }
    }
}

static NEXT_MATRIX_KEY: AtomicU64 = AtomicU64::new(1 << 63);

fn ctx_error(ctx: *const HosCtx) -> String {
    unsafe { CStr::from_ptr(hos_hip_last_error(ctx)) }.to_string_lossy().into_owned()
}

impl Gpu {
    pub fn new() -> Gpu {
        let mut ctx = std::ptr::null_mut();
        let rc = unsafe { hos_hip_create(0, &mut ctx) };
        assert!(rc == 0, "hos_hip_create failed ({rc})");
        Gpu { ctx }
    }
    fn check(&self, rc: c_int) {
        if rc != 0 {
            panic!("hip backend: {} ({rc})", ctx_error(self.ctx));
        }
    }
    pub fn clear_cache(&self) {
        self.check(unsafe { hos_hip_clear_cache(self.ctx) });
    }
    /// Plain f32 GEMM out[m, n] = a[m, k]·b[k, n] (no operand cached).
    pub fn matmul_f32(&self, a: &[f32], m: usize, k: usize, b: &[f32], n: usize) -> Vec<f32> {
        self.matmul_f32_keyed(a, m, k, b, n, None)
    }
    pub fn upload_matrix(&self, _w: &[f32], _n_rows: usize, _in_dim: usize) -> GpuMatrix {
        unreachable!("{NOT_HERE}")
    }
    /// `src/metal_be_stub.rs:46-53`: a GGUF weight [n_rows, in_dim] kept quantized on the device (Q8_0, Q4_K,
    /// Q6_K natively; Q4_0 / Q5_0 / Q5_K / F16 / BF16 / F32 repacked exactly on upload).
    pub fn upload_quant(&self, bytes: &[u8], ggml_type: u32, n_rows: usize, in_dim: usize) -> GpuMatrix {
        let key = NEXT_MATRIX_KEY.fetch_add(1, Ordering::Relaxed);
        self.upload_quant_keyed(key, bytes, ggml_type, n_rows, in_dim);
        GpuMatrix { n_rows, in_dim, ggml_type, key, ctx: self.ctx as usize }
    }
    pub fn matvec_into(&self, _w: &GpuMatrix, _x: &[f32], _out: &mut [f32]) {
        unreachable!("{NOT_HERE}")
    }
    pub fn matvec(&self, _w: &GpuMatrix, _x: &[f32]) -> Vec<f32> {
        unreachable!("{NOT_HERE}")
    }
    pub fn matmul_q4k_prefill_into(&self, _w: &GpuMatrix, _x: &[f32], _ntok: usize, _out: &mut [f32]) {
        unreachable!("{NOT_HERE}")
    }
    pub fn matmul_q6k_prefill_into(&self, _w: &GpuMatrix, _x: &[f32], _ntok: usize, _out: &mut [f32]) {
        unreachable!("{NOT_HERE}")
    }
    pub fn matmul_q4k_small_into(&self, _w: &GpuMatrix, _x: &[f32], _ntok: usize, _out: &mut [f32]) {
        unreachable!("{NOT_HERE}")
    }
    pub fn matmul_q6k_small_into(&self, _w: &GpuMatrix, _x: &[f32], _ntok: usize, _out: &mut [f32]) {
        unreachable!("{NOT_HERE}")
    }
    pub fn matmul_q4k_2tok_into(&self, _w: &GpuMatrix, _x: &[f32], _out: &mut [f32]) {
        unreachable!("{NOT_HERE}")
    }
    pub fn matmul_q6k_2tok_into(&self, _w: &GpuMatrix, _x: &[f32], _out: &mut [f32]) {
        unreachable!("{NOT_HERE}")
    }
    /// `gmm` (`src/tensor.rs:53-60`): out[m, n] = a[m, k]·b[k, n], b cached under its tensor id.
    pub fn matmul_f32_keyed(&self, a: &[f32], m: usize, k: usize, b: &[f32], n: usize, b_key: Option<u64>) -> Vec<f32> {
        assert!(a.len() >= m * k && b.len() >= k * n);
        let mut out = vec![0.0f32; m * n];
        self.check(unsafe {
            hos_hip_matmul_f32_keyed(self.ctx, a.as_ptr(), m, k, b.as_ptr(), n, b_key.unwrap_or(0), out.as_mut_ptr())
        });
        out
    }
    /// `gmm_abt` (`src/tensor.rs:81-88`): out[m, k] = a[m, n]·b[k, n]ᵀ, b cached under its tensor id.
    pub fn matmul_abt_keyed(&self, a: &[f32], m: usize, n: usize, b: &[f32], k: usize, b_key: Option<u64>) -> Vec<f32> {
        assert!(a.len() >= m * n && b.len() >= k * n);
        let mut out = vec![0.0f32; m * k];
        self.check(unsafe {
            hos_hip_matmul_abt_keyed(self.ctx, a.as_ptr(), m, n, b.as_ptr(), k, b_key.unwrap_or(0), out.as_mut_ptr())
        });
        out
    }
    /// `gmm_atb` (`src/tensor.rs:90-97`): out[k, n] = a[m, k]ᵀ·b[m, n], a cached under its tensor id.
    pub fn matmul_atb_keyed(&self, a: &[f32], k: usize, m: usize, b: &[f32], n: usize, a_key: Option<u64>) -> Vec<f32> {
        assert!(a.len() >= m * k && b.len() >= m * n);
        let mut out = vec![0.0f32; k * n];
        self.check(unsafe {
            hos_hip_matmul_atb_keyed(self.ctx, a.as_ptr(), k, m, b.as_ptr(), n, a_key.unwrap_or(0), out.as_mut_ptr())
        });
        out
    }
    pub fn conv3d_bn_relu_infer(&self, _x: &[f32], _w: &[f32], _scale: &[f32], _shift: &[f32], _shape: [usize; 5],
                                _k: [usize; 3], _stride: [usize; 3], _pad: [usize; 3], _cout: usize,
                                _w_key: u64) -> Vec<f32> {
        unreachable!("{NOT_HERE}")
    }
    pub fn conv3d_bn_relu_backward(&self, _x: &[f32], _w: &[f32], _scale: &[f32], _out: &[f32], _gout: &[f32],
                                   _shape: [usize; 5], _k: [usize; 3], _stride: [usize; 3], _pad: [usize; 3],
                                   _cout: usize, _w_key: u64, _need_dx: bool, _need_dw: bool)
                                   -> (Vec<f32>, Vec<f32>) {
        unreachable!("{NOT_HERE}")
    }
    pub fn depthwise_conv3d_forward(&self, _x: &[f32], _w: &[f32], _shape: [usize; 5], _k: [usize; 3],
                                    _stride: [usize; 3], _pad: [usize; 3], _w_key: u64) -> Vec<f32> {
        unreachable!("{NOT_HERE}")
    }
    pub fn depthwise_conv3d_backward(&self, _x: &[f32], _w: &[f32], _gout: &[f32], _shape: [usize; 5],
                                     _k: [usize; 3], _stride: [usize; 3], _pad: [usize; 3], _w_key: u64,
                                     _need_dx: bool, _need_dw: bool) -> (Vec<f32>, Vec<f32>) {
        unreachable!("{NOT_HERE}")
    }
    /// Drop the cached device copy of the operand keyed `key` (`gpu_evict`, `src/tensor.rs:63-70`, called when a
    /// tensor's data is mutated).
    pub fn evict(&self, key: u64) {
        self.check(unsafe { hos_hip_evict(self.ctx, key) });
    }

    // ---- beyond the stub: the quantized training GEMMs and device buffers ----

    /// y[t, n_rows] = x[t, in_dim]·deq(W)ᵀ for a weight from upload_quant (the frozen-base forward,
    /// `t_const(W)` + `Tensor::matmul`, `src/peft.rs:24-33`, `src/tensor.rs:307-327`).
    pub fn matmul_quant(&self, w: &GpuMatrix, x: &[f32], t: usize) -> Vec<f32> {
        assert!(x.len() >= t * w.in_dim);
        self.qgemm_fwd(w.key, x, t, w.n_rows)
    }
    /// dx[t, in_dim] = dy[t, n_rows]·deq(W) for a weight from upload_quant (`src/tensor.rs:347-360`).
    pub fn matmul_quant_dx(&self, w: &GpuMatrix, dy: &[f32], t: usize) -> Vec<f32> {
        assert!(dy.len() >= t * w.n_rows);
        self.qgemm_dx(w.key, dy, t, w.in_dim)
    }
    /// W dequantized to f32 exactly as `Gguf::dequant_into` does (`src/gguf.rs:330-505`).
    pub fn dequant(&self, w: &GpuMatrix) -> Vec<f32> {
        let mut out = vec![0.0f32; w.n_rows * w.in_dim];
        self.check(unsafe { hos_hip_dequant(self.ctx, w.key, out.as_mut_ptr()) });
        out
    }
    /// A resident f32 buffer holding `data` (what the Metal backend's residency path keeps per tensor).
    pub fn upload_buf(&self, data: &[f32]) -> GpuBuf {
        let bytes = data.len() * 4;
        let mut ptr = std::ptr::null_mut();
        self.check(unsafe { hos_hip_dev_alloc(self.ctx, bytes.max(4), &mut ptr) });
        self.check(unsafe { hos_hip_h2d(self.ctx, ptr, data.as_ptr() as *const c_void, bytes) });
        GpuBuf { ctx: self.ctx, ptr, bytes }
    }
    /// A frozen GGUF weight kept quantized on the device under a caller key (the reference dequantizes to f32).
    pub fn upload_quant_keyed(&self, key: u64, bytes: &[u8], ggml_type: u32, rows: usize, cols: usize) {
        self.check(unsafe {
            hos_hip_upload_quant(self.ctx, key, bytes.as_ptr(), bytes.len(), ggml_type, rows, cols)
        });
    }
    /// y[t, rows] = x[t, cols]·deq(W)ᵀ
    pub fn qgemm_fwd(&self, key: u64, x: &[f32], t: usize, rows: usize) -> Vec<f32> {
        let mut y = vec![0.0f32; t * rows];
        self.check(unsafe { hos_hip_qgemm_fwd(self.ctx, key, x.as_ptr(), t, y.as_mut_ptr()) });
        y
    }
    /// dx[t, cols] = dy[t, rows]·deq(W)
    pub fn qgemm_dx(&self, key: u64, dy: &[f32], t: usize, cols: usize) -> Vec<f32> {
        let mut dx = vec![0.0f32; t * cols];
        self.check(unsafe { hos_hip_qgemm_dx(self.ctx, key, dy.as_ptr(), t, dx.as_mut_ptr()) });
        dx
    }
    /// `quantize` (`src/gguf_write.rs:41-50`) run on the device, byte-identical to the reference encoders.
    pub fn quantize(&self, x: &[f32], ggml_type: u32) -> Vec<u8> {
        let n = unsafe { hos_hip_bytes_for(ggml_type, x.len()) };
        assert!(n > 0, "quantize: unsupported type {ggml_type}");
        let mut out = vec![0u8; n];
        self.check(unsafe { hos_hip_quantize(self.ctx, x.as_ptr(), x.len(), ggml_type, out.as_mut_ptr()) });
        out
    }
    /// Wait for every operation enqueued on this context.
    pub fn synchronize(&self) {
        self.check(unsafe { hos_hip_synchronize(self.ctx) });
    }
}

impl Drop for Gpu {
    fn drop(&mut self) {
        unsafe { hos_hip_destroy(self.ctx) }
    }
}

/// The whole LoRA (or RGA) training step on the device: `PeftModel::forward` + backward + `AdamW::step`
/// (`src/peft.rs:441-604`, `src/tensor.rs:2844-2881, 2923-2976`) behind one call per optimizer step.
pub struct PeftStep {
    p: *mut HosPeft,
}

impl PeftStep {
    /// `PeftModel::build_multi` (`src/peft.rs:134-231`) on `gpu`'s device; tensors follow with `set_tensor`.
    pub fn new(gpu: &Gpu, cfg: &HosPeftCfg) -> PeftStep {
        let mut p = std::ptr::null_mut();
        gpu.check(unsafe { hos_peft_create(gpu.ctx, cfg, &mut p) });
        PeftStep { p }
    }
    /// Base model and training config straight from a GGUF file (the library maps the metadata as
    /// `src/model.rs:713-771` does; `train` supplies the LoRA / arena fields). Returns the mapped config too.
    pub fn from_gguf(gpu: &Gpu, path: &str, train: &HosPeftCfg) -> (PeftStep, HosPeftCfg) {
        let c = CString::new(path).expect("path with NUL");
        let (mut p, mut cfg) = (std::ptr::null_mut(), HosPeftCfg::default());
        let rc = unsafe { hos_peft_create_from_gguf(gpu.ctx, c.as_ptr(), train, &mut p, &mut cfg) };
        assert!(rc == 0, "hos_peft_create_from_gguf failed ({rc}): {}", ctx_error(gpu.ctx));
        (PeftStep { p }, cfg)
    }
    fn check(&self, rc: c_int) {
        if rc != 0 {
            let msg = unsafe { CStr::from_ptr(hos_peft_last_error(self.p)) };
            panic!("hip peft: {} ({rc})", msg.to_string_lossy());
        }
    }
    /// One GGUF tensor by its GGUF name (`src/model.rs:713-921`).
    pub fn set_tensor(&self, name: &str, bytes: &[u8], ggml_type: u32, rows: usize, cols: usize) {
        let c = CString::new(name).expect("name with NUL");
        self.check(unsafe {
            hos_peft_set_tensor(self.p, c.as_ptr(), bytes.as_ptr(), bytes.len(), ggml_type, rows, cols)
        });
    }
    /// LoRA factors of (layer, target) in the reference layout: A [in, r], B [r, out]; target 0..6 = q, k, v, o,
    /// gate, up, down.
    pub fn set_lora(&self, layer: usize, target: usize, a: &[f32], b: &[f32]) {
        self.check(unsafe { hos_peft_set_lora(self.p, layer as c_int, target as c_int, a.as_ptr(), b.as_ptr()) });
    }
    pub fn get_lora(&self, layer: usize, target: usize, a: &mut [f32], b: &mut [f32]) {
        self.check(unsafe {
            hos_peft_get_lora(self.p, layer as c_int, target as c_int, a.as_mut_ptr(), b.as_mut_ptr())
        });
    }
    pub fn get_lora_grad(&self, layer: usize, target: usize, da: &mut [f32], db: &mut [f32]) {
        self.check(unsafe {
            hos_peft_get_lora_grad(self.p, layer as c_int, target as c_int, da.as_mut_ptr(), db.as_mut_ptr())
        });
    }
    /// An RGA parameter by its adapter tensor name (`src/peft.rs:741-760`).
    pub fn set_adapter(&self, name: &str, data: &[f32]) {
        let c = CString::new(name).expect("name with NUL");
        self.check(unsafe { hos_peft_set_adapter(self.p, c.as_ptr(), data.as_ptr(), data.len()) });
    }
    /// `train_minibatch` (`src/train.rs:33-52`, the `cmd_peft` loop body `src/main.rs:2583-2601`): zero the
    /// gradients, B sequences of T tokens with loss·(1/B), returns the mean loss.
    pub fn loss_grad(&self, ids: &[i32], targets: &[i32], batch: usize, seq: usize) -> f32 {
        assert!(ids.len() >= batch * seq && targets.len() >= batch * seq);
        let mut loss = 0.0f32;
        self.check(unsafe {
            hos_peft_loss_grad(self.p, ids.as_ptr(), targets.as_ptr(), batch as c_int, seq as c_int, &mut loss)
        });
        loss
    }
    /// `AdamW::step` (`src/tensor.rs:2923-2976`) over every trainable parameter.
    pub fn adamw(&self, lr: f32, wd: f32) {
        self.check(unsafe { hos_peft_adamw(self.p, lr, wd) });
    }
    /// `save_adapter` (`src/main.rs:2614-2688`): a version-2 `.hos` capsule (`src/format.rs`) with the card JSON,
    /// optionally with the AdamW state.
    pub fn save_hos(&self, path: &str, card_json: &str, with_optimizer: bool) {
        let (p, c) = (CString::new(path).expect("path"), CString::new(card_json).expect("card"));
        self.check(unsafe { hos_peft_save_hos(self.p, p.as_ptr(), c.as_ptr(), with_optimizer as c_int) });
    }
    pub fn load_hos(&self, path: &str, with_optimizer: bool) {
        let p = CString::new(path).expect("path");
        self.check(unsafe { hos_peft_load_hos(self.p, p.as_ptr(), with_optimizer as c_int) });
    }
}

impl Drop for PeftStep {
    fn drop(&mut self) {
        unsafe { hos_peft_destroy(self.p) }
    }
}

/// Stub resident runner (`src/metal_be_stub.rs:210-236`): the inference path is not part of this backend.
pub struct GpuRunner;

impl GpuRunner {
    pub fn new(_gpu: Gpu, _model: &Model) -> GpuRunner {
        unreachable!("{NOT_HERE}")
    }
    pub fn forward(&self, _model: &Model, _token: u32, _pos: usize) -> Vec<f32> {
        unreachable!("{NOT_HERE}")
    }
    pub fn prefill_step(&self, _model: &Model, _token: u32, _pos: usize) {
        unreachable!("{NOT_HERE}")
    }
    pub fn max_batch(&self) -> usize {
        1
    }
    pub fn forward_prefill_gpu(&self, _model: &Model, _tokens: &[u32], _pos0: usize) -> Option<Vec<f32>> {
        unreachable!("{NOT_HERE}")
    }
}

/// No-op autorelease wrapper (no Metal objects to drain).
pub fn autorelease<R>(f: impl FnOnce() -> R) -> R {
    f()
}
