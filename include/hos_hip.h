/*
 * hos_hip.h — C ABI of the MI355X (gfx950) backend for HOS's LoRA fine-tuning path.
 *
 * The reference reaches its GPU through the Rust `Gpu` method set that src/tensor.rs
 * calls (src/metal_be_stub.rs:35-208, implemented by src/metal_be.rs). This header is
 * the same surface as a plain C ABI (plain pointers and sizes, no torch types), plus
 * the quantized-weight GEMMs and the device-resident LoRA training step that the
 * reference runs on the CPU (src/peft.rs, src/tensor.rs, src/main.rs:2583-2601).
 *
 * Conventions
 *  - Every entry point returns an int status: HOS_OK (0) or an HOS_E_* code; the
 *    message is in hos_hip_last_error(ctx). Codes 1-7 mirror HosError
 *    (src/error.rs:12-27); the reference panics at this boundary instead, and the
 *    Rust shim (hip_be.rs) turns a non-zero status back into a panic.
 *  - Host pointers are caller-owned and only read/written during the call. Device
 *    memory is owned by the library (keyed caches, the training model) or by the
 *    caller when it comes from hos_hip_dev_alloc.
 *  - A context is bound to one device and one thread, like the reference's
 *    thread-local Gpu (src/tensor.rs:30-32). Calls are synchronous unless the name
 *    ends in _dev / _async (those enqueue on the context's stream).
 *  - ggml_type values are GGUF ids (src/gguf.rs:22-30): 0 F32, 8 Q8_0, 12 Q4_K, 14 Q6_K.
 */
#ifndef HOS_HIP_H
#define HOS_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  HOS_OK = 0,
  HOS_E_IO = 1,                /* HosError::Io */
  HOS_E_FORMAT = 2,            /* HosError::Format */
  HOS_E_MISSING_TENSOR = 3,    /* HosError::MissingTensor */
  HOS_E_UNSUPPORTED_QUANT = 4, /* HosError::UnsupportedQuant */
  HOS_E_UNSUPPORTED_ARCH = 5,  /* HosError::UnsupportedArch */
  HOS_E_MISSING_META = 6,      /* HosError::MissingMeta */
  HOS_E_SPEC = 7,              /* HosError::Spec */
  HOS_E_DEVICE = 8,            /* HIP runtime failure */
  HOS_E_INVALID = 9,           /* bad argument: null pointer, shape, unknown key */
  HOS_E_OOM = 10               /* device allocation failed */
};

typedef struct hos_ctx hos_ctx;

/* ---- context: Gpu::new (src/metal_be_stub.rs:36-38, src/metal_be.rs:1942-1954) ---- */
int hos_hip_create(int device, hos_ctx** out);
void hos_hip_destroy(hos_ctx* ctx);
const char* hos_hip_last_error(const hos_ctx* ctx);
int hos_hip_synchronize(hos_ctx* ctx);
/* gfx arch name of the context's device, e.g. "gfx950". */
int hos_hip_device_arch(hos_ctx* ctx, char* buf, size_t len);

/* ---- keyed f32 GEMMs: the training matmuls of src/tensor.rs:53-97 ----
 * matmul_f32_keyed  C[m,n] = A[m,k]·B[k,n]          src/metal_be_stub.rs:108-118, metal_be.rs:2434-2446
 * matmul_abt_keyed  C[m,k] = A[m,n]·B[k,n]ᵀ         src/metal_be_stub.rs:119-129, metal_be.rs:2338-2351
 * matmul_atb_keyed  C[k,n] = A[m,k]ᵀ·B[m,n]         src/metal_be_stub.rs:130-140, metal_be.rs:2353-2366
 * key != 0 caches that operand on the device under the key (a frozen weight), like
 * buf_keyed (src/metal_be.rs:2322-2334); key == 0 means "no caching" (None). */
int hos_hip_matmul_f32_keyed(hos_ctx* ctx, const float* a, size_t m, size_t k, const float* b, size_t n,
                             uint64_t b_key, float* out);
int hos_hip_matmul_abt_keyed(hos_ctx* ctx, const float* a, size_t m, size_t n, const float* b, size_t k,
                             uint64_t b_key, float* out);
int hos_hip_matmul_atb_keyed(hos_ctx* ctx, const float* a, size_t k, size_t m, const float* b, size_t n,
                             uint64_t a_key, float* out);
/* Gpu::evict / Gpu::clear_cache (src/metal_be.rs:2416-2428). Evicting an absent key is a no-op. */
int hos_hip_evict(hos_ctx* ctx, uint64_t key);
int hos_hip_clear_cache(hos_ctx* ctx);

/* ---- quantized frozen weights ----
 * upload_quant: Gpu::upload_quant (src/metal_be_stub.rs:45-53). `bytes` is one GGUF
 * tensor [rows, cols] row-major (cols % block == 0). Repacked once on the device. */
int hos_hip_upload_quant(hos_ctx* ctx, uint64_t key, const uint8_t* bytes, size_t nbytes, uint32_t ggml_type,
                         size_t rows, size_t cols);
/* Bit-exact Gguf::dequant_into (src/gguf.rs:330-505) of an uploaded weight, computed by the
 * same device function the GEMMs use. out: rows·cols floats (host). */
int hos_hip_dequant(hos_ctx* ctx, uint64_t key, float* out);
/* Y[t, rows] = X[t, cols]·deq(W)ᵀ — the frozen-base forward x·t_const(W) (src/peft.rs:24-33,
 * src/tensor.rs:316-327). Host pointers. */
int hos_hip_qgemm_fwd(hos_ctx* ctx, uint64_t key, const float* x, size_t t, float* y);
/* dX[t, cols] = dY[t, rows]·deq(W) — the frozen-base backward dA = g·Bᵀ (src/tensor.rs:347-360). */
int hos_hip_qgemm_dx(hos_ctx* ctx, uint64_t key, const float* dy, size_t t, float* dx);
/* Device-pointer variants (no host copies; enqueue + return). */
int hos_hip_qgemm_fwd_dev(hos_ctx* ctx, uint64_t key, const float* x_dev, size_t t, float* y_dev);
int hos_hip_qgemm_dx_dev(hos_ctx* ctx, uint64_t key, const float* dy_dev, size_t t, float* dx_dev);
/* A frozen-base GEMM with its LoRA term fused in the epilogue — the adapted linear of src/peft.rs:508-512
 * (base + s·(x·A)·B) and its input gradient (dY·W + du·Aᵀ): out[t, N] = op(in, deq(W)) + scale·U·L with
 * which 0: op = in·deq(W)ᵀ (N = rows), 1: op = in·deq(W) (N = cols); U [t, rank] with row stride ldu,
 * L(j, n) = l[j·slj + n·sln]. Device pointers; 1 <= rank <= 128. */
int hos_hip_qgemm_lora_dev(hos_ctx* ctx, int which, uint64_t key, const float* in_dev, size_t t, const float* u_dev,
                           size_t ldu, const float* l_dev, size_t slj, size_t sln, int rank, float scale,
                           float* out_dev);
/* Time `iters` launches of the fp16-MFMA GEMM kernel alone (which: 0 fwd, 1 dx) on an input
 * already converted to the fp16 row-scaled operand, with HIP events on the context stream.
 * Returns the mean kernel time in ms. */
int hos_hip_time_qgemm(hos_ctx* ctx, int which, uint64_t key, const float* in_dev, size_t t, float* out_dev,
                       int iters, float* avg_ms);
/* Elapsed time of whatever is enqueued on the context stream between the two calls, from HIP events
 * (timer_end waits for the stream; it fails with HOS_E_INVALID unless a timer_begin is open, so each end pairs with
 * exactly one begin). No counterpart in the reference; measurement only. */
int hos_hip_timer_begin(hos_ctx* ctx);
int hos_hip_timer_end(hos_ctx* ctx, float* ms);
/* quantize(x, ggml_type) of src/gguf_write.rs:41-50 (Q8_0 :178-196, Q4_K :355-416,
 * Q6_K :426-495), run on the device; byte-identical to the reference encoders.
 * x: n floats (host), out: bytes_for(type, n) bytes (host). */
int hos_hip_quantize(hos_ctx* ctx, const float* x, size_t n, uint32_t ggml_type, uint8_t* out);
/* hos_hip_quantize on device buffers (x_dev f32 [n] -> out_dev, hos_hip_bytes_for(type, n) bytes). */
int hos_hip_quantize_dev(hos_ctx* ctx, const float* x_dev, size_t n, uint32_t ggml_type, uint8_t* out_dev);
/* Synthetic data: n samples of N(0, stddev^2) into out_dev from a counter-based hash of (seed, index);
 * no counterpart in the reference (its Tensor::randn is a host xorshift). */
int hos_hip_randn_dev(hos_ctx* ctx, float* out_dev, size_t n, uint64_t seed, float stddev);
/* Precision of this context's qGEMMs: 1 = single fp16 pass (both operands rounded to 11 bits),
 * 2 = activation carried as fp16 hi + lo (2 MFMA passes), 3 = weight split too (3 passes),
 * 4 = weight carried as fp16 hi + lo, activation rounded once (2 passes), 5 = the precision of 3 by the faster
 * kernel for the launch: two passes against the exact integer codes (block scales applied in f32) for large
 * forward GEMMs on Q8_0, Q4_0 and Q5_0 weights, else mode 3.
 * Default 1.
 * (The reference has no counterpart: its GPU GEMMs are f32, src/metal_be.rs:1095-1142.) */
int hos_hip_set_gemm_passes(hos_ctx* ctx, int passes);
/* bytes_for (src/gguf.rs:548-561); 0 for an unsupported type. */
size_t hos_hip_bytes_for(uint32_t ggml_type, size_t n);

/* ---- op-level entry points: one per fused kernel of the training path, device pointers, enqueued on
 * the context stream (hos_hip_synchronize waits). Each is one of the reference's autograd ops
 * (src/tensor.rs) with its VJP; the training step below schedules the same kernels. ---- */
/* embedding (src/tensor.rs:2438-2457): out[r] = deq(table)[ids[r]], table uploaded under `key`. */
int hos_hip_embedding(hos_ctx* ctx, uint64_t key, const int32_t* ids_dev, size_t rows, float* out_dev);
/* rmsnorm_eps (src/tensor.rs:2500-2544): y = x·inv·w with inv = 1/sqrt(mean(x²)+eps) per row, and the
 * input gradient gx = g·w·inv − inv³·x/d·Σ(g·w·x) (norm weights are frozen in PEFT: no weight gradient). */
int hos_hip_rmsnorm_fwd(hos_ctx* ctx, const float* x, const float* w, size_t rows, size_t d, float eps, float* y,
                        float* inv);
int hos_hip_rmsnorm_bwd(hos_ctx* ctx, const float* g, const float* x, const float* inv, const float* w, size_t rows,
                        size_t d, float* gx);
/* rope (src/tensor.rs:2750-2814), in place on n_heads heads of head_dim at column col0 of rows [rows, ld];
 * position = row % seq_len; inverse != 0 applies the transpose rotation (the backward). */
int hos_hip_rope(hos_ctx* ctx, float* x, size_t rows, size_t ld, size_t col0, int n_heads, int head_dim, int seq_len,
                 float base, int neox, int inverse);
/* SwiGLU silu(gate)·up (src/tensor.rs:2082-2100, 458-480): gu rows [gate F | up F], h [rows, F]; backward
 * dgu rows [d gate | d up]. */
int hos_hip_swiglu_fwd(hos_ctx* ctx, const float* gu, size_t rows, size_t F, float* h);
int hos_hip_swiglu_bwd(hos_ctx* ctx, const float* gu, const float* dh, size_t rows, size_t F, float* dgu);
/* Causal GQA attention of PeftModel::forward (src/peft.rs:530-553; src/tensor.rs:2207-2280, 2460-2491) over
 * B sequences of T rows, head_dim 64: qkv rows [B·T, ld] with q heads at column 0, k at kcol, v at vcol;
 * o [B·T, ldo]; lse [B, n_heads, T] kept for the backward, which writes dq, dk, dv into dqkv (same layout). */
int hos_hip_attention_fwd(hos_ctx* ctx, const float* qkv, size_t ld, size_t kcol, size_t vcol, int B, int T,
                          int n_heads, int n_kv_heads, int head_dim, float* o, size_t ldo, float* lse);
int hos_hip_attention_bwd(hos_ctx* ctx, const float* qkv, size_t ld, size_t kcol, size_t vcol, const float* o,
                          const float* dout, size_t ldo, const float* lse, int B, int T, int n_heads, int n_kv_heads,
                          int head_dim, float* dqkv, size_t ldd);
/* cross_entropy (src/tensor.rs:2709-2743) per row: row_loss = −ln max(p_target, 1e−12),
 * dlogits = (p − onehot)·gscale (the reference's g/n: gscale = 1/rows). */
int hos_hip_cross_entropy(hos_ctx* ctx, const float* logits, size_t rows, size_t V, const int32_t* targets,
                          float gscale, float* row_loss, float* dlogits);
/* MoE router (src/forward.rs:542-552) on logits [rows, E] (E <= 64, 1 <= K <= E): softmax pfull [rows, E]; the top K
 * experts of each row by probability, ties to the lower expert (the reference's stable descending sort), with
 * their raw probabilities: sel_e / sel_p [rows, K] in selection order. slot [rows, K] = rank of the selection among
 * its expert's selections (token, then slot order); counts [E] = selections per expert. A NaN probability ranks
 * below every number, so every row still gets K distinct experts in [0, E). */
int hos_hip_moe_route(hos_ctx* ctx, const float* logits, size_t rows, int E, int K, float* pfull, int32_t* sel_e,
                      float* sel_p, int32_t* slot, int32_t* counts);
/* AdamW::step (src/tensor.rs:2952-2975) on n parameters at 1-based step t (bias corrections by f32 powi). */
int hos_hip_adamw(hos_ctx* ctx, float* p, const float* g, float* m, float* v, size_t n, float lr, float beta1,
                  float beta2, float eps, float wd, int step, int decay);
/* One LoRA branch y += s·(x·A)·B (src/peft.rs:508-512) and its backward (matmul VJPs, src/tensor.rs:340-391),
 * A [in, r], B [r, out] row-major, r <= 96: u = x·A, y += s·u·B (y may be NULL), dB = s·uᵀ·dy,
 * du = s·dy·Bᵀ, dA = xᵀ·du, dx += du·Aᵀ (dx may be NULL). */
int hos_hip_lora(hos_ctx* ctx, const float* x, const float* dy, size_t rows, size_t in, size_t out, int r,
                 const float* A, const float* B, float scale, float* y, float* u, float* dA, float* dB, float* dx);

/* hos_hip_lora without device allocation. No counterpart in the reference: it is for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Same arguments, kernels and results as hos_hip_lora; its scratch (A transposed, du, split partials) is one
 * 64 MiB device array per GPU, held until the process ends: shapes needing more fail with HOS_E_INVALID before
 * any launch. Every call on one GPU shares that array, so calls that overlap on one GPU (two streams or two
 * contexts) race; calls in one stream order are safe. The array's device address is looked up once per device,
 * so hipDeviceReset is not supported in a process that calls this entry point. */
int hos_hip_lora_noalloc(hos_ctx* ctx, const float* x, const float* dy, size_t rows, size_t in, size_t out, int r,
                         const float* A, const float* B, float scale, float* y, float* u, float* dA, float* dB,
                         float* dx);

/* ---- device memory (GpuBuf / download_buf analogue, src/metal_be_stub.rs:13-20) ---- */
int hos_hip_dev_alloc(hos_ctx* ctx, size_t nbytes, void** dptr);
int hos_hip_dev_free(hos_ctx* ctx, void* dptr);
int hos_hip_h2d(hos_ctx* ctx, void* dst_dev, const void* src_host, size_t nbytes);
int hos_hip_d2h(hos_ctx* ctx, void* dst_host, const void* src_dev, size_t nbytes);

/* ---- the LoRA training model: PeftModel (src/peft.rs) + AdamW (src/tensor.rs:2923-2976) ----
 * Llama/Qwen2-family decoder with a frozen quantized base and LoRA on the selected
 * projections. The reference adapts q and v only (src/peft.rs:52-59, 508-512); targets
 * extend that the same way (y += (x·A·B)·α/r after the base projection). */
enum {
  HOS_T_Q = 1,
  HOS_T_K = 2,
  HOS_T_V = 4,
  HOS_T_O = 8,
  HOS_T_GATE = 16,
  HOS_T_UP = 32,
  HOS_T_DOWN = 64
};

/* Config: src/model.rs:622-644 (Config) + src/peft.rs:121-126 (PeftCfg). */
typedef struct {
  int n_layers, dim, n_heads, n_kv_heads, head_dim, ffn_dim, vocab;
  float rms_eps, rope_base;
  int rope_neox, attn_bias;
  int lora_rank;
  float lora_alpha;
  uint32_t lora_targets;
  int max_batch, max_seq; /* sizes the device-resident activation arena */
  int gemm_passes;        /* qGEMM precision mode for every GEMM, as hos_hip_set_gemm_passes; 0 = default
                           * policy: layer forward 5, layer dX 3, head forward 1, head dX 4 */
  /* Mixture-of-experts FFN (src/model.rs:642-643; OLMoE): n_experts stacked SwiGLU experts
   * (blk.N.ffn_{gate,up,down}_exps.weight) behind an f32 router (blk.N.ffn_gate_inp.weight), top
   * n_experts_used by softmax probability, raw probabilities as weights (src/forward.rs:542-572).
   * 0 = dense FFN. LoRA targets gate/up/down are not allowed with experts. */
  int n_experts, n_experts_used;
  /* RMSNorm of the full q / k projections before RoPE (blk.N.attn_{q,k}_norm.weight, src/forward.rs:487-493) */
  int qk_norm;
  /* RGA adapters instead of LoRA (PeftModel "rga", src/peft.rs:61-96, 200-215, 565-584) when rga_genes > 0:
   * per layer, after the FFN, x += Σ_k sigmoid(x·W_r + genome·W_g)[:, k] ⊙ relu(x·down_k)·up_k, with
   * rga_genes genes of bottleneck rga_bottleneck and one genome; the loss adds (rga_lambda / L)·Σ_l mean(gate_l)
   * per sequence (loss_g, src/peft.rs:447-459). lora_targets must be 0 and n_experts 0 (the reference's PEFT
   * refuses mixture-of-experts models). Parameters are set and read by name (hos_peft_set_adapter). */
  int rga_genes, rga_bottleneck;
  float rga_lambda;
} hos_peft_cfg;

typedef struct hos_peft hos_peft;

/* PeftModel::build_multi (src/peft.rs:134-231): allocates the model on ctx's device. */
int hos_peft_create(hos_ctx* ctx, const hos_peft_cfg* cfg, hos_peft** out);
void hos_peft_destroy(hos_peft* p);
const char* hos_peft_last_error(const hos_peft* p);
/* One GGUF tensor by its GGUF name (src/model.rs:713-921): token_embd.weight, output.weight
 * (absent = tied to token_embd), output_norm.weight, blk.N.{attn_norm, attn_q, attn_k, attn_v,
 * attn_output, ffn_norm, ffn_gate, ffn_up, ffn_down}.weight, blk.N.attn_{q,k,v}.bias.
 * Norm weights and biases: F32. Linear weights: Q8_0, Q4_K or Q6_K. With n_experts > 0 the FFN tensors are
 * blk.N.ffn_gate_inp.weight (F32 [E, dim]) and blk.N.ffn_{gate,up,down}_exps.weight ([E·ffn, dim],
 * [E·ffn, dim], [E·dim, ffn]); with qk_norm, blk.N.attn_q_norm.weight / attn_k_norm.weight (F32). */
int hos_peft_set_tensor(hos_peft* p, const char* name, const uint8_t* bytes, size_t nbytes, uint32_t ggml_type,
                        size_t rows, size_t cols);
/* Model::load (src/model.rs:713-921) over the GGUF reader (src/gguf.rs:225-286): parses the file at path,
 * maps {arch}.embedding_length / block_count / attention.head_count[_kv] / feed_forward_length /
 * attention.layer_norm_rms_epsilon / rope.freq_base / attention.key_length | rope.dimension_count to the
 * model fields of *cfg (vocab from token_embd, attn_bias from blk.0.attn_q.bias, NEOX RoPE for qwen2),
 * keeping cfg's LoRA / arena fields as given. No device work; err (may be NULL) receives the message. */
int hos_gguf_config(const char* path, hos_peft_cfg* cfg, char* err, size_t err_len);
/* hos_gguf_config + hos_peft_create + hos_peft_set_tensor for every model tensor in the file. train
 * supplies the LoRA / arena fields; out_cfg (may be NULL) receives the mapped config. Architectures:
 * llama, qwen2, mistral; linear weights Q8_0 / Q4_K / Q6_K (else HOS_E_UNSUPPORTED_QUANT); 1-D F16 / BF16
 * tensors are widened to F32. */
int hos_peft_create_from_gguf(hos_ctx* ctx, const char* path, const hos_peft_cfg* train, hos_peft** out,
                              hos_peft_cfg* out_cfg);
/* LoRA factors of one (layer, target index 0..6 = q,k,v,o,gate,up,down), reference layout:
 * A [in, r], B [r, out] row-major (src/peft.rs:187-199). */
int hos_peft_set_lora(hos_peft* p, int layer, int target, const float* A, const float* B);
int hos_peft_get_lora(hos_peft* p, int layer, int target, float* A, float* B);
int hos_peft_get_lora_grad(hos_peft* p, int layer, int target, float* dA, float* dB);
/* An RGA parameter by its adapter tensor name and reference layout (PeftModel::adapter_tensors,
 * src/peft.rs:741-760): genome.0 [1, 8], wg [8, genes], rga.{l}.wr [dim, genes], rga.{l}.down.{k}
 * [dim, bottleneck], rga.{l}.up.{k} [bottleneck, dim]; n = the tensor's element count (else HOS_E_INVALID).
 * get: value and/or grad (either may be NULL). */
int hos_peft_set_adapter(hos_peft* p, const char* name, const float* data, size_t n);
int hos_peft_get_adapter(hos_peft* p, const char* name, float* value, float* grad, size_t n);
/* zero_grad + for each of B sequences: loss(seq)·(1/B), backward (src/main.rs:2583-2596,
 * src/train.rs:33-52). ids/targets: [B, T] int32 (host). *loss = Σ_b loss_b / B. */
int hos_peft_loss_grad(hos_peft* p, const int32_t* ids, const int32_t* targets, int B, int T, float* loss);
/* AdamW::step over all LoRA factors (β 0.9/0.95, eps 1e-8, decay on 2-D params). */
int hos_peft_adamw(hos_peft* p, float lr, float wd);
/* One optimizer step (loss_grad + adamw) on device-resident ids/targets; enqueues only.
 * loss_dev receives the step's loss (one float, device). */
int hos_peft_step_dev(hos_peft* p, const int32_t* ids_dev, const int32_t* targets_dev, int B, int T, float lr,
                      float wd, float* loss_dev);
/* hos_peft_step_dev replays a captured HIP graph of the whole step after its first call for a given
 * (B, T, ids, targets, loss) pointer set (default on; off = enqueue kernel by kernel). Profiling
 * (hos_peft_profile) always runs the step kernel by kernel. */
int hos_peft_use_graph(hos_peft* p, int enable);
/* Adapter / optimizer checkpoint in the .hos capsule layout (src/format.rs:1-26, writer :287-346,
 * reader :401-485; version 2, every tensor F32 with its FNV-1a 64 checksum, file checksum last).
 * Tensors: lora.{l}.a{t} [in, r] and lora.{l}.b{t} [r, out] (ROLE_WEIGHT) for every adapted target t in
 * q,k,v,o,gate,up,down order (PeftModel::adapter_tensors, src/peft.rs:731-740, whose q|v model writes
 * lora.{l}.{aq,bq,av,bv}); with_optimizer adds opt.m.{k} / opt.v.{k} (ROLE_OPT_STATE, the k-th parameter
 * in that order) and the scalars opt.step, opt.lr, opt.beta1, opt.beta2, opt.wd (ROLE_SCALAR), as the
 * lifecycle checkpoint of src/main.rs:6276-6307. card_json is stored verbatim; NULL writes a default
 * adapter card (Card::new + mode "adapter", id = hos_peft_adapter_id, resume.step = AdamW steps). */
int hos_peft_save_hos(hos_peft* p, const char* path, const char* card_json, int with_optimizer);
/* Inverse of hos_peft_save_hos (v1 and v2 files). Every adapted target's factors must be present with the
 * model's shapes (else HOS_E_MISSING_TENSOR / HOS_E_FORMAT); other tensors are ignored. Checksums are
 * verified; a failing file leaves the model unchanged. with_optimizer also restores m, v, the step count,
 * lr and wd (without it the optimizer state is left as it is). */
int hos_peft_load_hos(hos_peft* p, const char* path, int with_optimizer);
/* model_id (src/format.rs:100-111) of the adapter tensors: FNV-1a 64 over their f32 bytes, 16 hex digits
 * plus NUL into out17. */
int hos_peft_adapter_id(hos_peft* p, char* out17);
/* The base model's id as save_adapter records it (src/main.rs:2641-2646): FNV-1a 64 of the dequantized
 * f32 token embedding. */
int hos_peft_base_id(hos_peft* p, char* out17);
/* read_card (src/format.rs:270-285): the card JSON of a .hos file into out (NUL-terminated, truncated to
 * len); *needed (may be NULL) = its length + 1. On error out receives the message. No device work. */
int hos_format_card(const char* path, char* out, size_t len, size_t* needed);
/* load_raw (src/format.rs:401-485) without a model: parse the header, card and tensor table and verify every
 * tensor's checksum (and the F32 byte counts); *n_tensors (may be NULL) = the table size. No device work. */
int hos_format_verify(const char* path, size_t* n_tensors, char* err, size_t err_len);
/* ---- full-parameter finetune (FtModel, src/finetune.rs) ----
 * Every weight a trainable f32 parameter on the device: quantized tensors are dequantized once at load
 * (Weight::to_f32); a tied head becomes an untied copy of the embedding (src/finetune.rs:101-107). Dense
 * Llama family only (n_experts = 0, qk_norm = 0; the LoRA fields of the config are ignored). Weight GEMMs
 * in f32 (fp32 MFMA), weight gradients dW = dYᵀ·X (the matmul_atb of src/metal_be.rs:1212-1234). */
typedef struct hos_ft hos_ft;
int hos_ft_create(hos_ctx* ctx, const hos_peft_cfg* cfg, hos_ft** out);
void hos_ft_destroy(hos_ft* p);
const char* hos_ft_last_error(const hos_ft* p);
/* Same GGUF names as hos_peft_set_tensor; F32 or Q8_0 / Q4_K / Q6_K. */
int hos_ft_set_tensor(hos_ft* p, const char* name, const uint8_t* bytes, size_t nbytes, uint32_t ggml_type,
                      size_t rows, size_t cols);
/* Current value and gradient of one parameter by GGUF name, GGUF layout ([out, in] row-major); either
 * pointer may be NULL. */
int hos_ft_get(hos_ft* p, const char* name, float* value, float* grad);
/* zero_grad + B sequences, loss·(1/B) each (the accumulation of src/main.rs:2834-2855). */
int hos_ft_loss_grad(hos_ft* p, const int32_t* ids, const int32_t* targets, int B, int T, float* loss);
/* AdamW::step over FtModel::params (β 0.9/0.95, eps 1e-8, decay on 2-D tensors, src/main.rs:2803-2804). */
int hos_ft_adamw(hos_ft* p, float lr, float wd);
/* loss_grad + adamw on device-resident ids/targets; enqueues only. */
int hos_ft_step_dev(hos_ft* p, const int32_t* ids_dev, const int32_t* targets_dev, int B, int T, float lr, float wd,
                    float* loss_dev);
/* Logits [T, vocab] of one sequence (PeftModel::logits, src/peft.rs:462-464). */
int hos_peft_logits(hos_peft* p, const int32_t* ids, int T, float* out);
/* Per-kernel-class timing with HIP events around every launch (off by default). */
int hos_peft_profile(hos_peft* p, int enable);
/* Restrict the timing to one kernel class (NULL or "" = all classes). */
int hos_peft_profile_only(hos_peft* p, const char* cls);
/* Accumulated stats of one kernel class since profiling was enabled: launches, total ms,
 * algorithmic flops and HBM bytes. Classes: "qgemm_fwd", "qgemm_dx", "lora_down", "lora_db", "lora_du", "lora_da", "attn_fwd",
 * "attn_bwd", "rmsnorm", "swiglu", "rope", "ce", "adamw", "embed", "convert". */
int hos_peft_kernel_stats(hos_peft* p, const char* cls, long long* launches, double* total_ms, double* flops,
                          double* bytes);

#ifdef __cplusplus
}
#endif
#endif /* HOS_HIP_H */
