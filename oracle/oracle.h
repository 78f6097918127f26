// ORACLE — test infrastructure only (the parity checker for the HIP backend).
// Nothing in the product library links or calls this; only tests/, the smoke check
// and bench.py's cpu_baseline leg load liboracle.so.
//
// A CPU restatement of HOS's CPU training path (Rust reference, not buildable in this
// image: no cargo/rustc). Each definition cites the reference file:line it follows.
#pragma once
#include <cstddef>
#include <cstdint>

// GGUF tensor type ids, src/gguf.rs:22-30.
enum {
  GGML_F32 = 0,
  GGML_F16 = 1,
  GGML_Q4_0 = 2,
  GGML_Q5_0 = 6,
  GGML_Q8_0 = 8,
  GGML_Q4_K = 12,
  GGML_Q5_K = 13,
  GGML_Q6_K = 14,
  GGML_BF16 = 30,
};

enum { ORC_OK = 0, ORC_E_UNSUPPORTED_QUANT = 4, ORC_E_INVALID = 9 };

namespace orc {
float f16_to_f32(uint16_t h);
uint16_t f32_to_f16(float f);
size_t bytes_for(uint32_t t, size_t n);
int dequant_into(const uint8_t* bytes, uint32_t t, size_t n, float* out);
int quantize(const float* x, size_t n, uint32_t t, uint8_t* out);
void pack_scales_mins(const uint8_t* scales, const uint8_t* mins, uint8_t* q);
void qkx_scale_min(const float* x, int len, int nmax, float* out_scale, float* out_min);
}  // namespace orc

// LoRA target bits (q, k, v, o, gate, up, down). The reference adapts q and v only
// (src/peft.rs:52-59, 508-512); the other bits extend it the same way.
enum {
  ORC_T_Q = 1,
  ORC_T_K = 2,
  ORC_T_V = 4,
  ORC_T_O = 8,
  ORC_T_GATE = 16,
  ORC_T_UP = 32,
  ORC_T_DOWN = 64,
};

// Model hyper-parameters: src/model.rs:622-644 (Config) + src/peft.rs:121-126 (PeftCfg).
typedef struct {
  int n_layers, dim, n_heads, n_kv_heads, head_dim, ffn_dim, vocab;
  float rms_eps, rope_base;
  int rope_neox, attn_bias;
  int lora_rank;
  float lora_alpha;
  uint32_t lora_targets;
  // Mixture-of-experts FFN (src/model.rs:642-643, 792-795; 0 = dense) and OLMoE's QK-norm
  // (src/model.rs:698-699, 872-873).
  int n_experts, n_experts_used, qk_norm;
  // RGA adapters instead of LoRA (src/peft.rs:61-96, 200-215; PeftCfg genes / bottleneck, src/peft.rs:121-126)
  // when rga_genes > 0 (lora_targets must then be 0); rga_lambda is the gate sparsity weight of loss_g
  // (src/peft.rs:447-459; cmd_peft's PEFT_LAMBDA, src/main.rs:2559-2562).
  int rga_genes, rga_bottleneck;
  float rga_lambda;
} orc_cfg;
