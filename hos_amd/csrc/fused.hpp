// Launchers of the fused bandwidth-bound kernels and attention (fused.hip, attention.hip).
#pragma once
#include "kernels.hpp"

namespace hos {
void launch_embed(const QWeight& table, const int32_t* ids, float* x, int M, int d, hipStream_t st);
// src.splits > 0: x is first formed (and stored) from a split GEMM's deferred partials, as its reduction would.
void launch_rmsnorm_fwd(float* x, const float* w, float eps, int M, int d, float* xn, H16 out, float* inv,
                        hipStream_t st, SplitSrc src = SplitSrc{});
// out.data != null: also write dx's fp16 GEMM operand (as launch_to_h16 would). src.splits > 0: the incoming
// gradient g is formed from a split GEMM's deferred partials (g is then only written on the general path).
// dx_in != null: dx = dx_in + the input gradient (dx_in is left as it was) instead of dx += it.
void launch_rmsnorm_bwd(float* g, const float* x, const float* inv, const float* w, int M, int d, float* dx,
                        hipStream_t st, H16 out = H16{nullptr, nullptr, nullptr}, SplitSrc src = SplitSrc{},
                        const float* dx_in = nullptr);
void launch_rope(float* buf, long long ld, int col0, int n_heads, int hd, int T, const float2* tab, bool neox,
                 bool inverse, int M, hipStream_t st);
// RoPE (col0 = 0) fused with the fp16 row operand of the first W columns (row stride W), as launch_rope
// followed by the f32 -> fp16 row conversion.
// After a launch_attn_bwd with defer_group_sum: per row of dqkv, dK/dV summed over each GQA group from `part`, the
// inverse RoPE of the q and k heads (k right after q), the row stored back and written as the fp16 operand of its
// first W columns (W <= kAttnRowsMax). Equal to attn_group_sum + launch_rope_h16 (inverse) element for element.
constexpr int kAttnRowsMax = 4096;
void launch_attn_bwd_rows(float* dqkv, long long ld, int hd, int nh, int nkv, int vcol, const float* part, int T,
                          const float2* tab, bool neox, int M, int W, H16 out, hipStream_t st);
void launch_rope_h16(float* buf, long long ld, int n_heads, int hd, int T, const float2* tab, bool neox, bool inverse,
                     int M, int W, H16 out, hipStream_t st);
void launch_swiglu_fwd(const float* gu, int M, int F, float* h, H16 out, hipStream_t st);
void launch_swiglu_bwd(const float* gu, const float* dh, int M, int F, float* dgu, H16 out, hipStream_t st);
// dl32 != null: write the gradient as plain f32 there instead of the fp16 operand dl. rstat != null: the row's
// (max, exp-sum) per 64-column chunk, from the epilogue of the GEMM that wrote the logits (one read of them less).
void launch_ce(const float* logits, int M, int V, const int32_t* targets, float gscale, float* row_loss, H16 dl,
               hipStream_t st, float* dl32 = nullptr, const float2* rstat = nullptr);
void launch_loss_reduce(const float* row_loss, int B, int T, float* loss, hipStream_t st);
void launch_adamw(float* p, const float* g, float* m, float* v, long long n, float lr, float b1, float b2, float eps,
                  float wd, float bc1, float bc2, bool decay, hipStream_t st);
// AdamW hyper-parameters in device memory: lr, decoupled weight decay, 1-based step count.
struct AdamHyper {
  float lr, wd;
  int t, pad;
};
void launch_adam_tick(AdamHyper* h, hipStream_t st);
void launch_adamw_dev(float* p, const float* g, float* m, float* v, long long n, float b1, float b2, float eps,
                      const AdamHyper* h, bool decay, hipStream_t st);
void launch_fill(float* p, long long n, float v, hipStream_t st);
void launch_copy_rows(const float* src, long long lds, float* dst, long long ldd, int rows, int cols,
                      hipStream_t st);
// Attention (attention.hip). `scratch` holds the bf16 hi/lo planes of q, k and v: attn_scratch_bytes(...)
// bytes, 16-byte aligned; its contents need not survive between the calls — except that a backward with
// qkv_planes = true reuses the q, k, v planes the forward of the same qkv left in the same scratch.
size_t attn_scratch_bytes(int B, int T, int nh, int nkv, int hd);
// rope_tab set: q and k are rotated (RoPE, forward) on their way into the planes; qkv stays unrotated.
void launch_attn_fwd(const float* qkv, long long ld, int kcol, int vcol, int B, int T, int nh, int nkv, int hd,
                     float* o, long long ldo, float* lse, void* scratch, hipStream_t st,
                     const float2* rope_tab = nullptr, bool rope_neox = false);
void launch_attn_bwd(const float* qkv, long long ld, int kcol, int vcol, const float* o, const float* dout,
                     long long ldo, const float* lse, float* dvec, int B, int T, int nh, int nkv, int hd, float* dqkv,
                     long long ldd, float* part, void* scratch, hipStream_t st, bool qkv_planes = false,
                     bool defer_group_sum = false);
}  // namespace hos
