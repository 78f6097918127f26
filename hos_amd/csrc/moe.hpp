// Mixture-of-experts routing / combine kernels and OLMoE's QK-norm (launchers; see moe.hip).
#pragma once
#include "kernels.hpp"

namespace hos {

// In-place RMSNorm of the n columns starting at col0 of each of M rows (row stride ld): the pre-norm
// values go to pre [M][n], 1/rms to inv [M]. Backward: g (same place) ← ∂/∂x of the normed output.
void launch_qknorm_fwd(float* buf, long long ld, int col0, int n, const float* w, float eps, int M, float* pre,
                       float* inv, hipStream_t st);
void launch_qknorm_bwd(float* g, long long ld, int col0, int n, const float* w, const float* pre, const float* inv,
                       int M, hipStream_t st);

// Router: per row of logits [M][E] the softmax p (→ pfull), the top K by probability (ties: lower expert),
// sel_e / sel_p [M][K] in selection order, each selection's slot in its expert's list (its rank among the
// expert's selections in selection order) and counts[E], the per-expert totals.
void launch_moe_route(const float* logits, int M, int E, int K, float* pfull, int* sel_e, float* sel_p, int* slot,
                      int* counts, hipStream_t st);
// Per-expert offsets and the grouped-GEMM tile schedule (GROUP_BM-row tiles, max_tiles entries, unused = −1).
void launch_moe_plan(const int* counts, int E, int* offsets, int* tiles, int max_tiles, hipStream_t st);
// pos[t][s] = offsets[e] + slot; the H16 rows of the selected tokens gathered into expert order.
void launch_moe_gather(H16 src, long long lds, const int* sel_e, const int* slot, const int* offsets, int M, int K,
                       int d, int* pos, H16 dst, long long ldd, hipStream_t st);
// out[t] = resid[t] + Σ_s sel_p[t][s]·Y[pos[t][s]] (selection order).
void launch_moe_combine(const float* Y, const int* pos, const float* sel_p, const float* resid, int M, int K, int d,
                        float* out, hipStream_t st);
// Backward of the combine: dY[pos] = sel_p·g[t] (f32 rows), dp[t][s] = g[t]·Y[pos].
void launch_moe_combine_bwd(const float* g, const float* Y, const int* pos, const float* sel_p, int M, int K, int d,
                            float* dY, float* dp, hipStream_t st);
// The same with dY written as the fp16 row-scaled GEMM operand at row pos (what the f32 → fp16 conversion of
// the f32 dY gives); for d % 4 == 0, d <= 4096 (moe_combine_bwd_h16_ok).
bool moe_combine_bwd_h16_ok(int d);
void launch_moe_combine_bwd_h16(const float* g, const float* Y, const int* pos, const float* sel_p, int M, int K,
                                int d, H16 out, float* dp, hipStream_t st);
// Softmax backward restricted to the selected probabilities: dlogits[t][j] = p_j·(dp_j − Σ_i p_i·dp_i),
// dp_j = dp[t][s] for j = sel_e[t][s], else 0.
void launch_moe_router_bwd(const float* pfull, const float* dp, const int* sel_e, int M, int E, int K, float* dlogits,
                           hipStream_t st);
// dxn[t] = Σ_s dX[pos[t][s]] (selection order).
void launch_moe_gather_sum(const float* dX, const int* pos, int M, int K, int d, float* dxn, hipStream_t st);
// Zero n ints (graph-capturable; no memset nodes).
void launch_fill_i32(int* p, long long n, int v, hipStream_t st);

}  // namespace hos
