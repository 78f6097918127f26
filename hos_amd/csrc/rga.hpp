// RGA adapter kernels (rga.hip).
#pragma once
#include "kernels.hpp"

namespace hos {

constexpr int RGA_GLEN = 8;        // genome length (src/peft.rs:201)
constexpr int RGA_MAX_GENES = 64;  // genes per layer supported by the small kernels

// gb[k] = genome · wg[:, k]
void launch_rga_bias(const float* genome, const float* wg, int K, float* gb, hipStream_t st);
// Z [M][ldz] (gate logits | bottleneck pre-activations) → A (sigmoid gates | relu), Hg [M][ldh] = H ⊙ gate,
// gsum[m] = Σ_k gate
void launch_rga_act_fwd(const float* Z, int ldz, int M, int K, int b, const float* gb, float* A, float* Hg, int ldh,
                        float* gsum, hipStream_t st);
// dG = dX·Upᵀ → dZ [M][ldz]; pc = the sparsity term's gradient per gate element
void launch_rga_act_bwd(const float* A, int ldz, const float* dG, int ldh, int M, int K, int b, float pc, float* dZ,
                        hipStream_t st);
// out[k] = Σ_m dZ[m][k], k < K (deterministic)
void launch_rga_colsum(const float* dZ, int ldz, int M, int K, float* out, hipStream_t st);
// gradients of wg [8][K] and genome [8] from the per-layer gate-bias gradients dgb [L][K]
void launch_rga_genome_grad(const float* genome, const float* wg, const float* dgb, int L, int K, float* gwg,
                            float* ggen, hipStream_t st);
// loss += Σ_b (1/B)·(λ/L)·Σ_l mean(gate_l over sequence b); gsum: layer l's row sums at gsum + l·ldl;
// gm: scratch for the L·B means
void launch_rga_loss(const float* gsum, long long ldl, int L, int B, int T, int K, float lambda, float* gm,
                     float* loss, hipStream_t st);

}  // namespace hos
