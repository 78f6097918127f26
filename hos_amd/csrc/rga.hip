// RGA adapters (Regulatory Genome Adapters, src/peft.rs:61-96): the element-wise and reduction kernels of
//   gate = sigmoid(x·W_r + genome·W_g)          [M, K]      (src/peft.rs:491-499, 567)
//   x   += Σ_k gate[:, k] ⊙ relu(x·down_k)·up_k             (src/peft.rs:568-576)
//   loss += (λ/L)·Σ_l mean(gate_l) per sequence              (src/peft.rs:447-459)
// and of their backward. The projections are skinny f32 GEMMs run by the LoRA kernels on the stacked factors
// RT = [W_rᵀ; down_0ᵀ; …; down_{K-1}ᵀ] ([R][d], R = K + K·b, rounded up to a multiple of 4 with zero rows) and
// Up = [up_0; …; up_{K-1}] ([K·b][d]); the gene sum is one GEMM (H ⊙ gate)·Up, the same sum as the
// reference's per-gene (H_k·up_k) ⊙ gate_k added in gene order, with the gate applied before the product.
#include <cmath>

#include "rga.hpp"

namespace hos {
namespace {

#pragma clang fp contract(off)

// gb[k] = Σ_i genome[i]·wg[i·K + k], i ascending (Tensor::matmul's order for [1, 8]·[8, K])
__global__ void rga_bias_kernel(const float* __restrict__ genome, const float* __restrict__ wg, int K,
                                float* __restrict__ gb) {
  const int k = threadIdx.x;
  if (k >= K) return;
  float s = 0.0f;
  for (int i = 0; i < RGA_GLEN; i++) s += genome[i] * wg[i * K + k];
  gb[k] = s;
}

// One thread per row: Z [M][ldz] = x·RTᵀ → A [M][ldz] (gates | relu'd bottlenecks, padding zeroed),
// Hg [M][ldh] = H ⊙ gate per gene block, gsum[m] = Σ_k gate (k ascending).
__global__ void rga_act_fwd_kernel(const float* __restrict__ Z, int ldz, int M, int K, int b,
                                   const float* __restrict__ gb, float* __restrict__ A, float* __restrict__ Hg, int ldh,
                                   float* __restrict__ gsum) {
  const int m = blockIdx.x * blockDim.x + threadIdx.x;
  if (m >= M) return;
  const float* z = Z + (long long)m * ldz;
  float* a = A + (long long)m * ldz;
  float* h = Hg + (long long)m * ldh;
  float s = 0.0f;
  for (int k = 0; k < K; k++) {
    const float g = 1.0f / (1.0f + expf(-(z[k] + gb[k])));  // src/tensor.rs:2103-2106
    a[k] = g;
    s += g;
    for (int j = 0; j < b; j++) {
      const int c = k * b + j;
      const float v = z[K + c];
      const float hv = v > 0.0f ? v : 0.0f;  // src/tensor.rs:482-485
      a[K + c] = hv;
      h[c] = hv * g;
    }
  }
  for (int c = K + K * b; c < ldz; c++) a[c] = 0.0f;
  for (int c = K * b; c < ldh; c++) h[c] = 0.0f;
  gsum[m] = s;
}

// One thread per row. dG [M][ldh] = dX·Upᵀ. d gate_k = Σ_j H_kj·dG_kj + pc (the sparsity term's share of each
// gate), dZ_gate = d gate·s(1 − s) (src/tensor.rs:2108-2113); dZ_down = gate_k·dG where the bottleneck was
// positive, else 0 (src/tensor.rs:487-494).
__global__ void rga_act_bwd_kernel(const float* __restrict__ A, int ldz, const float* __restrict__ dG, int ldh, int M,
                                   int K, int b, float pc, float* __restrict__ dZ) {
  const int m = blockIdx.x * blockDim.x + threadIdx.x;
  if (m >= M) return;
  const float* a = A + (long long)m * ldz;
  const float* g = dG + (long long)m * ldh;
  float* dz = dZ + (long long)m * ldz;
  for (int k = 0; k < K; k++) {
    const float s = a[k];
    float dg = 0.0f;
    for (int j = 0; j < b; j++) {
      const int c = k * b + j;
      const float hv = a[K + c];
      dg += hv * g[c];
      dz[K + c] = hv > 0.0f ? g[c] * s : 0.0f;
    }
    dg += pc;
    dz[k] = dg * s * (1.0f - s);
  }
  for (int c = K + K * b; c < ldz; c++) dz[c] = 0.0f;
}

// out[k] = Σ_m dZ[m][k] over all rows (the gate bias's broadcast-add backward), one workgroup per k with a
// fixed-order tree: deterministic.
__global__ void __launch_bounds__(256) rga_colsum_kernel(const float* __restrict__ dZ, int ldz, int M,
                                                         float* __restrict__ out) {
  __shared__ float part[256];
  const int k = blockIdx.x;
  float s = 0.0f;
  for (int m = threadIdx.x; m < M; m += 256) s += dZ[(long long)m * ldz + k];
  part[threadIdx.x] = s;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if (threadIdx.x < w) part[threadIdx.x] += part[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) out[k] = part[0];
}

// dgb = Σ_l dgb_l; d wg = genomeᵀ·dgb, d genome = dgb·wgᵀ (Tensor::matmul's backward for [1, 8]·[8, K]).
__global__ void rga_genome_grad_kernel(const float* __restrict__ genome, const float* __restrict__ wg,
                                       const float* __restrict__ dgb, int L, int K, float* __restrict__ gwg,
                                       float* __restrict__ ggen) {
  __shared__ float t[RGA_MAX_GENES];
  const int k = threadIdx.x;
  if (k < K) {
    float s = 0.0f;
    for (int l = 0; l < L; l++) s += dgb[l * K + k];
    t[k] = s;
  }
  __syncthreads();
  if (k < K)
    for (int i = 0; i < RGA_GLEN; i++) gwg[i * K + k] = genome[i] * t[k];
  if (k < RGA_GLEN) {
    float s = 0.0f;
    for (int j = 0; j < K; j++) s += t[j] * wg[k * K + j];
    ggen[k] = s;
  }
}

// gm[l·B + b] = mean over sequence b of layer l's T·K gates (gsum + l·ldl: row sums), one workgroup each with a
// fixed-order tree.
__global__ void __launch_bounds__(256) rga_gate_mean_kernel(const float* __restrict__ gsum, long long ldl, int B,
                                                            int T, int K, float* __restrict__ gm) {
  __shared__ float part[256];
  const int l = blockIdx.x / B, b = blockIdx.x % B;
  const float* g = gsum + (long long)l * ldl + (long long)b * T;
  float s = 0.0f;
  for (int i = threadIdx.x; i < T; i += 256) s += g[i];
  part[threadIdx.x] = s;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if (threadIdx.x < w) part[threadIdx.x] += part[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) gm[blockIdx.x] = part[0] / (float)(T * K);
}

// loss += Σ_b (1/B)·(λ/L)·Σ_l gm[l·B + b] (layers in order, as loss_g adds the gate means). The means are
// staged in LDS by the whole workgroup (LOSS_STAGE at a time, sequence-major) and summed in order by one thread.
constexpr int LOSS_STAGE = 2048;
__global__ void __launch_bounds__(256) rga_loss_kernel(const float* __restrict__ gm, int L, int B, float lambda,
                                                       float* __restrict__ loss) {
  __shared__ float buf[LOSS_STAGE];
  const int per = LOSS_STAGE / L;  // sequences per stage (L <= LOSS_STAGE, checked by the launcher)
  float tot = 0.0f;
  for (int b0 = 0; b0 < B; b0 += per) {
    const int nb = min(per, B - b0);
    __syncthreads();
    for (int i = threadIdx.x; i < nb * L; i += blockDim.x) {
      const int bb = i / L, l = i % L;
      buf[i] = gm[l * B + b0 + bb];
    }
    __syncthreads();
    if (threadIdx.x == 0)
      for (int bb = 0; bb < nb; bb++) {
        float sl = 0.0f;
        for (int l = 0; l < L; l++) sl += buf[bb * L + l];
        tot += sl * (lambda / (float)L) * (1.0f / (float)B);
      }
  }
  if (threadIdx.x == 0) loss[0] += tot;
}

}  // namespace

void launch_rga_bias(const float* genome, const float* wg, int K, float* gb, hipStream_t st) {
  rga_bias_kernel<<<1, 64, 0, st>>>(genome, wg, K, gb);
  HOS_HIP_CHECK(hipGetLastError());
}
void launch_rga_act_fwd(const float* Z, int ldz, int M, int K, int b, const float* gb, float* A, float* Hg, int ldh,
                        float* gsum, hipStream_t st) {
  rga_act_fwd_kernel<<<ceil_div(M, 64), 64, 0, st>>>(Z, ldz, M, K, b, gb, A, Hg, ldh, gsum);
  HOS_HIP_CHECK(hipGetLastError());
}
void launch_rga_act_bwd(const float* A, int ldz, const float* dG, int ldh, int M, int K, int b, float pc, float* dZ,
                        hipStream_t st) {
  rga_act_bwd_kernel<<<ceil_div(M, 64), 64, 0, st>>>(A, ldz, dG, ldh, M, K, b, pc, dZ);
  HOS_HIP_CHECK(hipGetLastError());
}
void launch_rga_colsum(const float* dZ, int ldz, int M, int K, float* out, hipStream_t st) {
  rga_colsum_kernel<<<K, 256, 0, st>>>(dZ, ldz, M, out);
  HOS_HIP_CHECK(hipGetLastError());
}
void launch_rga_genome_grad(const float* genome, const float* wg, const float* dgb, int L, int K, float* gwg,
                            float* ggen, hipStream_t st) {
  rga_genome_grad_kernel<<<1, 64, 0, st>>>(genome, wg, dgb, L, K, gwg, ggen);
  HOS_HIP_CHECK(hipGetLastError());
}
void launch_rga_loss(const float* gsum, long long ldl, int L, int B, int T, int K, float lambda, float* gm,
                     float* loss, hipStream_t st) {
  rga_gate_mean_kernel<<<L * B, 256, 0, st>>>(gsum, ldl, B, T, K, gm);
  HOS_HIP_CHECK(hipGetLastError());
  HOS_REQUIRE(L <= LOSS_STAGE, HOS_E_INVALID, "rga: too many layers for the loss staging");
  rga_loss_kernel<<<1, 256, 0, st>>>(gm, L, B, lambda, loss);
  HOS_HIP_CHECK(hipGetLastError());
}

}  // namespace hos
