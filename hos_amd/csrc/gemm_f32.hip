// f32 GEMM on fp32 MFMA (v_mfma_f32_32x32x2f32): the keyed training matmuls of the
// reference's GPU boundary (matmul_f32 / abt / atb, src/metal_be.rs:1095-1142, 1212-1234)
// and the LoRA factor GEMMs (x·A, u·B and their gradients), where full f32 inputs keep the
// LoRA gradients close to the CPU f32 path.
//
// C[M,N] = alpha·Σ_k A(m,k)·B(k,n) + beta·C with arbitrary element strides, so one kernel
// serves NN, NT and TN. 64×64 tile, 16-deep slab, 4 waves of one 32×32 MFMA tile each;
// split-K with a deterministic reduction for the tall-skinny LoRA gradients (K = tokens).
#include "kernels.hpp"

namespace hos {
namespace {

constexpr int TB = 64, KB = 16, PADF = 4;

__global__ void __launch_bounds__(256) gemm_f32_kernel(int M, int N, int K, int k_per, float alpha,
                                                       const float* __restrict__ A, long long sam, long long sak,
                                                       const float* __restrict__ B, long long sbk, long long sbn,
                                                       float beta, float* __restrict__ C, long long ldc,
                                                       float* __restrict__ ws) {
  __shared__ float As[KB][TB + PADF];
  __shared__ float Bs[KB][TB + PADF];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int m0 = blockIdx.y * TB, n0 = blockIdx.x * TB;
  const int kbeg = blockIdx.z * k_per, kend = min(K, kbeg + k_per);
  const bool a_kmaj = (sak == 1);  // A rows contiguous along k
  const bool b_nmaj = (sbn == 1);  // B rows contiguous along n

  f16v acc;
#pragma unroll
  for (int r = 0; r < 16; r++) acc[r] = 0.0f;

  for (int k0 = kbeg; k0 < kend; k0 += KB) {
#pragma unroll
    for (int v = 0; v < 4; v++) {
      int idx = tid + 256 * v;
      int mm, kk;
      if (a_kmaj) { mm = idx >> 4; kk = idx & 15; } else { mm = idx & 63; kk = idx >> 6; }
      int m = m0 + mm, k = k0 + kk;
      As[kk][mm] = (m < M && k < kend) ? A[(long long)m * sam + (long long)k * sak] : 0.0f;
      int nn, kb;
      if (b_nmaj) { nn = idx & 63; kb = idx >> 6; } else { nn = idx >> 4; kb = idx & 15; }
      int n = n0 + nn, k2 = k0 + kb;
      Bs[kb][nn] = (n < N && k2 < kend) ? B[(long long)k2 * sbk + (long long)n * sbn] : 0.0f;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < KB; kk += 2) {
      float a = As[kk + (lane >> 5)][wm * 32 + (lane & 31)];
      float b = Bs[kk + (lane >> 5)][wn * 32 + (lane & 31)];
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, acc, 0, 0, 0);
    }
    __syncthreads();
  }
  const int col = n0 + wn * 32 + (lane & 31);
  if (col >= N) return;
#pragma unroll
  for (int r = 0; r < 16; r++) {
    int row = m0 + wm * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
    if (row >= M) continue;
    if (gridDim.z > 1) {
      ws[((long long)blockIdx.z * M + row) * N + col] = acc[r];
    } else {
      float* c = C + (long long)row * ldc + col;
      float v = alpha * acc[r];
      *c = beta == 0.0f ? v : v + beta * *c;
    }
  }
}

__global__ void gemm_f32_reduce(const float* __restrict__ ws, int splits, int M, int N, float alpha, float beta,
                                float* __restrict__ C, long long ldc) {
  long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long long)M * N) return;
  int row = (int)(i / N), col = (int)(i % N);
  float v = 0.0f;
  for (int z = 0; z < splits; z++) v += ws[(long long)z * M * N + i];
  float* c = C + (long long)row * ldc + col;
  v = alpha * v;
  *c = beta == 0.0f ? v : v + beta * *c;
}

}  // namespace

void launch_gemm_f32(long long M, long long N, long long K, float alpha, const float* A, long long sam, long long sak,
                     const float* B, long long sbk, long long sbn, float beta, float* C, long long ldc, float* ws,
                     size_t ws_bytes, hipStream_t st) {
  if (M <= 0 || N <= 0) return;
  int tiles = ceil_div(M, TB) * ceil_div(N, TB);
  int nk = ceil_div(K, KB);
  int splits = 1;
  while (tiles * splits < 512 && nk / (splits * 2) >= 8 && ws &&
         (size_t)(splits * 2) * M * N * sizeof(float) <= ws_bytes)
    splits *= 2;
  int per = ceil_div(nk, splits) * KB;
  splits = K > 0 ? ceil_div(K, per) : 1;
  if (K <= 0) per = 0;
  dim3 grid(ceil_div(N, TB), ceil_div(M, TB), splits);
  gemm_f32_kernel<<<grid, 256, 0, st>>>((int)M, (int)N, (int)K, per, alpha, A, sam, sak, B, sbk, sbn, beta, C, ldc,
                                        ws);
  HOS_HIP_CHECK(hipGetLastError());
  if (splits > 1) {
    long long n = M * N;
    gemm_f32_reduce<<<ceil_div(n, 256), 256, 0, st>>>(ws, splits, (int)M, (int)N, alpha, beta, C, ldc);
    HOS_HIP_CHECK(hipGetLastError());
  }
}

}  // namespace hos
