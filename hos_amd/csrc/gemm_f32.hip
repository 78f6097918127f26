// f32 GEMM on fp32 MFMA (v_mfma_f32_32x32x2f32): the keyed training matmuls of the
// reference's GPU boundary (matmul_f32 / abt / atb, src/metal_be.rs:1095-1142, 1212-1234)
// and the LoRA factor GEMMs (x·A, u·B and their gradients), where full f32 inputs keep the
// LoRA gradients close to the CPU f32 path.
//
// C[M,N] = alpha·Σ_k A(m,k)·B(k,n) + beta·C with arbitrary element strides, so one kernel
// serves NN, NT and TN. The workgroup tile adapts to the LoRA shapes (one side is the rank r ≤ 32):
// 64×64 square, 256×32 tall (N = r), 32×256 wide (M = r); 16-deep k slabs; 4 waves, each owning
// 32×32 MFMA tiles; split-K with a deterministic reduction for the long token contractions.
#include "kernels.hpp"

namespace hos {
namespace {

constexpr int KB = 16, PADF = 4;

template <int BM, int BN>
__global__ void __launch_bounds__(256) gemm_f32_kernel(int M, int N, int K, int k_per, float alpha,
                                                       const float* __restrict__ A, long long sam, long long sak,
                                                       const float* __restrict__ B, long long sbk, long long sbn,
                                                       float beta, float* __restrict__ C, long long ldc,
                                                       float* __restrict__ ws) {
  constexpr int WGM = BM >= BN ? (BM / 32 >= 4 ? 4 : 2) : 1;  // waves along M
  constexpr int WGN = 4 / WGM;
  constexpr int TMW = BM / 32 / WGM, TNW = BN / 32 / WGN;      // 32×32 tiles per wave
  static_assert(TMW >= 1 && TNW >= 1, "tile shape");
  __shared__ float As[KB][BM + PADF];
  __shared__ float Bs[KB][BN + PADF];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WGN, wn = wave % WGN;
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
  const int kbeg = blockIdx.z * k_per, kend = min(K, kbeg + k_per);
  const bool a_kmaj = (sak == 1);  // A rows contiguous along k
  const bool b_nmaj = (sbn == 1);  // B rows contiguous along n

  f16v acc[TMW][TNW];
#pragma unroll
  for (int i = 0; i < TMW; i++)
#pragma unroll
    for (int j = 0; j < TNW; j++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;

  for (int k0 = kbeg; k0 < kend; k0 += KB) {
#pragma unroll
    for (int v = 0; v < BM * KB / 256; v++) {
      int idx = tid + 256 * v, mm, kk;
      if (a_kmaj) { mm = idx / KB; kk = idx % KB; } else { mm = idx % BM; kk = idx / BM; }
      int m = m0 + mm, k = k0 + kk;
      As[kk][mm] = (m < M && k < kend) ? A[(long long)m * sam + (long long)k * sak] : 0.0f;
    }
#pragma unroll
    for (int v = 0; v < BN * KB / 256; v++) {
      int idx = tid + 256 * v, nn, kk;
      if (b_nmaj) { nn = idx % BN; kk = idx / BN; } else { nn = idx / KB; kk = idx % KB; }
      int n = n0 + nn, k = k0 + kk;
      Bs[kk][nn] = (n < N && k < kend) ? B[(long long)k * sbk + (long long)n * sbn] : 0.0f;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < KB; kk += 2) {
      float a[TMW], b[TNW];
#pragma unroll
      for (int i = 0; i < TMW; i++) a[i] = As[kk + (lane >> 5)][(wm * TMW + i) * 32 + (lane & 31)];
#pragma unroll
      for (int j = 0; j < TNW; j++) b[j] = Bs[kk + (lane >> 5)][(wn * TNW + j) * 32 + (lane & 31)];
#pragma unroll
      for (int i = 0; i < TMW; i++)
#pragma unroll
        for (int j = 0; j < TNW; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i], b[j], acc[i][j], 0, 0, 0);
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < TMW; i++)
#pragma unroll
    for (int j = 0; j < TNW; j++) {
      const int col = n0 + (wn * TNW + j) * 32 + (lane & 31);
      if (col >= N) continue;
#pragma unroll
      for (int r = 0; r < 16; r++) {
        int row = m0 + (wm * TMW + i) * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (row >= M) continue;
        if (gridDim.z > 1) {
          ws[((long long)blockIdx.z * M + row) * N + col] = acc[i][j][r];
        } else {
          float* c = C + (long long)row * ldc + col;
          float v = alpha * acc[i][j][r];
          *c = beta == 0.0f ? v : v + beta * *c;
        }
      }
    }
}

__global__ void gemm_f32_reduce(const float* __restrict__ ws, int splits, int M, int N, float alpha, float beta,
                                float* __restrict__ C, long long ldc) {
  long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long long)M * N) return;
  int row = (int)(i / N), col = (int)(i % N);
  float v = 0.0f;
  const long long stride = (long long)M * N;
  int z = 0;
  for (; z + 4 <= splits; z += 4) {  // four independent loads in flight
    float a0 = ws[z * stride + i], a1 = ws[(z + 1) * stride + i];
    float a2 = ws[(z + 2) * stride + i], a3 = ws[(z + 3) * stride + i];
    v += a0;
    v += a1;
    v += a2;
    v += a3;
  }
  for (; z < splits; z++) v += ws[z * stride + i];
  float* c = C + (long long)row * ldc + col;
  v = alpha * v;
  *c = beta == 0.0f ? v : v + beta * *c;
}

template <int BM, int BN>
void launch_tile(long long M, long long N, long long K, float alpha, const float* A, long long sam, long long sak,
                 const float* B, long long sbk, long long sbn, float beta, float* C, long long ldc, float* ws,
                 size_t ws_bytes, hipStream_t st) {
  int tiles = ceil_div(M, BM) * ceil_div(N, BN);
  int nk = ceil_div(K, KB);
  int splits = 1;
  // the LoRA shapes give a handful of tiles with long contractions: split until ~1k workgroups
  while (tiles * splits < 1024 && splits < 32 && nk / (splits * 2) >= 2 && ws &&
         (size_t)(splits * 2) * M * N * sizeof(float) <= ws_bytes)
    splits *= 2;
  int per = ceil_div(nk, splits) * KB;
  splits = K > 0 ? ceil_div(K, per) : 1;
  if (K <= 0) per = 0;
  dim3 grid(ceil_div(N, BN), ceil_div(M, BM), splits);
  gemm_f32_kernel<BM, BN><<<grid, 256, 0, st>>>((int)M, (int)N, (int)K, per, alpha, A, sam, sak, B, sbk, sbn, beta,
                                                C, ldc, ws);
  HOS_HIP_CHECK(hipGetLastError());
  if (splits > 1) {
    long long n = M * N;
    gemm_f32_reduce<<<ceil_div(n, 256), 256, 0, st>>>(ws, splits, (int)M, (int)N, alpha, beta, C, ldc);
    HOS_HIP_CHECK(hipGetLastError());
  }
}

}  // namespace

void launch_gemm_f32(long long M, long long N, long long K, float alpha, const float* A, long long sam, long long sak,
                     const float* B, long long sbk, long long sbn, float beta, float* C, long long ldc, float* ws,
                     size_t ws_bytes, hipStream_t st) {
  if (M <= 0 || N <= 0) return;
  if (N <= 32 && M >= 128)
    launch_tile<256, 32>(M, N, K, alpha, A, sam, sak, B, sbk, sbn, beta, C, ldc, ws, ws_bytes, st);
  else if (M <= 32 && N >= 128)
    launch_tile<32, 256>(M, N, K, alpha, A, sam, sak, B, sbk, sbn, beta, C, ldc, ws, ws_bytes, st);
  else
    launch_tile<64, 64>(M, N, K, alpha, A, sam, sak, B, sbk, sbn, beta, C, ldc, ws, ws_bytes, st);
}

}  // namespace hos
