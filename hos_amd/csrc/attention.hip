// Causal GQA softmax attention, forward and backward, without materialising [H, T, T].
//
// Semantics of PeftModel::forward (src/peft.rs:479-489, 530-553): scores = (q·kᵀ)·(1/√hd), the
// strictly-upper triangle masked (−1e9 there gives exactly zero probability, as skipping does),
// row softmax (src/tensor.rs:2460-2491), ctx = P·v, kv head = h / (n_heads / n_kv_heads)
// (repeat_interleave_dim0, src/tensor.rs:2819-2841). Backward = the bmm/softmax/repeat VJPs
// (src/tensor.rs:2260-2272, :2481-2490, :2831-2840) in flash form: P is recomputed from the saved
// log-sum-exp, dS = P∘(dP − rowsum(dO∘O)), and GQA gradients are summed over the group.
//
// Layout: qkv [M, ld] rows m = b·T + t, q heads at cols h·64, k at kcol + g·64, v at vcol + g·64.
// f32 throughout; 64×64 tiles in LDS; 4 threads per row (each owns 16 of the 64 columns).
#include "fused.hpp"

namespace hos {
namespace {

constexpr int HD = 64, BLK = 64, LP = HD + 1;  // padded LDS row

__global__ void __launch_bounds__(256) attn_fwd_kernel(const float* __restrict__ qkv, long long ld, int kcol, int vcol,
                                                       int T, int nh, int group, float scale, float* __restrict__ o,
                                                       long long ldo, float* __restrict__ lse) {
  __shared__ float Ks[BLK][LP];
  __shared__ float Vs[BLK][LP];
  __shared__ float Ps[BLK][BLK + 1];
  const int qb = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int g = h / group;
  const int tid = threadIdx.x, i = tid >> 2, c = tid & 3;
  const int qi = qb * BLK + i;  // query position
  const bool valid = qi < T;
  const long long rowq = (long long)b * T + (valid ? qi : T - 1);
  float q[HD];
#pragma unroll
  for (int d = 0; d < HD; d++) q[d] = qkv[rowq * ld + h * HD + d];
  float mrun = -INFINITY, lrun = 0.0f, acc[16];
#pragma unroll
  for (int d = 0; d < 16; d++) acc[d] = 0.0f;

  for (int kb = 0; kb <= qb; kb++) {
    __syncthreads();
    for (int e = tid; e < BLK * HD; e += 256) {
      int r = e / HD, d = e % HD;
      int kt = kb * BLK + r;
      long long row = (long long)b * T + (kt < T ? kt : T - 1);
      Ks[r][d] = qkv[row * ld + kcol + g * HD + d];
      Vs[r][d] = qkv[row * ld + vcol + g * HD + d];
    }
    __syncthreads();
    float s[16], mloc = -INFINITY;
#pragma unroll
    for (int jj = 0; jj < 16; jj++) {
      int j = c * 16 + jj, kt = kb * BLK + j;
      float dot = 0.0f;
#pragma unroll
      for (int d = 0; d < HD; d++) dot += q[d] * Ks[j][d];
      float sv = dot * scale;
      if (kt > qi || kt >= T) sv = -INFINITY;
      s[jj] = sv;
      mloc = fmaxf(mloc, sv);
    }
    mloc = fmaxf(mloc, __shfl_xor(mloc, 1));
    mloc = fmaxf(mloc, __shfl_xor(mloc, 2));
    float mnew = fmaxf(mrun, mloc);
    float alpha = (mrun == -INFINITY) ? 0.0f : expf(mrun - mnew);
    float psum = 0.0f;
#pragma unroll
    for (int jj = 0; jj < 16; jj++) {
      float p = (s[jj] == -INFINITY) ? 0.0f : expf(s[jj] - mnew);
      Ps[i][c * 16 + jj] = p;
      psum += p;
    }
    psum += __shfl_xor(psum, 1);
    psum += __shfl_xor(psum, 2);
    lrun = lrun * alpha + psum;
    mrun = mnew;
    __syncthreads();
#pragma unroll
    for (int d = 0; d < 16; d++) acc[d] *= alpha;
    for (int j = 0; j < BLK; j++) {
      float p = Ps[i][j];
#pragma unroll
      for (int d = 0; d < 16; d++) acc[d] += p * Vs[j][c * 16 + d];
    }
  }
  if (!valid) return;
  float inv = 1.0f / lrun;
  float* orow = o + ((long long)b * T + qi) * ldo + h * HD + c * 16;
#pragma unroll
  for (int d = 0; d < 16; d++) orow[d] = acc[d] * inv;
  if (c == 0) lse[((long long)b * nh + h) * T + qi] = mrun + logf(lrun);
}

// Dvec[b,h,t] = Σ_d dO·O over the head's 64 columns.
__global__ void attn_dvec_kernel(const float* __restrict__ o, const float* __restrict__ dout, long long ld, int T,
                                 int nh, int B, float* __restrict__ dvec) {
  long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long long)B * nh * T) return;
  int t = (int)(i % T);
  int h = (int)((i / T) % nh);
  int b = (int)(i / ((long long)T * nh));
  const float* orow = o + ((long long)b * T + t) * ld + h * HD;
  const float* drow = dout + ((long long)b * T + t) * ld + h * HD;
  float s = 0.0f;
  for (int d = 0; d < HD; d++) s += drow[d] * orow[d];
  dvec[i] = s;
}

// dQ for one (query block, head): dQ = scale·Σ_j dS[i][j]·K[j].
__global__ void __launch_bounds__(256) attn_dq_kernel(const float* __restrict__ qkv, long long ld, int kcol, int vcol,
                                                      const float* __restrict__ dout, long long ldd,
                                                      const float* __restrict__ lse, const float* __restrict__ dvec,
                                                      int T, int nh, int group, float scale, float* __restrict__ dq,
                                                      long long ldq) {
  __shared__ float Ks[BLK][LP];
  __shared__ float Vs[BLK][LP];
  __shared__ float Ss[BLK][BLK + 1];
  const int qb = blockIdx.x, h = blockIdx.y, b = blockIdx.z, g = h / group;
  const int tid = threadIdx.x, i = tid >> 2, c = tid & 3;
  const int qi = qb * BLK + i;
  const bool valid = qi < T;
  const long long row = (long long)b * T + (valid ? qi : T - 1);
  float q[HD], dov[HD];
#pragma unroll
  for (int d = 0; d < HD; d++) {
    q[d] = qkv[row * ld + h * HD + d];
    dov[d] = dout[row * ldd + h * HD + d];
  }
  const long long si = ((long long)b * nh + h) * T + (valid ? qi : T - 1);
  const float L = lse[si], Dv = dvec[si];
  float acc[16];
#pragma unroll
  for (int d = 0; d < 16; d++) acc[d] = 0.0f;
  for (int kb = 0; kb <= qb; kb++) {
    __syncthreads();
    for (int e = tid; e < BLK * HD; e += 256) {
      int r = e / HD, d = e % HD;
      int kt = kb * BLK + r;
      long long rr = (long long)b * T + (kt < T ? kt : T - 1);
      Ks[r][d] = qkv[rr * ld + kcol + g * HD + d];
      Vs[r][d] = qkv[rr * ld + vcol + g * HD + d];
    }
    __syncthreads();
#pragma unroll 4
    for (int jj = 0; jj < 16; jj++) {
      int j = c * 16 + jj, kt = kb * BLK + j;
      float dot = 0.0f, dp = 0.0f;
#pragma unroll
      for (int d = 0; d < HD; d++) {
        dot += q[d] * Ks[j][d];
        dp += dov[d] * Vs[j][d];
      }
      float p = (kt > qi || kt >= T) ? 0.0f : expf(dot * scale - L);
      Ss[i][j] = p * (dp - Dv);
    }
    __syncthreads();
    for (int j = 0; j < BLK; j++) {
      float ds = Ss[i][j];
#pragma unroll
      for (int d = 0; d < 16; d++) acc[d] += ds * Ks[j][c * 16 + d];
    }
  }
  if (!valid) return;
  float* out = dq + row * ldq + h * HD + c * 16;
#pragma unroll
  for (int d = 0; d < 16; d++) out[d] = acc[d] * scale;
}

// dK, dV for one (key block, kv head), summed over the group's query heads and all query blocks ≥ kb.
__global__ void __launch_bounds__(256) attn_dkdv_kernel(const float* __restrict__ qkv, long long ld, int kcol,
                                                        int vcol, const float* __restrict__ dout, long long ldd,
                                                        const float* __restrict__ lse,
                                                        const float* __restrict__ dvec, int T, int nh, int group,
                                                        float scale, float* __restrict__ dkv, long long ldk) {
  __shared__ float Qs[BLK][LP];
  __shared__ float Ds[BLK][LP];
  __shared__ float Ls[BLK], Dvs[BLK];
  const int kb = blockIdx.x, g = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, j = tid >> 2, c = tid & 3;
  const int kt = kb * BLK + j;
  const bool valid = kt < T;
  const long long row = (long long)b * T + (valid ? kt : T - 1);
  float k[HD], v[HD];
#pragma unroll
  for (int d = 0; d < HD; d++) {
    k[d] = qkv[row * ld + kcol + g * HD + d];
    v[d] = qkv[row * ld + vcol + g * HD + d];
  }
  float dk[16], dv[16];
#pragma unroll
  for (int d = 0; d < 16; d++) dk[d] = dv[d] = 0.0f;
  const int nqb = (T + BLK - 1) / BLK;
  for (int hh = 0; hh < group; hh++) {
    const int h = g * group + hh;
    for (int qb = kb; qb < nqb; qb++) {
      __syncthreads();
      for (int e = tid; e < BLK * HD; e += 256) {
        int r = e / HD, d = e % HD;
        int qt = qb * BLK + r;
        long long rr = (long long)b * T + (qt < T ? qt : T - 1);
        Qs[r][d] = qkv[rr * ld + h * HD + d];
        Ds[r][d] = dout[rr * ldd + h * HD + d];
      }
      if (tid < BLK) {
        int qt = qb * BLK + tid;
        long long si = ((long long)b * nh + h) * T + (qt < T ? qt : T - 1);
        Ls[tid] = lse[si];
        Dvs[tid] = dvec[si];
      }
      __syncthreads();
      // this thread's 16 queries i = c·16 .. c·16+15 against key j
      float pl[16], sl[16];
#pragma unroll
      for (int ii = 0; ii < 16; ii++) {
        int i = c * 16 + ii, qt = qb * BLK + i;
        float dot = 0.0f, dp = 0.0f;
#pragma unroll
        for (int d = 0; d < HD; d++) {
          dot += Qs[i][d] * k[d];
          dp += Ds[i][d] * v[d];
        }
        float p = (kt > qt || qt >= T || !valid) ? 0.0f : expf(dot * scale - Ls[i]);
        pl[ii] = p;
        sl[ii] = p * (dp - Dvs[i]);
      }
      // the 4 lanes of key j (consecutive lanes) each hold 16 of the 64 queries: exchange by shuffle
      const int lane = tid & 63;
#pragma unroll
      for (int src = 0; src < 4; src++) {
#pragma unroll
        for (int ii = 0; ii < 16; ii++) {
          float p = __shfl(pl[ii], (lane & ~3) | src);
          float ds = __shfl(sl[ii], (lane & ~3) | src);
          int i = src * 16 + ii;
#pragma unroll
          for (int d = 0; d < 16; d++) {
            dv[d] += p * Ds[i][c * 16 + d];
            dk[d] += ds * Qs[i][c * 16 + d];
          }
        }
      }
    }
  }
  if (!valid) return;
  float* dkr = dkv + row * ldk + kcol + g * HD + c * 16;
  float* dvr = dkv + row * ldk + vcol + g * HD + c * 16;
#pragma unroll
  for (int d = 0; d < 16; d++) {
    dkr[d] = dk[d] * scale;
    dvr[d] = dv[d];
  }
}

}  // namespace

void launch_attn_fwd(const float* qkv, long long ld, int kcol, int vcol, int B, int T, int nh, int nkv, int hd,
                     float* o, long long ldo, float* lse, hipStream_t st) {
  HOS_REQUIRE(hd == HD, HOS_E_INVALID, "attention: head_dim must be 64");
  dim3 grid(ceil_div(T, BLK), nh, B);
  attn_fwd_kernel<<<grid, 256, 0, st>>>(qkv, ld, kcol, vcol, T, nh, nh / nkv, 1.0f / sqrtf((float)hd), o, ldo, lse);
  HOS_HIP_CHECK(hipGetLastError());
}

void launch_attn_bwd(const float* qkv, long long ld, int kcol, int vcol, const float* o, const float* dout,
                     long long ldo, const float* lse, float* dvec, int B, int T, int nh, int nkv, int hd, float* dqkv,
                     long long ldd, hipStream_t st) {
  HOS_REQUIRE(hd == HD, HOS_E_INVALID, "attention: head_dim must be 64");
  float scale = 1.0f / sqrtf((float)hd);
  long long n = (long long)B * nh * T;
  attn_dvec_kernel<<<ceil_div(n, 256), 256, 0, st>>>(o, dout, ldo, T, nh, B, dvec);
  HOS_HIP_CHECK(hipGetLastError());
  dim3 gq(ceil_div(T, BLK), nh, B);
  attn_dq_kernel<<<gq, 256, 0, st>>>(qkv, ld, kcol, vcol, dout, ldo, lse, dvec, T, nh, nh / nkv, scale, dqkv, ldd);
  HOS_HIP_CHECK(hipGetLastError());
  dim3 gk(ceil_div(T, BLK), nkv, B);
  attn_dkdv_kernel<<<gk, 256, 0, st>>>(qkv, ld, kcol, vcol, dout, ldo, lse, dvec, T, nh, nh / nkv, scale, dqkv, ldd);
  HOS_HIP_CHECK(hipGetLastError());
}

}  // namespace hos
