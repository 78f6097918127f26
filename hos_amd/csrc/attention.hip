// Causal GQA softmax attention, forward and backward, on fp32 MFMA (v_mfma_f32_32x32x2f32), without
// materialising [H, T, T].
//
// Semantics of PeftModel::forward (src/peft.rs:479-489, 530-553): scores = (q·kᵀ)·(1/√hd), the
// strictly-upper triangle masked (−1e9 there gives exactly zero probability, as skipping does),
// row softmax (src/tensor.rs:2460-2491), ctx = P·v, kv head = h / (n_heads / n_kv_heads)
// (repeat_interleave_dim0, src/tensor.rs:2819-2841). Backward = the bmm/softmax/repeat VJPs
// (src/tensor.rs:2260-2272, :2481-2490, :2831-2840) in flash form: P is recomputed from the saved
// log-sum-exp, dS = P∘(dP − rowsum(dO∘O)), and GQA gradients are summed over the group.
// 1/√64 = 2^-3 is folded into q exactly.
//
// MFMA layout used throughout (32×32 tiles): the D matrix X[i][j] sits with column j = lane%32 and
// rows i = 8·(r/4) + 4·(lane/32) + r%4 in register r. Read back as an A operand, register r of that
// layout supplies row (lane%32) of Xᵀ at contraction index κ(r, lane/32) = 8·(r/4) + 4·(lane/32) + r%4,
// so a score tile feeds the next MFMA straight from registers provided the other operand is gathered
// in the same κ order. Per wave: 32 queries (or keys) × 64 head dims; one wave per workgroup.
#include "fused.hpp"

namespace hos {
namespace {

constexpr int HD = 64, TB = 32, LP = HD + 1;  // tile rows, padded LDS row (floats)

__device__ __forceinline__ int kap(int s, int h) { return 8 * (s >> 2) + 4 * h + (s & 3); }

// Load rows [r0, r0+32) × 64 cols (row stride ld, col offset col) into LDS [32][LP], clamping rows ≥ T
// to T-1 (masked later); scaled by `mul`.
__device__ __forceinline__ void load_tile(float (*dst)[LP], const float* __restrict__ src, long long base_row, int r0,
                                          int T, long long ld, int col, float mul) {
  const int lane = threadIdx.x;
  for (int e = lane; e < TB * HD / 4; e += 64) {
    int r = e / (HD / 4), c4 = e % (HD / 4);
    int t = r0 + r;
    long long row = base_row + (t < T ? t : T - 1);
    float4 v = *(const float4*)(src + row * ld + col + 4 * c4);
    dst[r][4 * c4] = v.x * mul;
    dst[r][4 * c4 + 1] = v.y * mul;
    dst[r][4 * c4 + 2] = v.z * mul;
    dst[r][4 * c4 + 3] = v.w * mul;
  }
}

// B-operand fragment of a [32 rows][64] matrix held in registers: frag[s] = X[row0 + lane%32][2s + lane/32].
__device__ __forceinline__ void load_frag(float* frag, const float* __restrict__ src, long long base_row, int r0,
                                          int T, long long ld, int col, float mul) {
  const int lane = threadIdx.x;
  int t = r0 + (lane & 31);
  long long row = base_row + (t < T ? t : T - 1);
  const float* p = src + row * ld + col + (lane >> 5);
#pragma unroll
  for (int s = 0; s < 32; s++) frag[s] = p[2 * s] * mul;
}

__global__ void __launch_bounds__(64) attn_fwd_kernel(const float* __restrict__ qkv, long long ld, int kcol, int vcol,
                                                      int T, int nh, int group, float* __restrict__ o, long long ldo,
                                                      float* __restrict__ lse) {
  __shared__ float Ks[TB][LP];
  __shared__ float Vs[TB][LP];
  __shared__ float xch[TB];
  const int qb = blockIdx.x, h = blockIdx.y, b = blockIdx.z, g = h / group;
  const int lane = threadIdx.x, hl = lane >> 5, q0 = qb * TB;
  const int myq = q0 + (lane & 31);  // this lane's query in the Sᵀ layout
  const long long base = (long long)b * T;
  float qf[32];
  load_frag(qf, qkv, base, q0, T, ld, h * HD, 0.125f);
  f16v O0, O1;
#pragma unroll
  for (int r = 0; r < 16; r++) O0[r] = O1[r] = 0.0f;
  float m = -INFINITY, l = 0.0f;
  const int nkb = min(qb + 1, (T + TB - 1) / TB);
  for (int kb = 0; kb < nkb; kb++) {
    const int k0 = kb * TB;
    __syncthreads();
    load_tile(Ks, qkv, base, k0, T, ld, kcol + g * HD, 1.0f);
    load_tile(Vs, qkv, base, k0, T, ld, vcol + g * HD, 1.0f);
    __syncthreads();
    f16v S;
#pragma unroll
    for (int r = 0; r < 16; r++) S[r] = 0.0f;
#pragma unroll
    for (int s = 0; s < 32; s++) S = __builtin_amdgcn_mfma_f32_32x32x2f32(Ks[lane & 31][2 * s + hl], qf[s], S, 0, 0, 0);
    // S[r] = score(key k0 + kap(r, hl), query myq)
    float mb = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; r++) {
      int key = k0 + kap(r, hl);
      if (key > myq || key >= T) S[r] = -INFINITY;
      mb = fmaxf(mb, S[r]);
    }
    mb = fmaxf(mb, __shfl_xor(mb, 32));
    const float mn = fmaxf(m, mb);
    const float alpha = (m == -INFINITY) ? 0.0f : expf(m - mn);
    float ps = 0.0f;
    float p[16];
#pragma unroll
    for (int r = 0; r < 16; r++) {
      p[r] = (S[r] == -INFINITY) ? 0.0f : expf(S[r] - mn);
      ps += p[r];
    }
    ps += __shfl_xor(ps, 32);
    l = l * alpha + ps;
    m = mn;
    // rescale O rows (queries q0 + kap(r, hl) in the O layout) by their alpha
    if (lane < 32) xch[lane] = alpha;
    __syncthreads();
#pragma unroll
    for (int r = 0; r < 16; r++) {
      float a = xch[kap(r, hl)];
      O0[r] *= a;
      O1[r] *= a;
    }
#pragma unroll
    for (int s = 0; s < 16; s++) {
      const float* vr = Vs[kap(s, hl)];
      O0 = __builtin_amdgcn_mfma_f32_32x32x2f32(p[s], vr[lane & 31], O0, 0, 0, 0);
      O1 = __builtin_amdgcn_mfma_f32_32x32x2f32(p[s], vr[32 + (lane & 31)], O1, 0, 0, 0);
    }
  }
  __syncthreads();
  if (lane < 32) xch[lane] = l;
  __syncthreads();
  if (lane < 32 && myq < T) lse[((long long)b * nh + h) * T + myq] = m + logf(l);
#pragma unroll
  for (int r = 0; r < 16; r++) {
    int q = q0 + kap(r, hl);
    if (q >= T) continue;
    float inv = 1.0f / xch[kap(r, hl)];
    float* orow = o + (base + q) * ldo + h * HD;
    orow[lane & 31] = O0[r] * inv;
    orow[32 + (lane & 31)] = O1[r] * inv;
  }
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

// dQ for 32 queries of head h: Sᵀ and dPᵀ with lanes on queries, dQ = (dS·K)·2^-3.
__global__ void __launch_bounds__(64) attn_dq_kernel(const float* __restrict__ qkv, long long ld, int kcol, int vcol,
                                                     const float* __restrict__ dout, long long ldd,
                                                     const float* __restrict__ lse, const float* __restrict__ dvec,
                                                     int T, int nh, int group, float* __restrict__ dq,
                                                     long long ldq) {
  __shared__ float Ks[TB][LP];
  __shared__ float Vs[TB][LP];
  const int qb = blockIdx.x, h = blockIdx.y, b = blockIdx.z, g = h / group;
  const int lane = threadIdx.x, hl = lane >> 5, q0 = qb * TB;
  const int myq = q0 + (lane & 31);
  const long long base = (long long)b * T;
  float qf[32], df[32];
  load_frag(qf, qkv, base, q0, T, ld, h * HD, 0.125f);
  load_frag(df, dout, base, q0, T, ldd, h * HD, 1.0f);
  const long long si = ((long long)b * nh + h) * T + (myq < T ? myq : T - 1);
  const float L = lse[si], Dv = dvec[si];
  f16v A0, A1;
#pragma unroll
  for (int r = 0; r < 16; r++) A0[r] = A1[r] = 0.0f;
  const int nkb = min(qb + 1, (T + TB - 1) / TB);
  for (int kb = 0; kb < nkb; kb++) {
    const int k0 = kb * TB;
    __syncthreads();
    load_tile(Ks, qkv, base, k0, T, ld, kcol + g * HD, 1.0f);
    load_tile(Vs, qkv, base, k0, T, ld, vcol + g * HD, 1.0f);
    __syncthreads();
    f16v S, dP;
#pragma unroll
    for (int r = 0; r < 16; r++) S[r] = dP[r] = 0.0f;
#pragma unroll
    for (int s = 0; s < 32; s++) {
      S = __builtin_amdgcn_mfma_f32_32x32x2f32(Ks[lane & 31][2 * s + hl], qf[s], S, 0, 0, 0);
      dP = __builtin_amdgcn_mfma_f32_32x32x2f32(Vs[lane & 31][2 * s + hl], df[s], dP, 0, 0, 0);
    }
    float ds[16];
#pragma unroll
    for (int r = 0; r < 16; r++) {
      int key = k0 + kap(r, hl);
      float pv = (key > myq || key >= T || myq >= T) ? 0.0f : expf(S[r] - L);
      ds[r] = pv * (dP[r] - Dv);
    }
#pragma unroll
    for (int s = 0; s < 16; s++) {
      const float* kr = Ks[kap(s, hl)];
      A0 = __builtin_amdgcn_mfma_f32_32x32x2f32(ds[s], kr[lane & 31], A0, 0, 0, 0);
      A1 = __builtin_amdgcn_mfma_f32_32x32x2f32(ds[s], kr[32 + (lane & 31)], A1, 0, 0, 0);
    }
  }
#pragma unroll
  for (int r = 0; r < 16; r++) {
    int q = q0 + kap(r, hl);
    if (q >= T) continue;
    float* out = dq + (base + q) * ldq + h * HD;
    out[lane & 31] = A0[r] * 0.125f;
    out[32 + (lane & 31)] = A1[r] * 0.125f;
  }
}

// dK, dV for 32 keys against query head h (kv head g = h / group): S and dP with lanes on keys.
// With group > 1 each head's contribution goes to part[(b·T + key)][h][2·64] and attn_group_sum adds
// the group in head order; with group == 1 it is written in place.
__global__ void __launch_bounds__(64) attn_dkdv_kernel(const float* __restrict__ qkv, long long ld, int kcol, int vcol,
                                                       const float* __restrict__ dout, long long ldd,
                                                       const float* __restrict__ lse,
                                                       const float* __restrict__ dvec, int T, int nh, int group,
                                                       float* __restrict__ dkv, long long ldk,
                                                       float* __restrict__ part) {
  __shared__ float Qs[TB][LP];
  __shared__ float Ds[TB][LP];
  __shared__ float Ls[TB], Dvs[TB];
  const int kb = blockIdx.x, h = blockIdx.y, b = blockIdx.z, g = h / group;
  const int lane = threadIdx.x, hl = lane >> 5, k0 = kb * TB;
  const int mykey = k0 + (lane & 31);
  const long long base = (long long)b * T;
  float kf[32], vf[32];
  load_frag(kf, qkv, base, k0, T, ld, kcol + g * HD, 1.0f);
  load_frag(vf, qkv, base, k0, T, ld, vcol + g * HD, 1.0f);
  f16v K0, K1, V0, V1;
#pragma unroll
  for (int r = 0; r < 16; r++) K0[r] = K1[r] = V0[r] = V1[r] = 0.0f;
  const int nqb = (T + TB - 1) / TB;
  {
    for (int qb = kb; qb < nqb; qb++) {
      const int q0 = qb * TB;
      __syncthreads();
      load_tile(Qs, qkv, base, q0, T, ld, h * HD, 0.125f);
      load_tile(Ds, dout, base, q0, T, ldd, h * HD, 1.0f);
      if (lane < TB) {
        int qt = q0 + lane;
        long long si = ((long long)b * nh + h) * T + (qt < T ? qt : T - 1);
        Ls[lane] = lse[si];
        Dvs[lane] = dvec[si];
      }
      __syncthreads();
      f16v S, dP;
#pragma unroll
      for (int r = 0; r < 16; r++) S[r] = dP[r] = 0.0f;
#pragma unroll
      for (int s = 0; s < 32; s++) {
        S = __builtin_amdgcn_mfma_f32_32x32x2f32(Qs[lane & 31][2 * s + hl], kf[s], S, 0, 0, 0);
        dP = __builtin_amdgcn_mfma_f32_32x32x2f32(Ds[lane & 31][2 * s + hl], vf[s], dP, 0, 0, 0);
      }
      // S[r] = score(query q0 + kap(r, hl), key mykey)
      float p[16], ds[16];
#pragma unroll
      for (int r = 0; r < 16; r++) {
        int qi = kap(r, hl), q = q0 + qi;
        float pv = (mykey > q || q >= T || mykey >= T) ? 0.0f : expf(S[r] - Ls[qi]);
        p[r] = pv;
        ds[r] = pv * (dP[r] - Dvs[qi]);
      }
#pragma unroll
      for (int s = 0; s < 16; s++) {
        const float* dr = Ds[kap(s, hl)];
        const float* qr = Qs[kap(s, hl)];
        V0 = __builtin_amdgcn_mfma_f32_32x32x2f32(p[s], dr[lane & 31], V0, 0, 0, 0);
        V1 = __builtin_amdgcn_mfma_f32_32x32x2f32(p[s], dr[32 + (lane & 31)], V1, 0, 0, 0);
        K0 = __builtin_amdgcn_mfma_f32_32x32x2f32(ds[s], qr[lane & 31], K0, 0, 0, 0);
        K1 = __builtin_amdgcn_mfma_f32_32x32x2f32(ds[s], qr[32 + (lane & 31)], K1, 0, 0, 0);
      }
    }
  }
  // Q in LDS carried the 2^-3 scale, so K0/K1 already hold dK = dSᵀ·Q·scale.
#pragma unroll
  for (int r = 0; r < 16; r++) {
    int key = k0 + kap(r, hl);
    if (key >= T) continue;
    float *kr, *vr;
    if (group == 1) {
      kr = dkv + (base + key) * ldk + kcol + g * HD;
      vr = dkv + (base + key) * ldk + vcol + g * HD;
    } else {
      kr = part + ((base + key) * nh + h) * 2 * HD;
      vr = kr + HD;
    }
    kr[lane & 31] = K0[r];
    kr[32 + (lane & 31)] = K1[r];
    vr[lane & 31] = V0[r];
    vr[32 + (lane & 31)] = V1[r];
  }
}

// dK/dV of kv head g = Σ over its group's heads, in head order (deterministic).
__global__ void attn_group_sum(const float* __restrict__ part, int M, int nh, int nkv, int group,
                               float* __restrict__ dkv, long long ldk, int kcol, int vcol) {
  long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long long)M * nkv * 2 * HD) return;
  int c = (int)(i % (2 * HD));
  long long t = i / (2 * HD);
  int g = (int)(t % nkv);
  long long m = t / nkv;
  float s = 0.0f;
  for (int hh = 0; hh < group; hh++) s += part[(m * nh + g * group + hh) * 2 * HD + c];
  int col = (c < HD ? kcol : vcol) + g * HD + (c % HD);
  dkv[m * ldk + col] = s;
}

}  // namespace

void launch_attn_fwd(const float* qkv, long long ld, int kcol, int vcol, int B, int T, int nh, int nkv, int hd,
                     float* o, long long ldo, float* lse, hipStream_t st) {
  HOS_REQUIRE(hd == HD, HOS_E_INVALID, "attention: head_dim must be 64");
  HOS_REQUIRE(ld % 4 == 0 && kcol % 4 == 0 && vcol % 4 == 0, HOS_E_INVALID, "attention: unaligned qkv layout");
  dim3 grid(ceil_div(T, TB), nh, B);
  attn_fwd_kernel<<<grid, 64, 0, st>>>(qkv, ld, kcol, vcol, T, nh, nh / nkv, o, ldo, lse);
  HOS_HIP_CHECK(hipGetLastError());
}

void launch_attn_bwd(const float* qkv, long long ld, int kcol, int vcol, const float* o, const float* dout,
                     long long ldo, const float* lse, float* dvec, int B, int T, int nh, int nkv, int hd, float* dqkv,
                     long long ldd, float* part, hipStream_t st) {
  HOS_REQUIRE(hd == HD, HOS_E_INVALID, "attention: head_dim must be 64");
  HOS_REQUIRE(nh == nkv || part != nullptr, HOS_E_INVALID, "attention: GQA backward needs a partial buffer");
  HOS_REQUIRE(ldo % 4 == 0, HOS_E_INVALID, "attention: unaligned dO layout");
  long long n = (long long)B * nh * T;
  attn_dvec_kernel<<<ceil_div(n, 256), 256, 0, st>>>(o, dout, ldo, T, nh, B, dvec);
  HOS_HIP_CHECK(hipGetLastError());
  dim3 gq(ceil_div(T, TB), nh, B);
  attn_dq_kernel<<<gq, 64, 0, st>>>(qkv, ld, kcol, vcol, dout, ldo, lse, dvec, T, nh, nh / nkv, dqkv, ldd);
  HOS_HIP_CHECK(hipGetLastError());
  dim3 gk(ceil_div(T, TB), nh, B);
  attn_dkdv_kernel<<<gk, 64, 0, st>>>(qkv, ld, kcol, vcol, dout, ldo, lse, dvec, T, nh, nh / nkv, dqkv, ldd, part);
  HOS_HIP_CHECK(hipGetLastError());
  if (nh != nkv) {
    long long ne = (long long)B * T * nkv * 2 * HD;
    attn_group_sum<<<ceil_div(ne, 256), 256, 0, st>>>(part, B * T, nh, nkv, nh / nkv, dqkv, ldd, kcol, vcol);
    HOS_HIP_CHECK(hipGetLastError());
  }
}

}  // namespace hos
