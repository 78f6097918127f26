// Causal GQA softmax attention, forward and backward, on bf16 MFMA with hi/lo-split operands (three
// products per multiply, ~2^-16 relative, fp32 accumulation; softmax and everything elementwise in f32),
// without materialising [H, T, T].
//
// Semantics of PeftModel::forward (src/peft.rs:479-489, 530-553): scores = (q·kᵀ)·(1/√hd), the
// strictly-upper triangle masked (−1e9 there gives exactly zero probability, as skipping does),
// row softmax (src/tensor.rs:2460-2491), ctx = P·v, kv head = h / (n_heads / n_kv_heads)
// (repeat_interleave_dim0, src/tensor.rs:2819-2841). Backward = the bmm/softmax/repeat VJPs
// (src/tensor.rs:2260-2272, :2481-2490, :2831-2840) in flash form: P is recomputed from the saved
// log-sum-exp, dS = P∘(dP − rowsum(dO∘O)), and GQA gradients are summed over the group.
// The scale 1/√hd is folded into q (exactly 2^-3 for hd = 64; the f32 value of 1/√128 for hd = 128).
//
// MFMA layout used throughout (32×32 tiles, here of v_mfma_f32_32x32x16_bf16 on hi/lo-split operands): the D matrix X[i][j] sits with column j = lane%32 and
// rows i = 8·(r/4) + 4·(lane/32) + r%4 in register r. Read back as an A operand, register r of that
// layout supplies row (lane%32) of Xᵀ at contraction index κ(r, lane/32) = 8·(r/4) + 4·(lane/32) + r%4,
// so a score tile feeds the next MFMA straight from registers provided the other operand is gathered
// in the same κ order. Per wave: 32 queries (or keys) × HD head dims (HD = 64 or 128, a template
// parameter); 4 waves per workgroup split the
// other sequence axis and merge in LDS, so there is no workgroup barrier inside the main loops.
#include "fused.hpp"

namespace hos {
namespace {

constexpr int TB = 32, KW = 4;  // tile rows, waves per workgroup
// per head dim: LDS row (padded), 1/√hd
template <int HD>
struct HdC {
  static constexpr int LP = HD + 1, NC = HD / 32;  // NC 32-column tiles per row
};
template <int HD>
__device__ __forceinline__ float qscale() {
  return HD == 64 ? 0.125f : 0.08838834764831845f;  // 1/√128 rounded to f32
}

__device__ __forceinline__ int kap(int s, int h) { return 8 * (s >> 2) + 4 * h + (s & 3); }

// Fragment of one row for a contraction over the HD head dims: frag[4j + e] = row[8j + 4·hl + e]·mul.
// Any bijection of the contraction index works as long as both MFMA operands use it; this one lets a
// lane fetch its 32 values as 8 float4.
template <int HD>
__device__ __forceinline__ void load_rowfrag(float* frag, const float* __restrict__ row, int hl, float mul) {
#pragma unroll
  for (int j = 0; j < HD / 8; j++) {
    const float4 v = *reinterpret_cast<const float4*>(row + 8 * j + 4 * hl);
    frag[4 * j] = v.x * mul;
    frag[4 * j + 1] = v.y * mul;
    frag[4 * j + 2] = v.z * mul;
    frag[4 * j + 3] = v.w * mul;
  }
}

// B operand over 32 rows indexed in κ order: col[16i + s] = X[r0 + κ(s, hl)][32i + c] for the NC column tiles.
template <int HD>
__device__ __forceinline__ void load_kapcols(float* col, const float* __restrict__ src, long long base_row, int r0,
                                             int T, long long ld, int off, int hl, int c, float mul) {
#pragma unroll
  for (int s = 0; s < 16; s++) {
    const int t = r0 + kap(s, hl);
    const float* row = src + (base_row + (t < T ? t : T - 1)) * ld + off;
#pragma unroll
    for (int i = 0; i < HdC<HD>::NC; i++) col[16 * i + s] = row[32 * i + c] * mul;
  }
}

// ---- bf16 hi/lo products: x = hi + lo with hi = bf16(x), lo = bf16(x − hi) (x − hi is exact in f32), and
// a·b ≈ a_hi·b_hi + a_hi·b_lo + a_lo·b_hi on v_mfma_f32_32x32x16_bf16 — relative error ~2^-16 per product
// (the dropped a_lo·b_lo and the rounding of lo), fp32 accumulation, f32 exponent range (no scaling of
// tiny gradients), at 5.3× the throughput of fp32 MFMA per contraction element.
// An HD-dim row fragment (rowfrag order) as HD/16 contraction steps of 8 values per lane.
template <int HD>
struct DFrag {
  bf8 h[HD / 16], l[HD / 16];
};
template <int HD>
__device__ __forceinline__ void to_dfrag(const float* f, DFrag<HD>& F) {
#pragma unroll
  for (int t = 0; t < HD / 16; t++)
#pragma unroll
    for (int i = 0; i < 8; i++) split_bf(f[8 * t + i], F.h[t], F.l[t], i);
}
// 16 κ-ordered values (a 32-row contraction shared by the two half-waves) as 2 steps of 8.
struct KFrag {
  bf8 h[2], l[2];
};
__device__ __forceinline__ void to_kfrag(const float* f, KFrag& F) {
#pragma unroll
  for (int t = 0; t < 2; t++)
#pragma unroll
    for (int i = 0; i < 8; i++) split_bf(f[8 * t + i], F.h[t], F.l[t], i);
}
__device__ __forceinline__ f16v mma3(const bf8& ah, const bf8& al, const bf8& bh, const bf8& bl, f16v c) {
  return mma3_bf16(ah, al, bh, bl, c);
}
// Σ over the HD head dims: D[i][j] += A_row_i · B_row_j (both in rowfrag order)
template <int HD>
__device__ __forceinline__ f16v mma_d(const DFrag<HD>& a, const DFrag<HD>& b, f16v c) {
#pragma unroll
  for (int t = 0; t < HD / 16; t++) c = mma3(a.h[t], a.l[t], b.h[t], b.l[t], c);
  return c;
}
// Σ over 32 κ-ordered rows: D += A(κ) · B(κ)
__device__ __forceinline__ f16v mma_k(const KFrag& a, const KFrag& b, f16v c) {
#pragma unroll
  for (int t = 0; t < 2; t++) c = mma3(a.h[t], a.l[t], b.h[t], b.l[t], c);
  return c;
}

// Forward. Workgroup = (32 queries, head, sequence); its 4 waves take key blocks w, w+4, … up to the
// diagonal, each keeping its own online-softmax state (m, l, O); the states are merged in LDS at the end.
template <int HD>
__global__ void __launch_bounds__(256) attn_fwd_kernel(const float* __restrict__ qkv, long long ld, int kcol, int vcol,
                                                       int T, int nh, int group, float* __restrict__ o, long long ldo,
                                                       float* __restrict__ lse) {
  constexpr int NC = HdC<HD>::NC;
  __shared__ float Os[KW][TB][HdC<HD>::LP];
  __shared__ float Ms[KW][TB], Ls[KW][TB];
  const int nqb = (T + TB - 1) / TB;
  const int qb = nqb - 1 - (int)blockIdx.x, h = blockIdx.y, b = blockIdx.z, g = h / group;  // long rows first
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, hl = lane >> 5, c = lane & 31, q0 = qb * TB;
  const int myq = q0 + c;  // this lane's query in the Sᵀ layout
  const long long base = (long long)b * T;
  DFrag<HD> qd;
  {
    float qf[HD / 2];
    load_rowfrag<HD>(qf, qkv + (base + (myq < T ? myq : T - 1)) * ld + h * HD, hl, qscale<HD>());
    to_dfrag(qf, qd);
  }
  f16v O[NC];
#pragma unroll
  for (int i = 0; i < NC; i++)
#pragma unroll
    for (int r = 0; r < 16; r++) O[i][r] = 0.0f;
  float m = -INFINITY, l = 0.0f;
  for (int kb = w; kb <= qb; kb += KW) {
    const int k0 = kb * TB, kr = k0 + c;
    float kf[HD / 2], vv[HD / 2];
    load_rowfrag<HD>(kf, qkv + (base + (kr < T ? kr : T - 1)) * ld + kcol + g * HD, hl, 1.0f);
    load_kapcols<HD>(vv, qkv, base, k0, T, ld, vcol + g * HD, hl, c, 1.0f);
    DFrag<HD> kd;
    to_dfrag(kf, kd);
    f16v S;
#pragma unroll
    for (int r = 0; r < 16; r++) S[r] = 0.0f;
    S = mma_d(kd, qd, S);
    // S[r] = score(key k0 + κ(r, hl), query myq)
    float mb = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; r++) {
      const int key = k0 + kap(r, hl);
      if (key > myq || key >= T) S[r] = -INFINITY;
      mb = fmaxf(mb, S[r]);
    }
    mb = fmaxf(mb, __shfl_xor(mb, 32));
    const float mn = fmaxf(m, mb);
    const float alpha = (m == -INFINITY) ? 0.0f : expf(m - mn);
    float ps = 0.0f, p[16];
#pragma unroll
    for (int r = 0; r < 16; r++) {
      p[r] = (S[r] == -INFINITY) ? 0.0f : expf(S[r] - mn);
      ps += p[r];
    }
    ps += __shfl_xor(ps, 32);
    l = l * alpha + ps;
    m = mn;
    // O rows are queries q0 + κ(r, hl): fetch their alpha from the lane that owns that query
#pragma unroll
    for (int r = 0; r < 16; r++) {
      const float a = __shfl(alpha, kap(r, hl));
#pragma unroll
      for (int i = 0; i < NC; i++) O[i][r] *= a;
    }
    KFrag pk;
    to_kfrag(p, pk);
#pragma unroll
    for (int i = 0; i < NC; i++) {
      KFrag vi;
      to_kfrag(vv + 16 * i, vi);
      O[i] = mma_k(pk, vi, O[i]);
    }
  }
  if (hl == 0) {
    Ms[w][c] = m;
    Ls[w][c] = l;
  }
#pragma unroll
  for (int r = 0; r < 16; r++)
#pragma unroll
    for (int i = 0; i < NC; i++) Os[w][kap(r, hl)][32 * i + c] = O[i][r];
  __syncthreads();
  // merge the four states: thread → (query tid/8, dims (HD/8)·(tid%8) .. +HD/8)
  const int qi = threadIdx.x >> 3, d0 = (threadIdx.x & 7) * (HD / 8), t = q0 + qi;
  if (t >= T) return;
  float mx = -INFINITY;
#pragma unroll
  for (int v = 0; v < KW; v++) mx = fmaxf(mx, Ms[v][qi]);
  float e[KW], den = 0.0f;
#pragma unroll
  for (int v = 0; v < KW; v++) {
    e[v] = Ms[v][qi] == -INFINITY ? 0.0f : expf(Ms[v][qi] - mx);
    den += Ls[v][qi] * e[v];
  }
  const float inv = 1.0f / den;
  float* orow = o + (base + t) * ldo + h * HD;
#pragma unroll
  for (int d = d0; d < d0 + HD / 8; d++) {
    float num = 0.0f;
#pragma unroll
    for (int v = 0; v < KW; v++) num += Os[v][qi][d] * e[v];
    orow[d] = num * inv;
  }
  if (d0 == 0) lse[((long long)b * nh + h) * T + t] = mx + logf(den);
}

// Dvec[b,h,t] = Σ_d dO·O over the head's HD columns.
template <int HD>
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

// dQ for 32 queries of head h: Sᵀ and dPᵀ with lanes on queries, dQ = (dS·K)·2^-3. The 4 waves take
// key blocks w, w+4, …; their partial dQ are summed in wave order.
template <int HD>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(HD == 64 ? 2 : 1))) attn_dq_kernel(const float* __restrict__ qkv, long long ld, int kcol, int vcol,
                                                      const float* __restrict__ dout, long long ldd,
                                                      const float* __restrict__ lse, const float* __restrict__ dvec,
                                                      int T, int nh, int group, float* __restrict__ dq,
                                                      long long ldq) {
  constexpr int NC = HdC<HD>::NC;
  __shared__ float As[KW][TB][HdC<HD>::LP];
  const int nqb = (T + TB - 1) / TB;
  const int qb = nqb - 1 - (int)blockIdx.x, h = blockIdx.y, b = blockIdx.z, g = h / group;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, hl = lane >> 5, c = lane & 31, q0 = qb * TB;
  const int myq = q0 + c;
  const long long base = (long long)b * T, qrow = base + (myq < T ? myq : T - 1);
  DFrag<HD> qd, dd;
  {
    float qf[HD / 2], df[HD / 2];
    load_rowfrag<HD>(qf, qkv + qrow * ld + h * HD, hl, qscale<HD>());
    load_rowfrag<HD>(df, dout + qrow * ldd + h * HD, hl, 1.0f);
    to_dfrag(qf, qd);
    to_dfrag(df, dd);
  }
  const long long si = ((long long)b * nh + h) * T + (myq < T ? myq : T - 1);
  const float L = lse[si], Dv = dvec[si];
  f16v A[NC];
#pragma unroll
  for (int i = 0; i < NC; i++)
#pragma unroll
    for (int r = 0; r < 16; r++) A[i][r] = 0.0f;
  for (int kb = w; kb <= qb; kb += KW) {
    const int k0 = kb * TB, kr = k0 + c;
    const long long krow = base + (kr < T ? kr : T - 1);
    DFrag<HD> kd, vd;
    {
      float kf[HD / 2], vf[HD / 2];
      load_rowfrag<HD>(kf, qkv + krow * ld + kcol + g * HD, hl, 1.0f);
      load_rowfrag<HD>(vf, qkv + krow * ld + vcol + g * HD, hl, 1.0f);
      to_dfrag(kf, kd);
      to_dfrag(vf, vd);
    }
    f16v S, dP;
#pragma unroll
    for (int r = 0; r < 16; r++) S[r] = dP[r] = 0.0f;
    S = mma_d(kd, qd, S);
    dP = mma_d(vd, dd, dP);
    float ds[16];
#pragma unroll
    for (int r = 0; r < 16; r++) {
      const int key = k0 + kap(r, hl);
      const float pv = (key > myq || key >= T || myq >= T) ? 0.0f : expf(S[r] - L);
      ds[r] = pv * (dP[r] - Dv);
    }
    float kk[HD / 2];
    load_kapcols<HD>(kk, qkv, base, k0, T, ld, kcol + g * HD, hl, c, 1.0f);
    KFrag dk;
    to_kfrag(ds, dk);
#pragma unroll
    for (int i = 0; i < NC; i++) {
      KFrag ki;
      to_kfrag(kk + 16 * i, ki);
      A[i] = mma_k(dk, ki, A[i]);
    }
  }
#pragma unroll
  for (int r = 0; r < 16; r++)
#pragma unroll
    for (int i = 0; i < NC; i++) As[w][kap(r, hl)][32 * i + c] = A[i][r];
  __syncthreads();
  const int qi = threadIdx.x >> 3, d0 = (threadIdx.x & 7) * (HD / 8), t = q0 + qi;
  if (t >= T) return;
  float* out = dq + (base + t) * ldq + h * HD;
#pragma unroll
  for (int d = d0; d < d0 + HD / 8; d++) {
    float v = As[0][qi][d];
#pragma unroll
    for (int u = 1; u < KW; u++) v += As[u][qi][d];
    out[d] = v * qscale<HD>();
  }
}

// dK, dV for 32 keys against query head h (kv head g = h / group): S and dP with lanes on keys. The
// 4 waves take query blocks kb + w, kb + w + 4, …; partials are summed in wave order. With group > 1
// each head's result goes to part[(b·T + key)][h][2·64] and attn_group_sum adds the group in head
// order; with group == 1 it is written in place.
template <int HD>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(HD == 64 ? 2 : 1))) attn_dkdv_kernel(const float* __restrict__ qkv, long long ld, int kcol, int vcol,
                                                        const float* __restrict__ dout, long long ldd,
                                                        const float* __restrict__ lse,
                                                        const float* __restrict__ dvec, int T, int nh, int group,
                                                        float* __restrict__ dkv, long long ldk,
                                                        float* __restrict__ part) {
  constexpr int NC = HdC<HD>::NC;
  __shared__ float Ps[KW][TB][HdC<HD>::LP];
  const int nkb = (T + TB - 1) / TB;
  const int kb = blockIdx.x, h = blockIdx.y, b = blockIdx.z, g = h / group;  // long columns first
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, hl = lane >> 5, c = lane & 31, k0 = kb * TB;
  const int mykey = k0 + c;
  const long long base = (long long)b * T, krow = base + (mykey < T ? mykey : T - 1);
  DFrag<HD> kd, vd;
  {
    float kf[HD / 2], vf[HD / 2];
    load_rowfrag<HD>(kf, qkv + krow * ld + kcol + g * HD, hl, 1.0f);
    load_rowfrag<HD>(vf, qkv + krow * ld + vcol + g * HD, hl, 1.0f);
    to_dfrag(kf, kd);
    to_dfrag(vf, vd);
  }
  f16v K[NC], V[NC];
#pragma unroll
  for (int i = 0; i < NC; i++)
#pragma unroll
    for (int r = 0; r < 16; r++) K[i][r] = V[i][r] = 0.0f;
  for (int qb = kb + w; qb < nkb; qb += KW) {
    const int q0 = qb * TB, qr = q0 + c;
    const long long qrow = base + (qr < T ? qr : T - 1);
    const long long si = ((long long)b * nh + h) * T + (qr < T ? qr : T - 1);
    const float Lq = lse[si], Dq = dvec[si];
    DFrag<HD> qd, dd;
    {
      float qa[HD / 2], da[HD / 2];
      load_rowfrag<HD>(qa, qkv + qrow * ld + h * HD, hl, qscale<HD>());
      load_rowfrag<HD>(da, dout + qrow * ldd + h * HD, hl, 1.0f);
      to_dfrag(qa, qd);
      to_dfrag(da, dd);
    }
    f16v S, dP;
#pragma unroll
    for (int r = 0; r < 16; r++) S[r] = dP[r] = 0.0f;
    S = mma_d(qd, kd, S);
    dP = mma_d(dd, vd, dP);
    // S[r] = score(query q0 + κ(r, hl), key mykey)
    float p[16], ds[16];
#pragma unroll
    for (int r = 0; r < 16; r++) {
      const int qi = kap(r, hl), q = q0 + qi;
      const float Lr = __shfl(Lq, qi), Dr = __shfl(Dq, qi);
      const float pv = (mykey > q || q >= T || mykey >= T) ? 0.0f : expf(S[r] - Lr);
      p[r] = pv;
      ds[r] = pv * (dP[r] - Dr);
    }
    float qs[HD / 2], dos[HD / 2];
    load_kapcols<HD>(qs, qkv, base, q0, T, ld, h * HD, hl, c, qscale<HD>());
    load_kapcols<HD>(dos, dout, base, q0, T, ldd, h * HD, hl, c, 1.0f);
    KFrag pf, dsf;
    to_kfrag(p, pf);
    to_kfrag(ds, dsf);
#pragma unroll
    for (int i = 0; i < NC; i++) {
      KFrag doi, qi;
      to_kfrag(dos + 16 * i, doi);
      to_kfrag(qs + 16 * i, qi);
      V[i] = mma_k(pf, doi, V[i]);
      K[i] = mma_k(dsf, qi, K[i]);
    }
  }
  // Q carried the scale, so K already holds dK = dSᵀ·Q·scale. Merge K, then V.
  const int ki = threadIdx.x >> 3, d0 = (threadIdx.x & 7) * (HD / 8), key = k0 + ki;
  float* kr = nullptr;
  float* vr = nullptr;
  if (key < T) {
    if (group == 1) {
      kr = dkv + (base + key) * ldk + kcol + g * HD;
      vr = dkv + (base + key) * ldk + vcol + g * HD;
    } else {
      kr = part + ((base + key) * nh + h) * 2 * HD;
      vr = kr + HD;
    }
  }
#pragma unroll
  for (int pass = 0; pass < 2; pass++) {
    if (pass) __syncthreads();
#pragma unroll
    for (int r = 0; r < 16; r++)
#pragma unroll
      for (int i = 0; i < NC; i++) Ps[w][kap(r, hl)][32 * i + c] = pass == 0 ? K[i][r] : V[i][r];
    __syncthreads();
    float* dst = pass == 0 ? kr : vr;
    if (dst) {
#pragma unroll
      for (int d = d0; d < d0 + HD / 8; d++) {
        float v = Ps[0][ki][d];
#pragma unroll
        for (int u = 1; u < KW; u++) v += Ps[u][ki][d];
        dst[d] = v;
      }
    }
  }
}

// dK/dV of kv head g = Σ over its group's heads, in head order (deterministic).
template <int HD>
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
  HOS_REQUIRE(hd == 64 || hd == 128, HOS_E_INVALID, "attention: head_dim must be 64 or 128");
  HOS_REQUIRE(ld % 4 == 0 && kcol % 4 == 0 && vcol % 4 == 0, HOS_E_INVALID, "attention: unaligned qkv layout");
  dim3 grid(ceil_div(T, TB), nh, B);
  if (hd == 64)
    attn_fwd_kernel<64><<<grid, 256, 0, st>>>(qkv, ld, kcol, vcol, T, nh, nh / nkv, o, ldo, lse);
  else
    attn_fwd_kernel<128><<<grid, 256, 0, st>>>(qkv, ld, kcol, vcol, T, nh, nh / nkv, o, ldo, lse);
  HOS_HIP_CHECK(hipGetLastError());
}

template <int HD>
static void attn_bwd_hd(const float* qkv, long long ld, int kcol, int vcol, const float* o, const float* dout,
                        long long ldo, const float* lse, float* dvec, int B, int T, int nh, int nkv, float* dqkv,
                        long long ldd, float* part, hipStream_t st) {
  long long n = (long long)B * nh * T;
  attn_dvec_kernel<HD><<<ceil_div(n, 256), 256, 0, st>>>(o, dout, ldo, T, nh, B, dvec);
  HOS_HIP_CHECK(hipGetLastError());
  dim3 gq(ceil_div(T, TB), nh, B);
  attn_dq_kernel<HD><<<gq, 256, 0, st>>>(qkv, ld, kcol, vcol, dout, ldo, lse, dvec, T, nh, nh / nkv, dqkv, ldd);
  HOS_HIP_CHECK(hipGetLastError());
  dim3 gk(ceil_div(T, TB), nh, B);
  attn_dkdv_kernel<HD><<<gk, 256, 0, st>>>(qkv, ld, kcol, vcol, dout, ldo, lse, dvec, T, nh, nh / nkv, dqkv, ldd, part);
  HOS_HIP_CHECK(hipGetLastError());
  if (nh != nkv) {
    long long ne = (long long)B * T * nkv * 2 * HD;
    attn_group_sum<HD><<<ceil_div(ne, 256), 256, 0, st>>>(part, B * T, nh, nkv, nh / nkv, dqkv, ldd, kcol, vcol);
    HOS_HIP_CHECK(hipGetLastError());
  }
}

void launch_attn_bwd(const float* qkv, long long ld, int kcol, int vcol, const float* o, const float* dout,
                     long long ldo, const float* lse, float* dvec, int B, int T, int nh, int nkv, int hd, float* dqkv,
                     long long ldd, float* part, hipStream_t st) {
  HOS_REQUIRE(hd == 64 || hd == 128, HOS_E_INVALID, "attention: head_dim must be 64 or 128");
  HOS_REQUIRE(nh == nkv || part != nullptr, HOS_E_INVALID, "attention: GQA backward needs a partial buffer");
  HOS_REQUIRE(ldo % 4 == 0 && ld % 4 == 0 && kcol % 4 == 0 && vcol % 4 == 0, HOS_E_INVALID, "attention: unaligned layout");
  if (hd == 64)
    attn_bwd_hd<64>(qkv, ld, kcol, vcol, o, dout, ldo, lse, dvec, B, T, nh, nkv, dqkv, ldd, part, st);
  else
    attn_bwd_hd<128>(qkv, ld, kcol, vcol, o, dout, ldo, lse, dvec, B, T, nh, nkv, dqkv, ldd, part, st);
}

}  // namespace hos
