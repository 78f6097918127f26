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
// 1/√64 = 2^-3 is folded into q exactly.
//
// MFMA layout used throughout (32×32 tiles, here of v_mfma_f32_32x32x16_bf16 on hi/lo-split operands): the D matrix X[i][j] sits with column j = lane%32 and
// rows i = 8·(r/4) + 4·(lane/32) + r%4 in register r. Read back as an A operand, register r of that
// layout supplies row (lane%32) of Xᵀ at contraction index κ(r, lane/32) = 8·(r/4) + 4·(lane/32) + r%4,
// so a score tile feeds the next MFMA straight from registers provided the other operand is gathered
// in the same κ order. Per wave: 32 queries (or keys) × 64 head dims; 4 waves per workgroup split the
// other sequence axis and merge in LDS, so there is no workgroup barrier inside the main loops.
#include "fused.hpp"

namespace hos {
namespace {

constexpr int HD = 64, TB = 32, KW = 4, LP = HD + 1;  // head dim, tile rows, waves per workgroup, LDS row

__device__ __forceinline__ int kap(int s, int h) { return 8 * (s >> 2) + 4 * h + (s & 3); }

// Fragment of one row for a contraction over the 64 head dims: frag[4j + e] = row[8j + 4·hl + e]·mul.
// Any bijection of the contraction index works as long as both MFMA operands use it; this one lets a
// lane fetch its 32 values as 8 float4.
__device__ __forceinline__ void load_rowfrag(float* frag, const float* __restrict__ row, int hl, float mul) {
#pragma unroll
  for (int j = 0; j < 8; j++) {
    const float4 v = *reinterpret_cast<const float4*>(row + 8 * j + 4 * hl);
    frag[4 * j] = v.x * mul;
    frag[4 * j + 1] = v.y * mul;
    frag[4 * j + 2] = v.z * mul;
    frag[4 * j + 3] = v.w * mul;
  }
}

// B operand over 32 rows indexed in κ order: col[s] = X[r0 + κ(s, hl)][c], col[16 + s] = …[32 + c].
__device__ __forceinline__ void load_kapcols(float* col, const float* __restrict__ src, long long base_row, int r0,
                                             int T, long long ld, int off, int hl, int c, float mul) {
#pragma unroll
  for (int s = 0; s < 16; s++) {
    const int t = r0 + kap(s, hl);
    const float* row = src + (base_row + (t < T ? t : T - 1)) * ld + off;
    col[s] = row[c] * mul;
    col[16 + s] = row[32 + c] * mul;
  }
}

// ---- bf16 hi/lo products: x = hi + lo with hi = bf16(x), lo = bf16(x − hi) (x − hi is exact in f32), and
// a·b ≈ a_hi·b_hi + a_hi·b_lo + a_lo·b_hi on v_mfma_f32_32x32x16_bf16 — relative error ~2^-16 per product
// (the dropped a_lo·b_lo and the rounding of lo), fp32 accumulation, f32 exponent range (no scaling of
// tiny gradients), at 5.3× the throughput of fp32 MFMA per contraction element.
// A 64-dim row fragment (rowfrag order) as 4 contraction steps of 8 values per lane.
struct DFrag {
  bf8 h[4], l[4];
};
__device__ __forceinline__ void to_dfrag(const float* f, DFrag& F) {
#pragma unroll
  for (int t = 0; t < 4; t++)
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
// Σ over the 64 head dims: D[i][j] += A_row_i · B_row_j (both in rowfrag order)
__device__ __forceinline__ f16v mma_d(const DFrag& a, const DFrag& b, f16v c) {
#pragma unroll
  for (int t = 0; t < 4; t++) c = mma3(a.h[t], a.l[t], b.h[t], b.l[t], c);
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
__global__ void __launch_bounds__(256) attn_fwd_kernel(const float* __restrict__ qkv, long long ld, int kcol, int vcol,
                                                       int T, int nh, int group, float* __restrict__ o, long long ldo,
                                                       float* __restrict__ lse) {
  __shared__ float Os[KW][TB][LP];
  __shared__ float Ms[KW][TB], Ls[KW][TB];
  const int nqb = (T + TB - 1) / TB;
  const int qb = nqb - 1 - (int)blockIdx.x, h = blockIdx.y, b = blockIdx.z, g = h / group;  // long rows first
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, hl = lane >> 5, c = lane & 31, q0 = qb * TB;
  const int myq = q0 + c;  // this lane's query in the Sᵀ layout
  const long long base = (long long)b * T;
  DFrag qd;
  {
    float qf[32];
    load_rowfrag(qf, qkv + (base + (myq < T ? myq : T - 1)) * ld + h * HD, hl, 0.125f);
    to_dfrag(qf, qd);
  }
  f16v O0, O1;
#pragma unroll
  for (int r = 0; r < 16; r++) O0[r] = O1[r] = 0.0f;
  float m = -INFINITY, l = 0.0f;
  for (int kb = w; kb <= qb; kb += KW) {
    const int k0 = kb * TB, kr = k0 + c;
    float kf[32], vv[32];
    load_rowfrag(kf, qkv + (base + (kr < T ? kr : T - 1)) * ld + kcol + g * HD, hl, 1.0f);
    load_kapcols(vv, qkv, base, k0, T, ld, vcol + g * HD, hl, c, 1.0f);
    DFrag kd;
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
      O0[r] *= a;
      O1[r] *= a;
    }
    KFrag pk, v0, v1;
    to_kfrag(p, pk);
    to_kfrag(vv, v0);
    to_kfrag(vv + 16, v1);
    O0 = mma_k(pk, v0, O0);
    O1 = mma_k(pk, v1, O1);
  }
  if (hl == 0) {
    Ms[w][c] = m;
    Ls[w][c] = l;
  }
#pragma unroll
  for (int r = 0; r < 16; r++) {
    Os[w][kap(r, hl)][c] = O0[r];
    Os[w][kap(r, hl)][32 + c] = O1[r];
  }
  __syncthreads();
  // merge the four states: thread → (query tid/8, dims 8·(tid%8) .. +8)
  const int qi = threadIdx.x >> 3, d0 = (threadIdx.x & 7) * 8, t = q0 + qi;
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
  for (int d = d0; d < d0 + 8; d++) {
    float num = 0.0f;
#pragma unroll
    for (int v = 0; v < KW; v++) num += Os[v][qi][d] * e[v];
    orow[d] = num * inv;
  }
  if (d0 == 0) lse[((long long)b * nh + h) * T + t] = mx + logf(den);
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

// dQ for 32 queries of head h: Sᵀ and dPᵀ with lanes on queries, dQ = (dS·K)·2^-3. The 4 waves take
// key blocks w, w+4, …; their partial dQ are summed in wave order.
__global__ void __launch_bounds__(256) attn_dq_kernel(const float* __restrict__ qkv, long long ld, int kcol, int vcol,
                                                      const float* __restrict__ dout, long long ldd,
                                                      const float* __restrict__ lse, const float* __restrict__ dvec,
                                                      int T, int nh, int group, float* __restrict__ dq,
                                                      long long ldq) {
  __shared__ float As[KW][TB][LP];
  const int nqb = (T + TB - 1) / TB;
  const int qb = nqb - 1 - (int)blockIdx.x, h = blockIdx.y, b = blockIdx.z, g = h / group;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, hl = lane >> 5, c = lane & 31, q0 = qb * TB;
  const int myq = q0 + c;
  const long long base = (long long)b * T, qrow = base + (myq < T ? myq : T - 1);
  DFrag qd, dd;
  {
    float qf[32], df[32];
    load_rowfrag(qf, qkv + qrow * ld + h * HD, hl, 0.125f);
    load_rowfrag(df, dout + qrow * ldd + h * HD, hl, 1.0f);
    to_dfrag(qf, qd);
    to_dfrag(df, dd);
  }
  const long long si = ((long long)b * nh + h) * T + (myq < T ? myq : T - 1);
  const float L = lse[si], Dv = dvec[si];
  f16v A0, A1;
#pragma unroll
  for (int r = 0; r < 16; r++) A0[r] = A1[r] = 0.0f;
  for (int kb = w; kb <= qb; kb += KW) {
    const int k0 = kb * TB, kr = k0 + c;
    const long long krow = base + (kr < T ? kr : T - 1);
    DFrag kd, vd;
    {
      float kf[32], vf[32];
      load_rowfrag(kf, qkv + krow * ld + kcol + g * HD, hl, 1.0f);
      load_rowfrag(vf, qkv + krow * ld + vcol + g * HD, hl, 1.0f);
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
    float kk[32];
    load_kapcols(kk, qkv, base, k0, T, ld, kcol + g * HD, hl, c, 1.0f);
    KFrag dk, k0f, k1f;
    to_kfrag(ds, dk);
    to_kfrag(kk, k0f);
    to_kfrag(kk + 16, k1f);
    A0 = mma_k(dk, k0f, A0);
    A1 = mma_k(dk, k1f, A1);
  }
#pragma unroll
  for (int r = 0; r < 16; r++) {
    As[w][kap(r, hl)][c] = A0[r];
    As[w][kap(r, hl)][32 + c] = A1[r];
  }
  __syncthreads();
  const int qi = threadIdx.x >> 3, d0 = (threadIdx.x & 7) * 8, t = q0 + qi;
  if (t >= T) return;
  float* out = dq + (base + t) * ldq + h * HD;
#pragma unroll
  for (int d = d0; d < d0 + 8; d++) {
    float v = As[0][qi][d];
#pragma unroll
    for (int u = 1; u < KW; u++) v += As[u][qi][d];
    out[d] = v * 0.125f;
  }
}

// dK, dV for 32 keys against query head h (kv head g = h / group): S and dP with lanes on keys. The
// 4 waves take query blocks kb + w, kb + w + 4, …; partials are summed in wave order. With group > 1
// each head's result goes to part[(b·T + key)][h][2·64] and attn_group_sum adds the group in head
// order; with group == 1 it is written in place.
__global__ void __launch_bounds__(256) attn_dkdv_kernel(const float* __restrict__ qkv, long long ld, int kcol, int vcol,
                                                        const float* __restrict__ dout, long long ldd,
                                                        const float* __restrict__ lse,
                                                        const float* __restrict__ dvec, int T, int nh, int group,
                                                        float* __restrict__ dkv, long long ldk,
                                                        float* __restrict__ part) {
  __shared__ float Ps[KW][TB][LP];
  const int nkb = (T + TB - 1) / TB;
  const int kb = blockIdx.x, h = blockIdx.y, b = blockIdx.z, g = h / group;  // long columns first
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, hl = lane >> 5, c = lane & 31, k0 = kb * TB;
  const int mykey = k0 + c;
  const long long base = (long long)b * T, krow = base + (mykey < T ? mykey : T - 1);
  DFrag kd, vd;
  {
    float kf[32], vf[32];
    load_rowfrag(kf, qkv + krow * ld + kcol + g * HD, hl, 1.0f);
    load_rowfrag(vf, qkv + krow * ld + vcol + g * HD, hl, 1.0f);
    to_dfrag(kf, kd);
    to_dfrag(vf, vd);
  }
  f16v K0, K1, V0, V1;
#pragma unroll
  for (int r = 0; r < 16; r++) K0[r] = K1[r] = V0[r] = V1[r] = 0.0f;
  for (int qb = kb + w; qb < nkb; qb += KW) {
    const int q0 = qb * TB, qr = q0 + c;
    const long long qrow = base + (qr < T ? qr : T - 1);
    const long long si = ((long long)b * nh + h) * T + (qr < T ? qr : T - 1);
    const float Lq = lse[si], Dq = dvec[si];
    DFrag qd, dd;
    {
      float qa[32], da[32];
      load_rowfrag(qa, qkv + qrow * ld + h * HD, hl, 0.125f);
      load_rowfrag(da, dout + qrow * ldd + h * HD, hl, 1.0f);
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
    float qs[32], dos[32];
    load_kapcols(qs, qkv, base, q0, T, ld, h * HD, hl, c, 0.125f);
    load_kapcols(dos, dout, base, q0, T, ldd, h * HD, hl, c, 1.0f);
    KFrag pf, dsf, do0, do1, q0f, q1f;
    to_kfrag(p, pf);
    to_kfrag(ds, dsf);
    to_kfrag(dos, do0);
    to_kfrag(dos + 16, do1);
    to_kfrag(qs, q0f);
    to_kfrag(qs + 16, q1f);
    V0 = mma_k(pf, do0, V0);
    V1 = mma_k(pf, do1, V1);
    K0 = mma_k(dsf, q0f, K0);
    K1 = mma_k(dsf, q1f, K1);
  }
  // Q carried the 2^-3 scale, so K0/K1 already hold dK = dSᵀ·Q·scale. Merge K, then V.
  const int ki = threadIdx.x >> 3, d0 = (threadIdx.x & 7) * 8, key = k0 + ki;
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
    const f16v& X0 = pass == 0 ? K0 : V0;
    const f16v& X1 = pass == 0 ? K1 : V1;
    if (pass) __syncthreads();
#pragma unroll
    for (int r = 0; r < 16; r++) {
      Ps[w][kap(r, hl)][c] = X0[r];
      Ps[w][kap(r, hl)][32 + c] = X1[r];
    }
    __syncthreads();
    float* dst = pass == 0 ? kr : vr;
    if (dst) {
#pragma unroll
      for (int d = d0; d < d0 + 8; d++) {
        float v = Ps[0][ki][d];
#pragma unroll
        for (int u = 1; u < KW; u++) v += Ps[u][ki][d];
        dst[d] = v;
      }
    }
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
  attn_fwd_kernel<<<grid, 256, 0, st>>>(qkv, ld, kcol, vcol, T, nh, nh / nkv, o, ldo, lse);
  HOS_HIP_CHECK(hipGetLastError());
}

void launch_attn_bwd(const float* qkv, long long ld, int kcol, int vcol, const float* o, const float* dout,
                     long long ldo, const float* lse, float* dvec, int B, int T, int nh, int nkv, int hd, float* dqkv,
                     long long ldd, float* part, hipStream_t st) {
  HOS_REQUIRE(hd == HD, HOS_E_INVALID, "attention: head_dim must be 64");
  HOS_REQUIRE(nh == nkv || part != nullptr, HOS_E_INVALID, "attention: GQA backward needs a partial buffer");
  HOS_REQUIRE(ldo % 4 == 0 && ld % 4 == 0 && kcol % 4 == 0 && vcol % 4 == 0, HOS_E_INVALID, "attention: unaligned layout");
  long long n = (long long)B * nh * T;
  attn_dvec_kernel<<<ceil_div(n, 256), 256, 0, st>>>(o, dout, ldo, T, nh, B, dvec);
  HOS_HIP_CHECK(hipGetLastError());
  dim3 gq(ceil_div(T, TB), nh, B);
  attn_dq_kernel<<<gq, 256, 0, st>>>(qkv, ld, kcol, vcol, dout, ldo, lse, dvec, T, nh, nh / nkv, dqkv, ldd);
  HOS_HIP_CHECK(hipGetLastError());
  dim3 gk(ceil_div(T, TB), nh, B);
  attn_dkdv_kernel<<<gk, 256, 0, st>>>(qkv, ld, kcol, vcol, dout, ldo, lse, dvec, T, nh, nh / nkv, dqkv, ldd, part);
  HOS_HIP_CHECK(hipGetLastError());
  if (nh != nkv) {
    long long ne = (long long)B * T * nkv * 2 * HD;
    attn_group_sum<<<ceil_div(ne, 256), 256, 0, st>>>(part, B * T, nh, nkv, nh / nkv, dqkv, ldd, kcol, vcol);
    HOS_HIP_CHECK(hipGetLastError());
  }
}

}  // namespace hos
