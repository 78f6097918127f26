// Mixture-of-experts FFN plumbing (OLMoE) and QK-norm for the LoRA training step.
//
// Forward semantics follow src/forward.rs:542-572 (router logits → softmax over all experts → the top
// n_experts_used by probability → Σ p_e·SwiGLU_e(x) with the raw probabilities, OLMoE's
// norm_topk_prob = false) and :487-493 (RMSNorm of the full q / k projections before RoPE). The
// reference's PEFT model has no MoE backward; the backward here is the chain rule of that forward: the
// routing choice is piecewise constant, so gradients reach x through the experts and the probabilities.
//
// Layout: the M·K (token, expert) selections are grouped by expert into P = M·K contiguous rows (expert e
// at offsets[e] .. offsets[e] + counts[e]); a selection's row is pos[t][s]. The expert GEMMs run over those
// rows against the stacked quantized weights (launch_qgemm_grouped), and the combine / its backward go
// back to token order with fixed (selection-order) summation; an expert's rows are its selections in
// selection order (a per-expert scan, no atomics), so the whole layer is deterministic.
#include "moe.hpp"

namespace hos {
namespace {

constexpr int NB = 256;

__device__ __forceinline__ float wsum(float v) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}
__device__ __forceinline__ float bsum(float v, float* red) {
  v = wsum(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float s = 0.0f;
  for (int i = 0; i < (int)(blockDim.x >> 6); i++) s += red[i];
  __syncthreads();
  return s;
}

// ---- QK-norm (the autograd rmsnorm_eps of src/tensor.rs:2500-2544 on a column block) ----
__global__ void __launch_bounds__(NB) qknorm_fwd_kernel(float* __restrict__ buf, long long ld, int col0, int n,
                                                         const float* __restrict__ w, float eps,
                                                         float* __restrict__ pre, float* __restrict__ inv) {
  __shared__ float red[4];
  const int row = blockIdx.x;
  float* xr = buf + (long long)row * ld + col0;
  float* pr = pre + (long long)row * n;
  float ss = 0.0f;
  for (int c = threadIdx.x; c < n; c += NB) {
    const float v = xr[c];
    pr[c] = v;
    ss += v * v;
  }
  ss = bsum(ss, red) / (float)n;
  const float iv = 1.0f / sqrtf(ss + eps);
  for (int c = threadIdx.x; c < n; c += NB) xr[c] = pr[c] * iv * w[c];
  if (threadIdx.x == 0) inv[row] = iv;
}

// g ← g·w·inv − inv³·x/n·Σ(g·w·x)
__global__ void __launch_bounds__(NB) qknorm_bwd_kernel(float* __restrict__ g, long long ld, int col0, int n,
                                                         const float* __restrict__ w, const float* __restrict__ pre,
                                                         const float* __restrict__ inv) {
  __shared__ float red[4];
  const int row = blockIdx.x;
  float* gr = g + (long long)row * ld + col0;
  const float* xr = pre + (long long)row * n;
  float s = 0.0f;
  for (int c = threadIdx.x; c < n; c += NB) s += gr[c] * w[c] * xr[c];
  s = bsum(s, red);
  const float iv = inv[row];
  const float k = iv * iv * iv / (float)n * s;
  for (int c = threadIdx.x; c < n; c += NB) gr[c] = gr[c] * w[c] * iv - xr[c] * k;
}

// Register-resident variants (n % 4 == 0, n <= 4·NB·4, 16-byte aligned rows): the row is read once; the same
// per-element arithmetic (the row sums are taken per thread over float4 columns, then across the block).
__global__ void __launch_bounds__(NB) qknorm_fwd_reg_kernel(float* __restrict__ buf, long long ld, int col0, int n,
                                                             const float* __restrict__ w, float eps,
                                                             float* __restrict__ pre, float* __restrict__ inv) {
  constexpr int NV = 4;
  __shared__ float red[4];
  const int row = blockIdx.x, n4 = n >> 2;
  float4* xr = reinterpret_cast<float4*>(buf + (long long)row * ld + col0);
  float4* pr = reinterpret_cast<float4*>(pre + (long long)row * n);
  float4 v[NV];
  float ss = 0.0f;
#pragma unroll
  for (int j = 0; j < NV; j++) {
    const int i = threadIdx.x + NB * j;
    if (i < n4) {
      v[j] = xr[i];
      pr[i] = v[j];
      ss += v[j].x * v[j].x;
      ss += v[j].y * v[j].y;
      ss += v[j].z * v[j].z;
      ss += v[j].w * v[j].w;
    }
  }
  ss = bsum(ss, red) / (float)n;
  const float iv = 1.0f / sqrtf(ss + eps);
#pragma unroll
  for (int j = 0; j < NV; j++) {
    const int i = threadIdx.x + NB * j;
    if (i < n4) {
      const float4 wv = reinterpret_cast<const float4*>(w)[i];
      xr[i] = make_float4(v[j].x * iv * wv.x, v[j].y * iv * wv.y, v[j].z * iv * wv.z, v[j].w * iv * wv.w);
    }
  }
  if (threadIdx.x == 0) inv[row] = iv;
}
__global__ void __launch_bounds__(NB) qknorm_bwd_reg_kernel(float* __restrict__ g, long long ld, int col0, int n,
                                                             const float* __restrict__ w,
                                                             const float* __restrict__ pre,
                                                             const float* __restrict__ inv) {
  constexpr int NV = 4;
  __shared__ float red[4];
  const int row = blockIdx.x, n4 = n >> 2;
  float4* gr = reinterpret_cast<float4*>(g + (long long)row * ld + col0);
  const float4* xr = reinterpret_cast<const float4*>(pre + (long long)row * n);
  float4 gw[NV], xv[NV];
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < NV; j++) {
    const int i = threadIdx.x + NB * j;
    if (i < n4) {
      const float4 gv = gr[i], wv = reinterpret_cast<const float4*>(w)[i];
      xv[j] = xr[i];
      gw[j] = make_float4(gv.x * wv.x, gv.y * wv.y, gv.z * wv.z, gv.w * wv.w);
      s += gw[j].x * xv[j].x;
      s += gw[j].y * xv[j].y;
      s += gw[j].z * xv[j].z;
      s += gw[j].w * xv[j].w;
    }
  }
  s = bsum(s, red);
  const float iv = inv[row];
  const float k = iv * iv * iv / (float)n * s;
#pragma unroll
  for (int j = 0; j < NV; j++) {
    const int i = threadIdx.x + NB * j;
    if (i < n4)
      gr[i] = make_float4(gw[j].x * iv - xv[j].x * k, gw[j].y * iv - xv[j].y * k, gw[j].z * iv - xv[j].z * k,
                          gw[j].w * iv - xv[j].w * k);
  }
}

// ---- router: one wave per token, lane j = expert j (E ≤ 64) ----
__global__ void __launch_bounds__(256) moe_route_kernel(const float* __restrict__ logits, int M, int E, int K,
                                                        float* __restrict__ pfull, int* __restrict__ sel_e,
                                                        float* __restrict__ sel_p) {
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6), j = threadIdx.x & 63;
  if (t >= M) return;
  const bool on = j < E;
  const float l = on ? logits[(long long)t * E + j] : -INFINITY;
  float mx = l;
  for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
  const float ex = on ? expf(l - mx) : 0.0f;
  const float p = ex / wsum(ex);
  if (on) pfull[(long long)t * E + j] = p;
  // top K: repeated arg-max, ties to the lower expert (the stable descending sort of the reference). A NaN
  // probability (diverged logits) ranks below every number but above taken lanes, so each slot is still
  // written exactly once with a distinct in-range expert and the NaN reaches the loss, not an index.
  bool taken = !on;
  for (int s = 0; s < K; s++) {
    float bv = taken ? -2.0f : (p != p ? -1.0f : p);
    int bi = taken ? 64 : j;
    for (int o = 32; o > 0; o >>= 1) {
      const float ov = __shfl_xor(bv, o);
      const int oi = __shfl_xor(bi, o);
      if (ov > bv || (ov == bv && oi < bi)) {
        bv = ov;
        bi = oi;
      }
    }
    if (j == bi) {
      taken = true;
      const long long q = (long long)t * K + s;
      sel_e[q] = j;
      sel_p[q] = p;
    }
  }
}

// Rows of expert e: one workgroup per expert ranks its selections in selection order (token, then slot):
// slot[q] = #{q' < q : sel_e[q'] = e}, counts[e] = the total. Each wave takes a contiguous quarter of the
// selections, 64 at a time (coalesced loads, ballot + popcount ranks). Deterministic, no atomics.
constexpr int SLOT_NW = 16;  // waves per workgroup
__global__ void __launch_bounds__(64 * SLOT_NW) moe_slot_kernel(const int* __restrict__ sel_e, int P,
                                                                int* __restrict__ slot, int* __restrict__ counts) {
  __shared__ int wsum[SLOT_NW];
  const int e = blockIdx.x, lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int per = (P + 64 * SLOT_NW - 1) / (64 * SLOT_NW) * 64, q0 = w * per, q1 = min(P, q0 + per);
  constexpr int NB8 = 8;  // 64-selection groups whose loads are issued together
  int c = 0;
  for (int qb = q0; qb < q1; qb += 64 * NB8) {
    bool f[NB8];
#pragma unroll
    for (int i = 0; i < NB8; i++) {
      const int q = qb + 64 * i + lane;
      f[i] = q < q1 && sel_e[q] == e;
    }
#pragma unroll
    for (int i = 0; i < NB8; i++) c += __popcll(__ballot(f[i]));
  }
  if (lane == 0) wsum[w] = c;
  __syncthreads();
  int r = 0;
  for (int i = 0; i < w; i++) r += wsum[i];
  const unsigned long long below = (1ull << lane) - 1ull;
  for (int qb = q0; qb < q1; qb += 64 * NB8) {
    bool f[NB8];
#pragma unroll
    for (int i = 0; i < NB8; i++) {
      const int q = qb + 64 * i + lane;
      f[i] = q < q1 && sel_e[q] == e;
    }
#pragma unroll
    for (int i = 0; i < NB8; i++) {
      const unsigned long long m = __ballot(f[i]);
      if (f[i]) slot[qb + 64 * i + lane] = r + __popcll(m & below);
      r += __popcll(m);
    }
  }
  if (threadIdx.x == 0) {
    int tot = 0;
    for (int i = 0; i < SLOT_NW; i++) tot += wsum[i];
    counts[e] = tot;
  }
}

// One wave, lane e = expert e (E <= 64): exclusive scans of the row counts (→ offsets) and of the tile counts
// (→ each expert's first schedule entry), each lane writing its expert's tiles, then the unused tail = −1.
__global__ void __launch_bounds__(64) moe_plan_kernel(const int* __restrict__ counts, int E,
                                                      int* __restrict__ offsets, int* __restrict__ tiles,
                                                      int max_tiles) {
  const int e = threadIdx.x;
  const int n = e < E ? counts[e] : 0, nt = (n + GROUP_BM - 1) / GROUP_BM;
  int off = n, t0 = nt;  // inclusive scans
  for (int o = 1; o < 64; o <<= 1) {
    const int a = __shfl_up(off, o), b = __shfl_up(t0, o);
    if (e >= o) {
      off += a;
      t0 += b;
    }
  }
  const int total = __shfl(off, 63), ttot = __shfl(t0, 63);
  off -= n;
  t0 -= nt;
  if (e < E) offsets[e] = off;
  if (e == 0) offsets[E] = total;
  for (int i = 0; i < nt; i++) {
    const int ti = t0 + i;
    if (ti < max_tiles) {
      tiles[3 * ti] = e;
      tiles[3 * ti + 1] = off + i * GROUP_BM;
      tiles[3 * ti + 2] = min(GROUP_BM, n - i * GROUP_BM);
    }
  }
  for (int i = ttot + e; i < max_tiles; i += 64) tiles[3 * i] = -1;
}

// one workgroup per selection: copy the token's operand row (hi, lo, row scale) to its expert-order row
// (8 halves per 16-byte access: d and both row strides multiples of 8, checked by the launcher)
__global__ void __launch_bounds__(NB) moe_gather_kernel(H16 src, long long lds, const int* __restrict__ sel_e,
                                                         const int* __restrict__ slot, const int* __restrict__ offsets,
                                                         int K, int d, int* __restrict__ pos, H16 dst, long long ldd) {
  const long long q = blockIdx.x;
  const int t = (int)(q / K);
  const int p = offsets[sel_e[q]] + slot[q];
  if (threadIdx.x == 0) {
    pos[q] = p;
    dst.rinv[p] = src.rinv[t];
  }
  const int d8 = d >> 3;
  const int4* sh = reinterpret_cast<const int4*>(src.data + (long long)t * lds);
  int4* dh = reinterpret_cast<int4*>(dst.data + (long long)p * ldd);
  for (int c = threadIdx.x; c < d8; c += NB) dh[c] = sh[c];
  if (dst.lo) {
    const int4* sl = reinterpret_cast<const int4*>(src.lo + (long long)t * lds);
    int4* dl = reinterpret_cast<int4*>(dst.lo + (long long)p * ldd);
    for (int c = threadIdx.x; c < d8; c += NB) dl[c] = sl[c];
  }
}

// one thread per 4 consecutive output columns (d % 4 == 0, checked by the launcher); per element the same
// selection-order sum as a scalar loop
__global__ void moe_combine_kernel(const float* __restrict__ Y, const int* __restrict__ pos,
                                   const float* __restrict__ sel_p, const float* __restrict__ resid, int M, int K,
                                   int d, float* __restrict__ out) {
#pragma clang fp contract(off)
  const int d4 = d >> 2;
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long long)M * d4) return;
  const int t = (int)(i / d4), c = 4 * (int)(i % d4);
  float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  for (int s = 0; s < K; s++) {
    const float w = sel_p[t * K + s];
    const float4 y = *reinterpret_cast<const float4*>(Y + (long long)pos[t * K + s] * d + c);
    acc.x += w * y.x;
    acc.y += w * y.y;
    acc.z += w * y.z;
    acc.w += w * y.w;
  }
  const float4 r = *reinterpret_cast<const float4*>(resid + (long long)t * d + c);
  *reinterpret_cast<float4*>(out + (long long)t * d + c) = make_float4(r.x + acc.x, r.y + acc.y, r.z + acc.z, r.w + acc.w);
}

// one workgroup per selection (float4 columns, d % 4 == 0)
__global__ void __launch_bounds__(NB) moe_combine_bwd_kernel(const float* __restrict__ g, const float* __restrict__ Y,
                                                              const int* __restrict__ pos,
                                                              const float* __restrict__ sel_p, int K, int d,
                                                              float* __restrict__ dY, float* __restrict__ dp) {
  __shared__ float red[4];
  const long long q = blockIdx.x;
  const int t = (int)(q / K);
  const long long p = pos[q];
  const float w = sel_p[q];
  const float4* gr = reinterpret_cast<const float4*>(g + (long long)t * d);
  const float4* yr = reinterpret_cast<const float4*>(Y + p * d);
  float4* dr = reinterpret_cast<float4*>(dY + p * d);
  float s = 0.0f;
  for (int c = threadIdx.x; c < (d >> 2); c += NB) {
    const float4 gv = gr[c], yv = yr[c];
    dr[c] = make_float4(w * gv.x, w * gv.y, w * gv.z, w * gv.w);
    s += yv.x * gv.x;
    s += yv.y * gv.y;
    s += yv.z * gv.z;
    s += yv.w * gv.w;
  }
  s = bsum(s, red);
  if (threadIdx.x == 0) dp[q] = s;
}

// The same backward writing dY straight as the fp16 row-scaled GEMM operand (hi, lo, 1/scale) of the expert
// dX GEMM instead of f32: the row held in registers (d % 4 == 0, d <= 4·NB·4); scale and rounding as the
// f32 → fp16 conversion applies them to the f32 row.
typedef _Float16 moe_h16x4 __attribute__((ext_vector_type(4)));
__global__ void __launch_bounds__(NB) moe_combine_bwd_h16_kernel(const float* __restrict__ g,
                                                                  const float* __restrict__ Y,
                                                                  const int* __restrict__ pos,
                                                                  const float* __restrict__ sel_p, int K, int d,
                                                                  H16 out, float* __restrict__ dp) {
  constexpr int NV = 4;
  __shared__ float red[4];
  const long long q = blockIdx.x;
  const int t = (int)(q / K), d4 = d >> 2;
  const long long p = pos[q];
  const float w = sel_p[q];
  const float4* gr = reinterpret_cast<const float4*>(g + (long long)t * d);
  const float4* yr = reinterpret_cast<const float4*>(Y + p * d);
  float4 v[NV];
  float s = 0.0f, amax = 0.0f;
#pragma unroll
  for (int j = 0; j < NV; j++) {
    const int i = threadIdx.x + NB * j;
    if (i < d4) {
      const float4 gv = gr[i], yv = yr[i];
      v[j] = make_float4(w * gv.x, w * gv.y, w * gv.z, w * gv.w);
      s += yv.x * gv.x;
      s += yv.y * gv.y;
      s += yv.z * gv.z;
      s += yv.w * gv.w;
      amax = fmaxf(fmaxf(amax, fmaxf(fabsf(v[j].x), fabsf(v[j].y))), fmaxf(fabsf(v[j].z), fabsf(v[j].w)));
    }
  }
  s = bsum(s, red);
  if (threadIdx.x == 0) dp[q] = s;
  for (int o = 32; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  int e = 0;
  if (amax > 0.0f && amax < 3.0e38f) {
    int ex;
    frexpf(amax, &ex);
    e = 15 - ex;
    e = e > 100 ? 100 : (e < -100 ? -100 : e);
  }
  const float sc = ldexpf(1.0f, e);
  if (threadIdx.x == 0) out.rinv[p] = ldexpf(1.0f, -e);
#pragma unroll
  for (int j = 0; j < NV; j++) {
    const int i = threadIdx.x + NB * j;
    if (i < d4) {
      const float a = v[j].x * sc, b = v[j].y * sc, c = v[j].z * sc, dd = v[j].w * sc;
      const moe_h16x4 h{(_Float16)a, (_Float16)b, (_Float16)c, (_Float16)dd};
      *reinterpret_cast<moe_h16x4*>(out.data + p * d + 4 * i) = h;
      if (out.lo) {
        const moe_h16x4 l{(_Float16)(a - (float)h.x), (_Float16)(b - (float)h.y), (_Float16)(c - (float)h.z),
                          (_Float16)(dd - (float)h.w)};
        *reinterpret_cast<moe_h16x4*>(out.lo + p * d + 4 * i) = l;
      }
    }
  }
}

__global__ void __launch_bounds__(256) moe_router_bwd_kernel(const float* __restrict__ pfull,
                                                             const float* __restrict__ dp,
                                                             const int* __restrict__ sel_e, int M, int E, int K,
                                                             float* __restrict__ dlogits) {
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6), j = threadIdx.x & 63;
  if (t >= M) return;
  float dpj = 0.0f;
  for (int s = 0; s < K; s++)
    if (sel_e[t * K + s] == j) dpj = dp[t * K + s];
  const float p = j < E ? pfull[(long long)t * E + j] : 0.0f;
  const float S = wsum(p * dpj);
  if (j < E) dlogits[(long long)t * E + j] = p * (dpj - S);
}

// one thread per 4 consecutive columns (d % 4 == 0); per element the selection-order sum
__global__ void moe_gather_sum_kernel(const float* __restrict__ dX, const int* __restrict__ pos, int M, int K, int d,
                                      float* __restrict__ dxn) {
  const int d4 = d >> 2;
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long long)M * d4) return;
  const int t = (int)(i / d4), c = 4 * (int)(i % d4);
  float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  for (int s = 0; s < K; s++) {
    const float4 v = *reinterpret_cast<const float4*>(dX + (long long)pos[t * K + s] * d + c);
    acc.x += v.x;
    acc.y += v.y;
    acc.z += v.z;
    acc.w += v.w;
  }
  *reinterpret_cast<float4*>(dxn + (long long)t * d + c) = acc;
}

__global__ void fill_i32_kernel(int* p, long long n, int v) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

}  // namespace

void launch_qknorm_fwd(float* buf, long long ld, int col0, int n, const float* w, float eps, int M, float* pre,
                       float* inv, hipStream_t st) {
  if (M <= 0) return;
  auto al = [](const void* p) { return ((uintptr_t)p % 16) == 0; };
  if (n % 4 == 0 && n <= 4 * NB * 4 && ld % 4 == 0 && col0 % 4 == 0 && al(buf) && al(w) && al(pre))
    qknorm_fwd_reg_kernel<<<M, NB, 0, st>>>(buf, ld, col0, n, w, eps, pre, inv);
  else
    qknorm_fwd_kernel<<<M, NB, 0, st>>>(buf, ld, col0, n, w, eps, pre, inv);
  HOS_HIP_CHECK(hipGetLastError());
}
void launch_qknorm_bwd(float* g, long long ld, int col0, int n, const float* w, const float* pre, const float* inv,
                       int M, hipStream_t st) {
  if (M <= 0) return;
  auto al = [](const void* p) { return ((uintptr_t)p % 16) == 0; };
  if (n % 4 == 0 && n <= 4 * NB * 4 && ld % 4 == 0 && col0 % 4 == 0 && al(g) && al(w) && al(pre))
    qknorm_bwd_reg_kernel<<<M, NB, 0, st>>>(g, ld, col0, n, w, pre, inv);
  else
    qknorm_bwd_kernel<<<M, NB, 0, st>>>(g, ld, col0, n, w, pre, inv);
  HOS_HIP_CHECK(hipGetLastError());
}
void launch_moe_route(const float* logits, int M, int E, int K, float* pfull, int* sel_e, float* sel_p, int* slot,
                      int* counts, hipStream_t st) {
  HOS_REQUIRE(E >= 1 && E <= 64 && K >= 1 && K <= E, HOS_E_INVALID, "moe: need 1 <= experts used <= experts <= 64");
  if (M <= 0) return;
  moe_route_kernel<<<ceil_div(M, 4), 256, 0, st>>>(logits, M, E, K, pfull, sel_e, sel_p);
  HOS_HIP_CHECK(hipGetLastError());
  moe_slot_kernel<<<E, 64 * SLOT_NW, 0, st>>>(sel_e, M * K, slot, counts);
  HOS_HIP_CHECK(hipGetLastError());
}
void launch_moe_plan(const int* counts, int E, int* offsets, int* tiles, int max_tiles, hipStream_t st) {
  moe_plan_kernel<<<1, 64, 0, st>>>(counts, E, offsets, tiles, max_tiles);
  HOS_HIP_CHECK(hipGetLastError());
}
void launch_moe_gather(H16 src, long long lds, const int* sel_e, const int* slot, const int* offsets, int M, int K,
                       int d, int* pos, H16 dst, long long ldd, hipStream_t st) {
  if (M <= 0) return;
  HOS_REQUIRE(d % 8 == 0 && lds % 8 == 0 && ldd % 8 == 0, HOS_E_INVALID, "moe_gather: d and strides must be multiples of 8");
  moe_gather_kernel<<<(unsigned)((long long)M * K), NB, 0, st>>>(src, lds, sel_e, slot, offsets, K, d, pos, dst, ldd);
  HOS_HIP_CHECK(hipGetLastError());
}
void launch_moe_combine(const float* Y, const int* pos, const float* sel_p, const float* resid, int M, int K, int d,
                        float* out, hipStream_t st) {
  const long long n = (long long)M * (d / 4);
  if (n <= 0) return;
  HOS_REQUIRE(d % 4 == 0, HOS_E_INVALID, "moe_combine: d must be a multiple of 4");
  moe_combine_kernel<<<ceil_div(n, 256), 256, 0, st>>>(Y, pos, sel_p, resid, M, K, d, out);
  HOS_HIP_CHECK(hipGetLastError());
}
void launch_moe_combine_bwd(const float* g, const float* Y, const int* pos, const float* sel_p, int M, int K, int d,
                            float* dY, float* dp, hipStream_t st) {
  if (M <= 0) return;
  HOS_REQUIRE(d % 4 == 0, HOS_E_INVALID, "moe_combine: d must be a multiple of 4");
  moe_combine_bwd_kernel<<<(unsigned)((long long)M * K), NB, 0, st>>>(g, Y, pos, sel_p, K, d, dY, dp);
  HOS_HIP_CHECK(hipGetLastError());
}
bool moe_combine_bwd_h16_ok(int d) { return d % 4 == 0 && d <= 4 * NB * 4; }
void launch_moe_combine_bwd_h16(const float* g, const float* Y, const int* pos, const float* sel_p, int M, int K,
                                int d, H16 out, float* dp, hipStream_t st) {
  if (M <= 0) return;
  HOS_REQUIRE(moe_combine_bwd_h16_ok(d), HOS_E_INVALID, "moe_combine_bwd_h16: d must be a multiple of 4, <= 4096");
  moe_combine_bwd_h16_kernel<<<(unsigned)((long long)M * K), NB, 0, st>>>(g, Y, pos, sel_p, K, d, out, dp);
  HOS_HIP_CHECK(hipGetLastError());
}
void launch_moe_router_bwd(const float* pfull, const float* dp, const int* sel_e, int M, int E, int K, float* dlogits,
                           hipStream_t st) {
  if (M <= 0) return;
  moe_router_bwd_kernel<<<ceil_div(M, 4), 256, 0, st>>>(pfull, dp, sel_e, M, E, K, dlogits);
  HOS_HIP_CHECK(hipGetLastError());
}
void launch_moe_gather_sum(const float* dX, const int* pos, int M, int K, int d, float* dxn, hipStream_t st) {
  const long long n = (long long)M * (d / 4);
  if (n <= 0) return;
  HOS_REQUIRE(d % 4 == 0, HOS_E_INVALID, "moe_gather_sum: d must be a multiple of 4");
  moe_gather_sum_kernel<<<ceil_div(n, 256), 256, 0, st>>>(dX, pos, M, K, d, dxn);
  HOS_HIP_CHECK(hipGetLastError());
}
void launch_fill_i32(int* p, long long n, int v, hipStream_t st) {
  if (n <= 0) return;
  fill_i32_kernel<<<ceil_div(n, 256), 256, 0, st>>>(p, n, v);
  HOS_HIP_CHECK(hipGetLastError());
}

}  // namespace hos
