// Bandwidth-bound fused kernels of the LoRA training step (one workgroup per row where a row
// reduction is needed; wave64 shuffle + LDS reductions; coalesced row-major access).
//
//   embed_rows     Tensor::embedding of the frozen table (src/tensor.rs:2438-2457), dequant fused
//   rmsnorm_fwd    src/tensor.rs:2500-2517, also emitting the fp16 row-scaled GEMM operand
//   rmsnorm_bwd    src/tensor.rs:2521-2540 (gx only: norm weights are frozen), accumulated into dx
//   rope_apply     src/tensor.rs:2750-2814, fwd rotation and its transpose (bwd), bit-exact
//   swiglu_fwd     silu(g)·u (src/tensor.rs:2082-2087, :458-462), fp16 operand out
//   swiglu_bwd     mul + silu VJPs (src/tensor.rs:466-477, :2088-2098)
//   ce_fwd_bwd     cross_entropy + its VJP (src/tensor.rs:2709-2743), fp16 dlogits out
//   adamw          AdamW::step (src/tensor.rs:2952-2975), bit-exact given the same gradient
#include "fused.hpp"

namespace hos {

namespace {

constexpr int RB = 256;  // threads per row workgroup

__device__ __forceinline__ float warp_sum(float v) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}
__device__ __forceinline__ float warp_max(float v) {
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}
// Block-wide reductions for RB = 256 threads (4 waves). `red` holds 8 floats.
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = warp_sum(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  return red[0] + red[1] + red[2] + red[3];
}
__device__ __forceinline__ float block_max(float v, float* red) {
  v = warp_max(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// fp16 operand element (+ its rounding residual when the operand keeps one).
__device__ __forceinline__ void put_h16(float v, _Float16* hi, _Float16* lo, long long i) {
  _Float16 h = (_Float16)v;
  hi[i] = h;
  if (lo) lo[i] = (_Float16)(v - (float)h);
}

// Four consecutive elements of the fp16 operand at once.
typedef _Float16 h16x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void put_h16x4(float4 v, _Float16* hi, _Float16* lo, long long i) {
  h16x4 h{(_Float16)v.x, (_Float16)v.y, (_Float16)v.z, (_Float16)v.w};
  *reinterpret_cast<h16x4*>(hi + i) = h;
  if (lo) {
    h16x4 l{(_Float16)(v.x - (float)h.x), (_Float16)(v.y - (float)h.y), (_Float16)(v.z - (float)h.z),
            (_Float16)(v.w - (float)h.w)};
    *reinterpret_cast<h16x4*>(lo + i) = l;
  }
}
__device__ __forceinline__ float4 scale4(float4 v, float s) { return make_float4(v.x * s, v.y * s, v.z * s, v.w * s); }
__device__ __forceinline__ float amax4(float a, float4 v) {
  return fmaxf(fmaxf(a, fmaxf(fabsf(v.x), fabsf(v.y))), fmaxf(fabsf(v.z), fabsf(v.w)));
}

// Power-of-two scale that maps a row max-abs into [2^14, 2^15) (exact in fp16 and f32).
__device__ __forceinline__ int row_exp(float amax) {
  if (!(amax > 0.0f) || amax >= 3.0e38f) return 0;
  int ex;
  frexpf(amax, &ex);
  int e = 15 - ex;
  return e > 100 ? 100 : (e < -100 ? -100 : e);
}

__global__ void embed_kernel(QWeightView table, const int32_t* __restrict__ ids, float* __restrict__ x, int M,
                             int d) {
  long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long long)M * d) return;
  int m = (int)(i / d), c = (int)(i % d);
  x[i] = deq_one(table, ids[m], c);
}

__global__ void __launch_bounds__(RB) rmsnorm_fwd_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                          float eps, int d, float* __restrict__ xn,
                                                          _Float16* __restrict__ xh, _Float16* __restrict__ xl,
                                                          float* __restrict__ rinv, float* __restrict__ inv_out) {
  __shared__ float red[8];
  const int row = blockIdx.x;
  const float* xr = x + (long long)row * d;
  float ss = 0.0f;
  for (int c = threadIdx.x; c < d; c += RB) ss += xr[c] * xr[c];
  ss = block_sum(ss, red) / (float)d;
  float inv = 1.0f / sqrtf(ss + eps);
  float amax = 0.0f;
  for (int c = threadIdx.x; c < d; c += RB) {
    float y = xr[c] * inv * w[c];
    amax = fmaxf(amax, fabsf(y));
    if (xn) xn[(long long)row * d + c] = y;
  }
  amax = block_max(amax, red);
  int e = row_exp(amax);
  float sc = ldexpf(1.0f, e);
  for (int c = threadIdx.x; c < d; c += RB) put_h16(xr[c] * inv * w[c] * sc, xh, xl, (long long)row * d + c);
  if (threadIdx.x == 0) {
    rinv[row] = ldexpf(1.0f, -e);
    inv_out[row] = inv;
  }
}

// dx += g·w·inv − inv³·x/d·Σ(g·w·x)
// (hd != null: also the fp16 GEMM operand of the updated dx row, as to_h16 makes it)
__global__ void __launch_bounds__(RB) rmsnorm_bwd_kernel(const float* __restrict__ g, const float* __restrict__ x,
                                                          const float* __restrict__ inv_in,
                                                          const float* __restrict__ w, int d, float* __restrict__ dx,
                                                          _Float16* __restrict__ hd, _Float16* __restrict__ hl,
                                                          float* __restrict__ hr) {
  __shared__ float red[8];
  const int row = blockIdx.x;
  const float* gr = g + (long long)row * d;
  const float* xr = x + (long long)row * d;
  float s = 0.0f;
  for (int c = threadIdx.x; c < d; c += RB) s += gr[c] * w[c] * xr[c];
  s = block_sum(s, red);
  float inv = inv_in[row];
  float k = inv * inv * inv / (float)d * s;
  float* dr = dx + (long long)row * d;
  for (int c = threadIdx.x; c < d; c += RB) dr[c] += gr[c] * w[c] * inv - xr[c] * k;
  if (hd) block_row_h16(dr, d, hd + (long long)row * d, hl ? hl + (long long)row * d : nullptr, hr + row);
}

// RoPE on [M, ld] rows, heads at column col0 + h·hd. tab: (sin, cos) per (position, i), built on the host
// with the same powf/sinf/cosf calls as the reference. inverse: apply Rᵀ (the backward).
__global__ void rope_kernel(float* __restrict__ buf, long long ld, int col0, int n_heads, int hd, int T,
                            const float2* __restrict__ tab, int neox, int inverse, int M) {
#pragma clang fp contract(off)
  const int half = hd >> 1;
  long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  long long total = (long long)M * n_heads * half;
  if (i >= total) return;
  int p = (int)(i % half);
  long long t2 = i / half;
  int h = (int)(t2 % n_heads);
  int m = (int)(t2 / n_heads);
  float2 sc = tab[(m % T) * half + p];
  float s = sc.x, c = sc.y;
  float* base = buf + (long long)m * ld + col0 + h * hd;
  int ia = neox ? p : 2 * p, ib = neox ? p + half : 2 * p + 1;
  float a = base[ia], b = base[ib];
  // plain operators under this function's contract(off): each product and sum rounds separately, as in
  // the reference (intrinsics inlined from headers would keep the headers' contraction setting)
  if (!inverse) {
    base[ia] = a * c - b * s;
    base[ib] = a * s + b * c;
  } else {
    base[ia] = a * c + b * s;
    base[ib] = -a * s + b * c;
  }
}

// RoPE over the first n_heads heads of each row of [M, ld] (col0 = 0) fused with the fp16 operand of the whole
// row's first W columns: one workgroup per row rotates in place (the same arithmetic as rope_kernel), then
// writes hi/lo/1-over-scale exactly as the f32 -> fp16 conversion of the rotated row would.
__global__ void __launch_bounds__(256) rope_h16_kernel(float* __restrict__ buf, long long ld, int n_heads, int hd,
                                                        int T, const float2* __restrict__ tab, int neox, int inverse,
                                                        int W, _Float16* __restrict__ oh, _Float16* __restrict__ ol,
                                                        float* __restrict__ orinv) {
#pragma clang fp contract(off)
  __shared__ float red[8];
  const int m = blockIdx.x, half = hd >> 1, nrot = n_heads * half;
  float* row = buf + (long long)m * ld;
  float amax = 0.0f;
  for (int i = threadIdx.x; i < nrot; i += RB) {
    const int h = i / half, p = i % half;
    const float2 sc2 = tab[(m % T) * half + p];
    const float sn = sc2.x, cs = sc2.y;
    float* base = row + h * hd;
    const int ia = neox ? p : 2 * p, ib = neox ? p + half : 2 * p + 1;
    const float a = base[ia], b = base[ib];
    float ra, rb;
    if (!inverse) {
      ra = a * cs - b * sn;
      rb = a * sn + b * cs;
    } else {
      ra = a * cs + b * sn;
      rb = -a * sn + b * cs;
    }
    base[ia] = ra;
    base[ib] = rb;
    amax = fmaxf(amax, fmaxf(fabsf(ra), fabsf(rb)));
  }
  for (int c = n_heads * hd + threadIdx.x; c < W; c += RB) amax = fmaxf(amax, fabsf(row[c]));
  amax = block_max(amax, red);  // its barriers also make the rotated row visible to the whole workgroup
  const int e = row_exp(amax);
  const float sc = ldexpf(1.0f, e);
  for (int c = threadIdx.x; c < W; c += RB) put_h16(row[c] * sc, oh, ol, (long long)m * W + c);
  if (threadIdx.x == 0) orinv[m] = ldexpf(1.0f, -e);
}

// The row pass after the training step's attention backward, per row m of dqkv [M, ld] (q heads at 0, k heads at
// kcol = nh·hd right after them, v heads at vcol): the k and v columns formed from the per-query-head partials
// part[(m·nh + head)·2·hd + (0 | hd) + i] by summing each GQA group in head order (as attn_group_sum; group == 1:
// dqkv already holds them), the q and k heads rotated back (inverse RoPE with rope_kernel's arithmetic), the row
// stored back in f32 and written as the fp16 operand of its first W columns (the f32 -> fp16 row conversion).
// One workgroup per row, 16-byte accesses (every head dim and W a multiple of 4); the formed row is staged in LDS for
// the rotation's partner reads; W <= 4·RB·ROWS_NV.
constexpr int ROWS_NV = 4;
static_assert(4 * RB * ROWS_NV == kAttnRowsMax, "row pass capacity");
__global__ void __launch_bounds__(RB) attn_bwd_rows_kernel(float* __restrict__ dqkv, long long ld, int hd, int nh,
                                                           int nkv, int group, int vcol,
                                                           const float* __restrict__ part, int T,
                                                           const float2* __restrict__ tab, int neox, int W,
                                                           _Float16* __restrict__ oh, _Float16* __restrict__ ol,
                                                           float* __restrict__ orinv) {
#pragma clang fp contract(off)
  extern __shared__ float rowbuf[];
  __shared__ float red[8];
  const int m = blockIdx.x, half = hd >> 1, kcol = nh * hd, nrotc = (nh + nkv) * hd, W4 = W >> 2;
  float* row = dqkv + (long long)m * ld;
  for (int c4 = threadIdx.x; c4 < W4; c4 += RB) {
    const int c = 4 * c4;
    float4 v;
    if (group > 1 && c >= kcol && c < vcol + nkv * hd && (c < kcol + nkv * hd || c >= vcol)) {
      const bool isv = c >= vcol;
      const int cc = isv ? c - vcol : c - kcol, g = cc / hd, i = cc % hd;
      const float* pp = part + ((long long)m * nh + (long long)g * group) * 2 * hd + (isv ? hd : 0) + i;
      v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      for (int hh = 0; hh < group; hh++) {
        const float4 t = *reinterpret_cast<const float4*>(pp + (long long)hh * 2 * hd);
        v.x += t.x;
        v.y += t.y;
        v.z += t.z;
        v.w += t.w;
      }
    } else {
      v = reinterpret_cast<const float4*>(row)[c4];
    }
    reinterpret_cast<float4*>(rowbuf)[c4] = v;
  }
  __syncthreads();
  const float2* tr = tab + (long long)(m % T) * half;
  float4 rv[ROWS_NV];
  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < ROWS_NV; j++) {
    const int c4 = threadIdx.x + RB * j;
    if (c4 >= W4) break;
    float r[4];
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const int c = 4 * c4 + e;
      r[e] = rowbuf[c];
      if (c < nrotc) {
        const int hb = c - c % hd, i = c % hd;
        int p, ia, ib;
        if (neox) {
          p = i < half ? i : i - half;
          ia = p;
          ib = p + half;
        } else {
          p = i >> 1;
          ia = 2 * p;
          ib = 2 * p + 1;
        }
        const float a = rowbuf[hb + ia], b = rowbuf[hb + ib];
        const float2 sc2 = tr[p];
        const float sn = sc2.x, cs = sc2.y;
        r[e] = (i == ia) ? a * cs + b * sn : -a * sn + b * cs;
      }
      amax = fmaxf(amax, fabsf(r[e]));
    }
    rv[j] = make_float4(r[0], r[1], r[2], r[3]);
    reinterpret_cast<float4*>(row)[c4] = rv[j];
  }
  amax = block_max(amax, red);
  const int ex = row_exp(amax);
  const float sc = ldexpf(1.0f, ex);
#pragma unroll
  for (int j = 0; j < ROWS_NV; j++) {
    const int c4 = threadIdx.x + RB * j;
    if (c4 >= W4) break;
    put_h16x4(make_float4(rv[j].x * sc, rv[j].y * sc, rv[j].z * sc, rv[j].w * sc), oh, ol, (long long)m * W + 4 * c4);
  }
  if (threadIdx.x == 0) orinv[m] = ldexpf(1.0f, -ex);
}

__device__ __forceinline__ float silu_f(float x) { return x / (1.0f + expf(-x)); }

// gu rows = [gate (F) | up (F)] -> h = silu(gate)·up: f32 (optional) + fp16 operand.
__global__ void __launch_bounds__(RB) swiglu_fwd_kernel(const float* __restrict__ gu, int F, float* __restrict__ h,
                                                         _Float16* __restrict__ hh, _Float16* __restrict__ hl,
                                                         float* __restrict__ rinv) {
  __shared__ float red[8];
  const int row = blockIdx.x;
  const float* g = gu + (long long)row * 2 * F;
  const float* u = g + F;
  float amax = 0.0f;
  for (int c = threadIdx.x; c < F; c += RB) {
    float v = silu_f(g[c]) * u[c];
    amax = fmaxf(amax, fabsf(v));
    if (h) h[(long long)row * F + c] = v;
  }
  amax = block_max(amax, red);
  int e = row_exp(amax);
  float sc = ldexpf(1.0f, e);
  for (int c = threadIdx.x; c < F; c += RB) put_h16(silu_f(g[c]) * u[c] * sc, hh, hl, (long long)row * F + c);
  if (threadIdx.x == 0) rinv[row] = ldexpf(1.0f, -e);
}

// dh -> d[gate | up] (f32 optional, fp16 operand with row scale)
__global__ void __launch_bounds__(RB) swiglu_bwd_kernel(const float* __restrict__ gu, const float* __restrict__ dh,
                                                         int F, float* __restrict__ dgu, _Float16* __restrict__ dgh,
                                                         _Float16* __restrict__ dgl, float* __restrict__ rinv) {
  __shared__ float red[8];
  const int row = blockIdx.x;
  const float* g = gu + (long long)row * 2 * F;
  const float* u = g + F;
  const float* d = dh + (long long)row * F;
  float amax = 0.0f;
  for (int c = threadIdx.x; c < F; c += RB) {
    float x = g[c];
    float s = 1.0f / (1.0f + expf(-x));
    float dg = d[c] * u[c] * (s + x * s * (1.0f - s));
    float du = d[c] * (x / (1.0f + expf(-x)));
    amax = fmaxf(amax, fmaxf(fabsf(dg), fabsf(du)));
    if (dgu) {
      dgu[(long long)row * 2 * F + c] = dg;
      dgu[(long long)row * 2 * F + F + c] = du;
    }
  }
  amax = block_max(amax, red);
  int e = row_exp(amax);
  float sc = ldexpf(1.0f, e);
  for (int c = threadIdx.x; c < F; c += RB) {
    float x = g[c];
    float s = 1.0f / (1.0f + expf(-x));
    float dg = d[c] * u[c] * (s + x * s * (1.0f - s));
    float du = d[c] * (x / (1.0f + expf(-x)));
    put_h16(dg * sc, dgh, dgl, (long long)row * 2 * F + c);
    put_h16(du * sc, dgh, dgl, (long long)row * 2 * F + F + c);
  }
  if (threadIdx.x == 0) rinv[row] = ldexpf(1.0f, -e);
}

// Register-resident variants of the two kernels above for F % 4 == 0, F <= 4·RB·NV: each thread loads its
// float4 columns once (i = tid + RB·j), so the row is read from HBM once and the fp16 pass works from
// registers; the same per-element arithmetic and the same row max, hence the same outputs.
constexpr int SWIGLU_NV = 8;

__global__ void __launch_bounds__(RB) swiglu_fwd_reg_kernel(const float* __restrict__ gu, int F,
                                                             float* __restrict__ h, _Float16* __restrict__ hh,
                                                             _Float16* __restrict__ hl, float* __restrict__ rinv) {
  __shared__ float red[8];
  const int row = blockIdx.x, F4 = F >> 2;
  const float4* g = reinterpret_cast<const float4*>(gu + (long long)row * 2 * F);
  const float4* u = g + F4;
  float4 gv[SWIGLU_NV], uv[SWIGLU_NV];
#pragma unroll
  for (int j = 0; j < SWIGLU_NV; j++) {
    const int i = threadIdx.x + RB * j;
    if (i < F4) {
      gv[j] = g[i];
      uv[j] = u[i];
    }
  }
  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < SWIGLU_NV; j++) {
    const int i = threadIdx.x + RB * j;
    if (i < F4) {
      const float4 v = make_float4(silu_f(gv[j].x) * uv[j].x, silu_f(gv[j].y) * uv[j].y, silu_f(gv[j].z) * uv[j].z,
                                   silu_f(gv[j].w) * uv[j].w);
      gv[j] = v;
      amax = amax4(amax, v);
      if (h) reinterpret_cast<float4*>(h + (long long)row * F)[i] = v;
    }
  }
  amax = block_max(amax, red);
  const int e = row_exp(amax);
  const float sc = ldexpf(1.0f, e);
#pragma unroll
  for (int j = 0; j < SWIGLU_NV; j++) {
    const int i = threadIdx.x + RB * j;
    if (i < F4) put_h16x4(scale4(gv[j], sc), hh, hl, (long long)row * F + 4 * i);
  }
  if (threadIdx.x == 0) rinv[row] = ldexpf(1.0f, -e);
}

__device__ __forceinline__ void swiglu_vjp(float x, float uu, float dd, float& dg, float& du) {
  float s = 1.0f / (1.0f + expf(-x));
  dg = dd * uu * (s + x * s * (1.0f - s));
  du = dd * (x / (1.0f + expf(-x)));
}

__global__ void __launch_bounds__(RB) swiglu_bwd_reg_kernel(const float* __restrict__ gu,
                                                             const float* __restrict__ dh, int F,
                                                             float* __restrict__ dgu, _Float16* __restrict__ dgh,
                                                             _Float16* __restrict__ dgl, float* __restrict__ rinv) {
  __shared__ float red[8];
  const int row = blockIdx.x, F4 = F >> 2;
  const float4* g = reinterpret_cast<const float4*>(gu + (long long)row * 2 * F);
  const float4* u = g + F4;
  const float4* d = reinterpret_cast<const float4*>(dh + (long long)row * F);
  float4 gv[SWIGLU_NV], uv[SWIGLU_NV];
  {
    float4 dv[SWIGLU_NV];
#pragma unroll
    for (int j = 0; j < SWIGLU_NV; j++) {
      const int i = threadIdx.x + RB * j;
      if (i < F4) {
        gv[j] = g[i];
        uv[j] = u[i];
        dv[j] = d[i];
      }
    }
#pragma unroll
    for (int j = 0; j < SWIGLU_NV; j++) {
      const int i = threadIdx.x + RB * j;
      if (i < F4) {
        float4 a, b;
        swiglu_vjp(gv[j].x, uv[j].x, dv[j].x, a.x, b.x);
        swiglu_vjp(gv[j].y, uv[j].y, dv[j].y, a.y, b.y);
        swiglu_vjp(gv[j].z, uv[j].z, dv[j].z, a.z, b.z);
        swiglu_vjp(gv[j].w, uv[j].w, dv[j].w, a.w, b.w);
        gv[j] = a;  // d gate
        uv[j] = b;  // d up
      }
    }
  }
  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < SWIGLU_NV; j++) {
    const int i = threadIdx.x + RB * j;
    if (i < F4) {
      amax = amax4(amax4(amax, gv[j]), uv[j]);
      if (dgu) {
        float4* o = reinterpret_cast<float4*>(dgu + (long long)row * 2 * F);
        o[i] = gv[j];
        o[F4 + i] = uv[j];
      }
    }
  }
  amax = block_max(amax, red);
  const int e = row_exp(amax);
  const float sc = ldexpf(1.0f, e);
#pragma unroll
  for (int j = 0; j < SWIGLU_NV; j++) {
    const int i = threadIdx.x + RB * j;
    if (i < F4) {
      put_h16x4(scale4(gv[j], sc), dgh, dgl, (long long)row * 2 * F + 4 * i);
      put_h16x4(scale4(uv[j], sc), dgh, dgl, (long long)row * 2 * F + F + 4 * i);
    }
  }
  if (threadIdx.x == 0) rinv[row] = ldexpf(1.0f, -e);
}

// Four consecutive elements (offset off = m·n + c) of a row formed from a split qGEMM's deferred partials: summed in
// split order, times the row's scale, plus the residual — splitk_reduce4's arithmetic for the same output.
__device__ __forceinline__ float4 split_row4(const SplitSrc& s, long long off, float ri) {
  float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int z = 0; z < s.splits; z++) {
    const float4 p = *reinterpret_cast<const float4*>(s.ws + z * s.mn + off);
    v.x += p.x;
    v.y += p.y;
    v.z += p.z;
    v.w += p.w;
  }
  float4 x = make_float4(v.x * ri, v.y * ri, v.z * ri, v.w * ri);
  if (s.resid) {
    const float4 a = *reinterpret_cast<const float4*>(s.resid + off);
    x = make_float4(a.x + x.x, a.y + x.y, a.z + x.z, a.w + x.w);
  }
  return x;
}

// Register-resident RMSNorm forward / backward for d % 4 == 0, d <= 4·RB·NORM_NV (same per-element arithmetic as
// the kernels above; the row sums are taken over each thread's float4 columns, then across the block).
constexpr int NORM_NV = 4;

// src.splits > 0: the input row is formed from a split GEMM's deferred partials (split_row4) and written to x.
__global__ void __launch_bounds__(RB) rmsnorm_fwd_reg_kernel(float* __restrict__ x, const float* __restrict__ w,
                                                              float eps, int d, float* __restrict__ xn,
                                                              _Float16* __restrict__ xh, _Float16* __restrict__ xl,
                                                              float* __restrict__ rinv,
                                                              float* __restrict__ inv_out, SplitSrc src) {
  __shared__ float red[8];
  const int row = blockIdx.x, d4 = d >> 2;
  float4* xr = reinterpret_cast<float4*>(x + (long long)row * d);
  const float sri = src.splits ? src.rinv[row] : 0.0f;
  float4 xv[NORM_NV];
  float ss = 0.0f;
#pragma unroll
  for (int j = 0; j < NORM_NV; j++) {
    const int i = threadIdx.x + RB * j;
    if (i < d4) {
      if (src.splits) {
        xv[j] = split_row4(src, (long long)row * d + 4 * i, sri);
        xr[i] = xv[j];
      } else {
        xv[j] = xr[i];
      }
      ss += xv[j].x * xv[j].x;
      ss += xv[j].y * xv[j].y;
      ss += xv[j].z * xv[j].z;
      ss += xv[j].w * xv[j].w;
    }
  }
  ss = block_sum(ss, red) / (float)d;
  const float inv = 1.0f / sqrtf(ss + eps);
  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < NORM_NV; j++) {
    const int i = threadIdx.x + RB * j;
    if (i < d4) {
      const float4 wv = reinterpret_cast<const float4*>(w)[i];
      const float4 y = make_float4(xv[j].x * inv * wv.x, xv[j].y * inv * wv.y, xv[j].z * inv * wv.z,
                                   xv[j].w * inv * wv.w);
      xv[j] = y;
      amax = amax4(amax, y);
      if (xn) reinterpret_cast<float4*>(xn + (long long)row * d)[i] = y;
    }
  }
  amax = block_max(amax, red);
  const int e = row_exp(amax);
  const float sc = ldexpf(1.0f, e);
#pragma unroll
  for (int j = 0; j < NORM_NV; j++) {
    const int i = threadIdx.x + RB * j;
    if (i < d4) put_h16x4(scale4(xv[j], sc), xh, xl, (long long)row * d + 4 * i);
  }
  if (threadIdx.x == 0) {
    rinv[row] = ldexpf(1.0f, -e);
    inv_out[row] = inv;
  }
}

// src.splits > 0: the incoming gradient row g is formed from a split GEMM's deferred partials (split_row4).
__global__ void __launch_bounds__(RB) rmsnorm_bwd_reg_kernel(const float* __restrict__ g, const float* __restrict__ x,
                                                              const float* __restrict__ inv_in,
                                                              const float* __restrict__ w, int d,
                                                              float* __restrict__ dx, _Float16* __restrict__ hd,
                                                              _Float16* __restrict__ hl, float* __restrict__ hr,
                                                              SplitSrc src, const float* __restrict__ dxin) {
  __shared__ float red[8];
  const int row = blockIdx.x, d4 = d >> 2;
  const float4* gr = reinterpret_cast<const float4*>(g + (long long)row * d);
  const float sri = src.splits ? src.rinv[row] : 0.0f;
  const float4* xr = reinterpret_cast<const float4*>(x + (long long)row * d);
  float4* dr = reinterpret_cast<float4*>(dx + (long long)row * d);
  float4 gw[NORM_NV], xv[NORM_NV];
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < NORM_NV; j++) {
    const int i = threadIdx.x + RB * j;
    if (i < d4) {
      const float4 wv = reinterpret_cast<const float4*>(w)[i];
      const float4 gv = src.splits ? split_row4(src, (long long)row * d + 4 * i, sri) : gr[i];
      xv[j] = xr[i];
      gw[j] = make_float4(gv.x * wv.x, gv.y * wv.y, gv.z * wv.z, gv.w * wv.w);
      s += gw[j].x * xv[j].x;
      s += gw[j].y * xv[j].y;
      s += gw[j].z * xv[j].z;
      s += gw[j].w * xv[j].w;
    }
  }
  s = block_sum(s, red);
  const float inv = inv_in[row];
  const float k = inv * inv * inv / (float)d * s;
  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < NORM_NV; j++) {
    const int i = threadIdx.x + RB * j;
    if (i < d4) {
      float4 o = dxin ? reinterpret_cast<const float4*>(dxin + (long long)row * d)[i] : dr[i];
      o.x += gw[j].x * inv - xv[j].x * k;
      o.y += gw[j].y * inv - xv[j].y * k;
      o.z += gw[j].z * inv - xv[j].z * k;
      o.w += gw[j].w * inv - xv[j].w * k;
      dr[i] = o;
      xv[j] = o;
      amax = amax4(amax, o);
    }
  }
  if (!hd) return;
  amax = block_max(amax, red);
  const int e = row_exp(amax);
  const float sc = ldexpf(1.0f, e);
#pragma unroll
  for (int j = 0; j < NORM_NV; j++) {
    const int i = threadIdx.x + RB * j;
    if (i < d4) put_h16x4(scale4(xv[j], sc), hd, hl, (long long)row * d + 4 * i);
  }
  if (threadIdx.x == 0) hr[row] = ldexpf(1.0f, -e);
}

// Softmax cross-entropy of one row + its gradient (p − onehot)·gscale as an fp16 operand.
// Online softmax state: (m, s) with s = Σ exp(x − m); merging two states keeps the larger max.
__device__ __forceinline__ void sm_add(float& m, float& s, float x) {
  if (x > m) {
    s = s * expf(m - x) + 1.0f;
    m = x;
  } else {
    s += expf(x - m);
  }
}
__device__ __forceinline__ void sm_merge(float& m, float& s, float m2, float s2, bool hw = false) {
  // hw: the states came from the head GEMM's epilogue, which exponentiates with exp_rs; rescale with it too
  if (m2 > m) {
    s = s * (hw ? exp_rs(m - m2) : expf(m - m2)) + s2;
    m = m2;
  } else if (m2 > -INFINITY) {
    s += s2 * (hw ? exp_rs(m2 - m) : expf(m2 - m));
  }
}

// Softmax cross-entropy forward + backward of one row (src/tensor.rs:2709-2743): one read of the logits
// for the row max and exp-sum together (online softmax) — or, given rstat, the (max, exp-sum) of each 64-column
// chunk that the head GEMM's epilogue computed, merged in chunk order — and one more to write the gradient
// (p − onehot)·gscale as the fp16 row-scaled operand of the head's dX GEMM.
__global__ void __launch_bounds__(RB) ce_kernel(const float* __restrict__ logits, int V,
                                                 const int32_t* __restrict__ targets, float gscale,
                                                 float* __restrict__ row_loss, _Float16* __restrict__ dl,
                                                 _Float16* __restrict__ dll, float* __restrict__ rinv,
                                                 float* __restrict__ dl32, const float2* __restrict__ rstat, int nch) {
  __shared__ float rm[RB / 64], rs[RB / 64];
  const int row = blockIdx.x;
  const float* lr = logits + (long long)row * V;
  float m = -INFINITY, sum = 0.0f;
  const bool vec = (V & 3) == 0;
  if (rstat) {
    const float2* rr = rstat + (long long)row * nch;
    for (int c = threadIdx.x; c < nch; c += RB) {
      const float2 x = rr[c];
      sm_merge(m, sum, x.x, x.y, true);
    }
  } else if (vec) {
    const float4* l4 = reinterpret_cast<const float4*>(lr);
    auto add4 = [&](float4 x) {
      sm_add(m, sum, x.x);
      sm_add(m, sum, x.y);
      sm_add(m, sum, x.z);
      sm_add(m, sum, x.w);
    };
    // two loads in flight, elements folded in the thread's column order
    int c = threadIdx.x;
    for (; c + RB < V / 4; c += 2 * RB) {
      const float4 x0 = l4[c], x1 = l4[c + RB];
      add4(x0);
      add4(x1);
    }
    if (c < V / 4) add4(l4[c]);
  } else {
    for (int c = threadIdx.x; c < V; c += RB) sm_add(m, sum, lr[c]);
  }
  // With statistics from the head GEMM's epilogue, every exponential below (merges and numerators) uses the
  // epilogue's exp_rs, so the denominator and the numerators come from one function; expf when they were computed
  // here (the op-level entry).
  const bool hw = rstat != nullptr;
  for (int o = 32; o > 0; o >>= 1) sm_merge(m, sum, __shfl_xor(m, o), __shfl_xor(sum, o), hw);
  if ((threadIdx.x & 63) == 0) {
    rm[threadIdx.x >> 6] = m;
    rs[threadIdx.x >> 6] = sum;
  }
  __syncthreads();
  m = rm[0];
  sum = rs[0];
#pragma unroll
  for (int w = 1; w < RB / 64; w++) sm_merge(m, sum, rm[w], rs[w], hw);
  const int t = targets[row];
  auto ex = [hw](float d) { return hw ? exp_rs(d) : expf(d); };
  const float pt = ex(lr[t] - m) / sum;
  if (threadIdx.x == 0) row_loss[row] = -logf(fmaxf(pt, 1e-12f));
  // max |p − onehot| = max(1/sum, 1 − p_t) (the row max has p = 1/sum)
  const float amax = fmaxf(1.0f / sum, 1.0f - pt) * fabsf(gscale);
  const int e = row_exp(amax);
  const float sc = ldexpf(1.0f, e), inv = 1.0f / sum;
  if (dl32) {  // plain f32 gradient (the op-level entry point)
    for (int c = threadIdx.x; c < V; c += RB) {
      float p = ex(lr[c] - m) * inv;
      if (c == t) p -= 1.0f;
      dl32[(long long)row * V + c] = p * gscale;
    }
    return;
  }
  if (vec && ((uintptr_t)dl & 7) == 0 && ((uintptr_t)dll & 7) == 0) {
    // float4 loads (two in flight) and 8-byte fp16 stores; the same per-element arithmetic as below
    const float4* l4 = reinterpret_cast<const float4*>(lr);
    const int V4 = V >> 2;
    auto grad4 = [&](float4 x, int c4) {
      const int c = 4 * c4;
      float4 p = make_float4(ex(x.x - m) * inv, ex(x.y - m) * inv, ex(x.z - m) * inv, ex(x.w - m) * inv);
      if (c == t) p.x -= 1.0f;
      if (c + 1 == t) p.y -= 1.0f;
      if (c + 2 == t) p.z -= 1.0f;
      if (c + 3 == t) p.w -= 1.0f;
      put_h16x4(make_float4(p.x * gscale * sc, p.y * gscale * sc, p.z * gscale * sc, p.w * gscale * sc), dl, dll,
                (long long)row * V + c);
    };
    int c4 = threadIdx.x;
    for (; c4 + RB < V4; c4 += 2 * RB) {
      const float4 x0 = l4[c4], x1 = l4[c4 + RB];
      grad4(x0, c4);
      grad4(x1, c4 + RB);
    }
    if (c4 < V4) grad4(l4[c4], c4);
  } else {
    for (int c = threadIdx.x; c < V; c += RB) {
      float p = ex(lr[c] - m) * inv;
      if (c == t) p -= 1.0f;
      put_h16(p * gscale * sc, dl, dll, (long long)row * V + c);
    }
  }
  if (threadIdx.x == 0) rinv[row] = ldexpf(1.0f, -e);
}

// loss = Σ_b (Σ_t term[b,t] / T) · (1/B), in sequence order (src/main.rs:2588-2596). Each sequence is
// staged in LDS by the whole workgroup and summed in order by one thread.
__global__ void __launch_bounds__(256) loss_reduce_kernel(const float* __restrict__ row_loss, int B, int T,
                                                          float* __restrict__ loss) {
  __shared__ __attribute__((aligned(16))) float buf[2048];
  float mean = 0.0f;
  for (int b = 0; b < B; b++) {
    float s = 0.0f;
    for (int t0 = 0; t0 < T; t0 += 2048) {
      const int n = min(2048, T - t0);
      __syncthreads();
      for (int i = threadIdx.x; i < n; i += 256) buf[i] = row_loss[(long long)b * T + t0 + i];
      __syncthreads();
      if (threadIdx.x == 0) {
        // the same in-order sum; four 16-byte reads in flight ahead of the adds instead of one read per add
        int i = 0;
        for (; i + 16 <= n; i += 16) {
          const float4 a = *(const float4*)(buf + i), c = *(const float4*)(buf + i + 4);
          const float4 d = *(const float4*)(buf + i + 8), e = *(const float4*)(buf + i + 12);
          s += a.x; s += a.y; s += a.z; s += a.w;
          s += c.x; s += c.y; s += c.z; s += c.w;
          s += d.x; s += d.y; s += d.z; s += d.w;
          s += e.x; s += e.y; s += e.z; s += e.w;
        }
        for (; i < n; i++) s += buf[i];
      }
    }
    if (threadIdx.x == 0) mean += (s / (float)T) * (1.0f / (float)B);
  }
  if (threadIdx.x == 0) *loss = mean;
}

__global__ void adamw_kernel(float* __restrict__ p, const float* __restrict__ g, float* __restrict__ m,
                             float* __restrict__ v, long long n, float lr, float b1, float b2, float eps, float wd,
                             float bc1, float bc2, int decay) {
#pragma clang fp contract(off)
  long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  // plain operators under contract(off) (see rope_kernel); correctly rounded division and sqrt
  const float gi = g[i];
  const float mi = b1 * m[i] + (1.0f - b1) * gi;
  const float vi = b2 * v[i] + (1.0f - b2) * gi * gi;
  m[i] = mi;
  v[i] = vi;
  const float mh = div_rn(mi, bc1), vh = div_rn(vi, bc2);
  float u = div_rn(lr * mh, sqrt_rn(vh) + eps);
  if (decay) u = u + lr * wd * p[i];
  p[i] = p[i] - u;
}

// The same update with lr, wd and the step count read from device memory (hyper = {lr, wd, t}), so a
// captured step graph replays with the current values; adam_tick advances t first (one thread).
__global__ void adam_tick_kernel(AdamHyper* h) {
  if (threadIdx.x == 0 && blockIdx.x == 0) h->t += 1;
}
__device__ float powi_dev(float a, int b) {
#pragma clang fp contract(off)
  const bool recip = b < 0;
  float r = 1.0f;
  while (true) {
    if (b & 1) r = r * a;
    b /= 2;
    if (b == 0) break;
    a = a * a;
  }
  return recip ? div_rn(1.0f, r) : r;
}
__global__ void adamw_dev_kernel(float* __restrict__ p, const float* __restrict__ g, float* __restrict__ m,
                                 float* __restrict__ v, long long n, float b1, float b2, float eps,
                                 const AdamHyper* __restrict__ h, int decay) {
#pragma clang fp contract(off)
  long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float lr = h->lr, wd = h->wd;
  const float bc1 = 1.0f - powi_dev(b1, h->t), bc2 = 1.0f - powi_dev(b2, h->t);
  const float gi = g[i];
  const float mi = b1 * m[i] + (1.0f - b1) * gi;
  const float vi = b2 * v[i] + (1.0f - b2) * gi * gi;
  m[i] = mi;
  v[i] = vi;
  const float mh = div_rn(mi, bc1), vh = div_rn(vi, bc2);
  float u = div_rn(lr * mh, sqrt_rn(vh) + eps);
  if (decay) u = u + lr * wd * p[i];
  p[i] = p[i] - u;
}

__global__ void fill_kernel(float* __restrict__ p, long long n, float v) {
  long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

__global__ void copy_rows_kernel(const float* __restrict__ src, long long lds, float* __restrict__ dst,
                                 long long ldd, int cols, long long total) {
  long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  long long r = i / cols;
  int c = (int)(i % cols);
  dst[r * ldd + c] = src[r * lds + c];
}

// splitmix64 finaliser as the counter-based generator; Box–Muller on two 24-bit uniforms in (0, 1)
__device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
__global__ void randn_kernel(float* __restrict__ out, long long n, uint64_t seed, float stddev) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const uint64_t h = mix64(seed ^ mix64((uint64_t)i));
  const float u1 = ((float)(h >> 40) + 0.5f) * (1.0f / 16777216.0f);
  const float u2 = ((float)((h >> 16) & 0xFFFFFF) + 0.5f) * (1.0f / 16777216.0f);
  out[i] = stddev * sqrtf(-2.0f * logf(u1)) * cosf(6.283185307f * u2);
}

}  // namespace

void launch_randn(float* out, size_t n, uint64_t seed, float stddev, hipStream_t st) {
  if (n == 0) return;
  randn_kernel<<<ceil_div((long long)n, 256), 256, 0, st>>>(out, (long long)n, seed, stddev);
  HOS_HIP_CHECK(hipGetLastError());
}

void launch_embed(const QWeight& table, const int32_t* ids, float* x, int M, int d, hipStream_t st) {
  long long n = (long long)M * d;
  embed_kernel<<<ceil_div(n, 256), 256, 0, st>>>(view(table), ids, x, M, d);
  HOS_HIP_CHECK(hipGetLastError());
}
static bool norm_reg_ok(int d, const void* a, const void* b, const void* c, const void* h, const void* l) {
  auto al = [](const void* p, uintptr_t n) { return ((uintptr_t)p % n) == 0; };
  return d % 4 == 0 && d <= 4 * RB * NORM_NV && al(a, 16) && al(b, 16) && al(c, 16) && al(h, 8) && al(l, 8);
}
// The deferred partials of a split GEMM reduced into dst [M, d] (the general path when a row kernel cannot fuse it).
static void reduce_split_src(const SplitSrc& s, float* dst, int M, int d, hipStream_t st) {
  GemmEpi e{};
  e.out = dst;
  e.ldo = d;
  e.resid = s.resid;
  launch_qgemm_split_reduce(s.ws, s.splits, M, d, s.rinv, e, st);
}
static bool split_ok(const SplitSrc& s) {
  return s.splits > 0 && ((uintptr_t)s.ws & 15) == 0 && ((uintptr_t)s.resid & 15) == 0;
}
void launch_rmsnorm_fwd(float* x, const float* w, float eps, int M, int d, float* xn, H16 out, float* inv,
                        hipStream_t st, SplitSrc src) {
  const bool reg = norm_reg_ok(d, x, w, xn, out.data, out.lo);
  if (src.splits > 0 && !(reg && split_ok(src))) {
    reduce_split_src(src, x, M, d, st);
    src = SplitSrc{};
  }
  if (reg)
    rmsnorm_fwd_reg_kernel<<<M, RB, 0, st>>>(x, w, eps, d, xn, out.data, out.lo, out.rinv, inv, src);
  else
    rmsnorm_fwd_kernel<<<M, RB, 0, st>>>(x, w, eps, d, xn, out.data, out.lo, out.rinv, inv);
  HOS_HIP_CHECK(hipGetLastError());
}
void launch_rmsnorm_bwd(float* g, const float* x, const float* inv, const float* w, int M, int d, float* dx,
                        hipStream_t st, H16 out, SplitSrc src, const float* dx_in) {
  auto al = [](const void* p, uintptr_t n) { return ((uintptr_t)p % n) == 0; };
  if (dx_in == dx) dx_in = nullptr;
  const bool reg = norm_reg_ok(d, g, x, w, out.data, out.lo) && al(dx, 16) && al(dx_in, 16);
  if (dx_in && !reg) {  // the general kernel updates in place: start from a copy
    HOS_HIP_CHECK(hipMemcpyAsync(dx, dx_in, (size_t)M * d * sizeof(float), hipMemcpyDeviceToDevice, st));
    dx_in = nullptr;
  }
  if (src.splits > 0 && !(reg && split_ok(src))) {
    reduce_split_src(src, g, M, d, st);
    src = SplitSrc{};
  }
  if (reg)
    rmsnorm_bwd_reg_kernel<<<M, RB, 0, st>>>(g, x, inv, w, d, dx, out.data, out.lo, out.rinv, src, dx_in);
  else
    rmsnorm_bwd_kernel<<<M, RB, 0, st>>>(g, x, inv, w, d, dx, out.data, out.lo, out.rinv);
  HOS_HIP_CHECK(hipGetLastError());
}
void launch_rope(float* buf, long long ld, int col0, int n_heads, int hd, int T, const float2* tab, bool neox,
                 bool inverse, int M, hipStream_t st) {
  long long n = (long long)M * n_heads * (hd / 2);
  rope_kernel<<<ceil_div(n, 256), 256, 0, st>>>(buf, ld, col0, n_heads, hd, T, tab, neox, inverse, M);
  HOS_HIP_CHECK(hipGetLastError());
}
void launch_attn_bwd_rows(float* dqkv, long long ld, int hd, int nh, int nkv, int vcol, const float* part, int T,
                          const float2* tab, bool neox, int M, int W, H16 out, hipStream_t st) {
  HOS_REQUIRE(nkv > 0 && nh % nkv == 0 && W <= ld && W <= kAttnRowsMax && W % 4 == 0 && ld % 4 == 0 && hd % 4 == 0 &&
                  vcol % 4 == 0 && vcol >= (nh + nkv) * hd && vcol + nkv * hd <= W && (nh == nkv || part != nullptr) &&
                  ((uintptr_t)dqkv & 15) == 0 && ((uintptr_t)part & 15) == 0 && ((uintptr_t)out.data & 7) == 0 &&
                  ((uintptr_t)out.lo & 7) == 0,
              HOS_E_INVALID, "attention rows pass: bad layout");
  if (M <= 0) return;
  attn_bwd_rows_kernel<<<M, RB, (size_t)W * sizeof(float), st>>>(dqkv, ld, hd, nh, nkv, nh / nkv, vcol, part, T, tab,
                                                                  neox, W, out.data, out.lo, out.rinv);
  HOS_HIP_CHECK(hipGetLastError());
}
void launch_rope_h16(float* buf, long long ld, int n_heads, int hd, int T, const float2* tab, bool neox, bool inverse,
                     int M, int W, H16 out, hipStream_t st) {
  HOS_REQUIRE(n_heads * hd <= W && W <= ld, HOS_E_INVALID, "rope_h16: rotated heads must lie within the row");
  if (M <= 0) return;
  rope_h16_kernel<<<M, RB, 0, st>>>(buf, ld, n_heads, hd, T, tab, neox, inverse, W, out.data, out.lo, out.rinv);
  HOS_HIP_CHECK(hipGetLastError());
}
// The register-resident kernels need F % 4 == 0, F <= 4·RB·SWIGLU_NV and 16-byte (f32) / 8-byte (fp16) aligned
// rows; other shapes take the two-pass kernels.
static bool swiglu_reg_ok(int F, const void* a, const void* b, const void* c, const void* d, const void* e) {
  auto al = [](const void* p, uintptr_t n) { return ((uintptr_t)p % n) == 0; };
  return F % 4 == 0 && F <= 4 * RB * SWIGLU_NV && al(a, 16) && al(b, 16) && al(c, 16) && al(d, 8) && al(e, 8);
}
void launch_swiglu_fwd(const float* gu, int M, int F, float* h, H16 out, hipStream_t st) {
  if (swiglu_reg_ok(F, gu, h, nullptr, out.data, out.lo))
    swiglu_fwd_reg_kernel<<<M, RB, 0, st>>>(gu, F, h, out.data, out.lo, out.rinv);
  else
    swiglu_fwd_kernel<<<M, RB, 0, st>>>(gu, F, h, out.data, out.lo, out.rinv);
  HOS_HIP_CHECK(hipGetLastError());
}
void launch_swiglu_bwd(const float* gu, const float* dh, int M, int F, float* dgu, H16 out, hipStream_t st) {
  if (swiglu_reg_ok(F, gu, dh, dgu, out.data, out.lo))
    swiglu_bwd_reg_kernel<<<M, RB, 0, st>>>(gu, dh, F, dgu, out.data, out.lo, out.rinv);
  else
    swiglu_bwd_kernel<<<M, RB, 0, st>>>(gu, dh, F, dgu, out.data, out.lo, out.rinv);
  HOS_HIP_CHECK(hipGetLastError());
}
void launch_ce(const float* logits, int M, int V, const int32_t* targets, float gscale, float* row_loss, H16 dl,
               hipStream_t st, float* dl32, const float2* rstat) {
  ce_kernel<<<M, RB, 0, st>>>(logits, V, targets, gscale, row_loss, dl.data, dl.lo, dl.rinv, dl32, rstat,
                              (V + 63) / 64);
  HOS_HIP_CHECK(hipGetLastError());
}
void launch_loss_reduce(const float* row_loss, int B, int T, float* loss, hipStream_t st) {
  loss_reduce_kernel<<<1, 256, 0, st>>>(row_loss, B, T, loss);
  HOS_HIP_CHECK(hipGetLastError());
}
void launch_adamw(float* p, const float* g, float* m, float* v, long long n, float lr, float b1, float b2, float eps,
                  float wd, float bc1, float bc2, bool decay, hipStream_t st) {
  adamw_kernel<<<ceil_div(n, 256), 256, 0, st>>>(p, g, m, v, n, lr, b1, b2, eps, wd, bc1, bc2, decay);
  HOS_HIP_CHECK(hipGetLastError());
}
void launch_adam_tick(AdamHyper* h, hipStream_t st) {
  adam_tick_kernel<<<1, 64, 0, st>>>(h);
  HOS_HIP_CHECK(hipGetLastError());
}
void launch_adamw_dev(float* p, const float* g, float* m, float* v, long long n, float b1, float b2, float eps,
                      const AdamHyper* h, bool decay, hipStream_t st) {
  adamw_dev_kernel<<<ceil_div(n, 256), 256, 0, st>>>(p, g, m, v, n, b1, b2, eps, h, decay);
  HOS_HIP_CHECK(hipGetLastError());
}
void launch_fill(float* p, long long n, float v, hipStream_t st) {
  if (n <= 0) return;
  fill_kernel<<<ceil_div(n, 256), 256, 0, st>>>(p, n, v);
  HOS_HIP_CHECK(hipGetLastError());
}
void launch_copy_rows(const float* src, long long lds, float* dst, long long ldd, int rows, int cols,
                      hipStream_t st) {
  long long n = (long long)rows * cols;
  if (n <= 0) return;
  copy_rows_kernel<<<ceil_div(n, 256), 256, 0, st>>>(src, lds, dst, ldd, cols, n);
  HOS_HIP_CHECK(hipGetLastError());
}

}  // namespace hos
