// GGUF block codec on gfx950: repack of uploaded GGUF tensors into the device weight
// layout, bit-exact dequantization (the device function every qGEMM shares), and the
// device quantizers used to build the benchmark's frozen base.
//
// Bit-exactness: the reference decodes in f32 with one rounding per operation
// (src/gguf.rs:354-367 Q8_0, :385-413 Q4_K, :449-477 Q6_K) and never fuses a*b-c. All
// arithmetic here keeps the reference's order, and this file is compiled with -ffp-contract=off so no
// product is fused into a following add (header intrinsics included).
#include "kernels.hpp"

namespace hos {

__device__ __forceinline__ float f16bits_to_f32(uint16_t h) {
  _Float16 v;
  __builtin_memcpy(&v, &h, 2);
  return (float)v;  // exact widening
}

// get_scale_min_k4, src/gguf.rs:43-51.
__device__ __forceinline__ void scale_min_k4(int j, const uint8_t* q, uint32_t* d, uint32_t* m) {
  if (j < 4) {
    *d = q[j] & 63;
    *m = q[j + 4] & 63;
  } else {
    *d = (q[j + 4] & 0x0F) | ((q[j - 4] >> 6) << 4);
    *m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
  }
}

// ---------------------------------------------------------------------------------------
// Repack: one thread per group (Q8_0 block of 32, Q4_K sub-block of 32, Q6_K group of 16).
// ---------------------------------------------------------------------------------------

__global__ void repack_q8_0(const uint8_t* __restrict__ src, int8_t* __restrict__ q, float* __restrict__ s,
                            long long nblocks) {
  long long b = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= nblocks) return;
  const uint8_t* blk = src + b * 34;
  s[b] = f16bits_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
  int8_t* dst = q + b * 32;
  for (int j = 0; j < 32; j++) dst[j] = (int8_t)blk[2 + j];
}

// Q4_K super-block (144 B): d f16, dmin f16, scales[12], qs[128]. Sub-block j (32 values) is
// the low (even j) or high (odd j) nibble of qs[32·(j/2) + l] (src/gguf.rs:385-413).
__global__ void repack_q4_k(const uint8_t* __restrict__ src, uint8_t* __restrict__ q, float2* __restrict__ s,
                            long long nsub) {
#pragma clang fp contract(off)
  long long g = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (g >= nsub) return;
  long long sb = g >> 3;
  int j = (int)(g & 7);
  const uint8_t* blk = src + sb * 144;
  float d = f16bits_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
  float dmin = f16bits_to_f32((uint16_t)(blk[2] | (blk[3] << 8)));
  uint32_t sc, m;
  scale_min_k4(j, blk + 4, &sc, &m);
  s[g] = make_float2(__fmul_rn(d, (float)sc), __fmul_rn(dmin, (float)m));
  const uint8_t* qs = blk + 16 + 32 * (j >> 1);
  int sh = (j & 1) * 4;
  uint8_t* dst = q + g * 16;
  for (int i = 0; i < 16; i++) {
    uint32_t lo = (qs[2 * i] >> sh) & 15u, hi = (qs[2 * i + 1] >> sh) & 15u;
    dst[i] = (uint8_t)(lo | (hi << 4));
  }
}

// Q6_K super-block (210 B): ql[128], qh[64], int8 scales[16], d f16. Element e uses scale
// sc[e/16] (src/gguf.rs:449-477).
__global__ void repack_q6_k(const uint8_t* __restrict__ src, int8_t* __restrict__ q, float* __restrict__ s,
                            long long ngroups) {
#pragma clang fp contract(off)
  long long g = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (g >= ngroups) return;
  long long sb = g >> 4;
  int grp = (int)(g & 15);
  const uint8_t* blk = src + sb * 210;
  float d = f16bits_to_f32((uint16_t)(blk[208] | (blk[209] << 8)));
  s[g] = __fmul_rn(d, (float)(int8_t)blk[192 + grp]);
  int8_t* dst = q + g * 16;
  for (int i = 0; i < 16; i++) {
    int e = grp * 16 + i;
    int n128 = e >> 7, r = e & 127, qq = r >> 5, l = r & 31;
    uint32_t lq = blk[64 * n128 + l + 32 * (qq & 1)];
    uint32_t low = (qq >> 1) ? (lq >> 4) : (lq & 15u);
    uint32_t hb = (blk[128 + 32 * n128 + l] >> (2 * qq)) & 3u;
    dst[i] = (int8_t)((int)(low | (hb << 4)) - 32);
  }
}

// Q4_0 block (18 B): d f16, qs[16]; element j < 16 is the low nibble of qs[j], j ≥ 16 the high nibble of
// qs[j − 16], value (q − 8)·d (src/gguf.rs:368-384). Stored as the Q8_0 layout with int8 q − 8: the Q8_0 decode
// (float)q · d is then the same product, bit for bit.
__global__ void repack_q4_0(const uint8_t* __restrict__ src, int8_t* __restrict__ q, float* __restrict__ s,
                            long long nblocks) {
  long long b = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= nblocks) return;
  const uint8_t* blk = src + b * 18;
  s[b] = f16bits_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
  int8_t* dst = q + b * 32;
  for (int j = 0; j < 16; j++) {
    dst[j] = (int8_t)((int)(blk[2 + j] & 15u) - 8);
    dst[j + 16] = (int8_t)((int)(blk[2 + j] >> 4) - 8);
  }
}

// Q5_0 block (22 B): d f16, qh u32 (bit j = 5th bit of element j), qs[16] as Q4_0; value (q − 16)·d
// (src/gguf.rs:478-505). Stored as the Q8_0 layout with int8 q − 16.
__global__ void repack_q5_0(const uint8_t* __restrict__ src, int8_t* __restrict__ q, float* __restrict__ s,
                            long long nblocks) {
  long long b = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= nblocks) return;
  const uint8_t* blk = src + b * 22;
  s[b] = f16bits_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
  const uint32_t qh = (uint32_t)blk[2] | ((uint32_t)blk[3] << 8) | ((uint32_t)blk[4] << 16) | ((uint32_t)blk[5] << 24);
  int8_t* dst = q + b * 32;
  for (int j = 0; j < 16; j++) {
    const int x0 = (int)((blk[6 + j] & 15u) | (((qh >> j) & 1u) << 4));
    const int x1 = (int)((blk[6 + j] >> 4) | (((qh >> (j + 16)) & 1u) << 4));
    dst[j] = (int8_t)(x0 - 16);
    dst[j + 16] = (int8_t)(x1 - 16);
  }
}

// Q5_K super-block (176 B): d f16, dmin f16, scales[12], qh[32], qs[128]; sub-block j (32 values) takes the low
// (even j) or high (odd j) nibbles of qs[32·(j/2) + l] plus 16 when bit j of qh[l] is set (src/gguf.rs:414-448).
// Stored as one byte per 5-bit code and float2 {d·sc, dmin·m} per sub-block, as Q4_K's scales.
__global__ void repack_q5_k(const uint8_t* __restrict__ src, uint8_t* __restrict__ q, float2* __restrict__ s,
                            long long nsub) {
#pragma clang fp contract(off)
  long long g = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (g >= nsub) return;
  long long sb = g >> 3;
  int j = (int)(g & 7);
  const uint8_t* blk = src + sb * 176;
  float d = f16bits_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
  float dmin = f16bits_to_f32((uint16_t)(blk[2] | (blk[3] << 8)));
  uint32_t sc, m;
  scale_min_k4(j, blk + 4, &sc, &m);
  s[g] = make_float2(__fmul_rn(d, (float)sc), __fmul_rn(dmin, (float)m));
  const uint8_t* qh = blk + 16;
  const uint8_t* qs = blk + 48 + 32 * (j >> 1);
  const int sh = (j & 1) * 4;
  uint8_t* dst = q + g * 32;
  for (int l = 0; l < 32; l++) dst[l] = (uint8_t)(((qs[l] >> sh) & 15u) | (((qh[l] >> j) & 1u) << 4));
}

// Dequant of the whole weight to f32 (for the bit-exact check); one thread per element.
__global__ void dequant_kernel(QWeightView w, float* __restrict__ out, long long n) {
  long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  long long r = i / w.cols, c = i % w.cols;
  out[i] = deq_one(w, r, c);
}

// ---------------------------------------------------------------------------------------
// Device quantizers (byte-identical to src/gguf_write.rs).
// ---------------------------------------------------------------------------------------

__device__ __forceinline__ int sat_i32(float v) {
  if (v != v) return 0;
  if (v >= 2147483647.0f) return 2147483647;
  if (v <= -2147483648.0f) return (-2147483647 - 1);
  return (int)v;
}
__device__ __forceinline__ int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }
__device__ __forceinline__ uint16_t f32_to_f16bits(float v) {
  _Float16 h = (_Float16)v;  // IEEE round-to-nearest-even
  uint16_t b;
  __builtin_memcpy(&b, &h, 2);
  return b;
}

// quantize_q8_0, src/gguf_write.rs:178-196. One thread per 32-block.
__global__ void quantize_q8_0_kernel(const float* __restrict__ x, uint8_t* __restrict__ out, long long nblocks) {
#pragma clang fp contract(off)
  long long b = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= nblocks) return;
  const float* v = x + b * 32;
  float amax = 0.0f;
  for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(v[i]));
  float d = div_rn(amax, 127.0f);
  float id = d != 0.0f ? div_rn(1.0f, d) : 0.0f;
  uint8_t* o = out + b * 34;
  uint16_t hd = f32_to_f16bits(d);
  o[0] = (uint8_t)(hd & 0xff);
  o[1] = (uint8_t)(hd >> 8);
  for (int i = 0; i < 32; i++) {
    float r = roundf(__fmul_rn(v[i], id));
    r = (r != r) ? r : fminf(fmaxf(r, -127.0f), 127.0f);
    o[2 + i] = (uint8_t)(int8_t)((r != r) ? 0 : (int)r);
  }
}

// qkx_scale_min, src/gguf_write.rs:293-351.
__device__ void qkx_scale_min(const float* x, int nmax, float* out_s, float* out_m) {
#pragma clang fp contract(off)
  float mn = x[0], mx = x[0];
  for (int i = 0; i < 32; i++) {
    mn = fminf(mn, x[i]);
    mx = fmaxf(mx, x[i]);
  }
  if (mn > 0.0f) mn = 0.0f;
  if (mx == mn) {
    *out_s = 0.0f;
    *out_m = -mn;
    return;
  }
  float nf = 32.0f, span = __fsub_rn(mx, mn), nm = (float)nmax;
  float best_s = div_rn(span, nm), best_m = -mn, best_err = 3.40282347e+38f;
  for (int it = 0; it <= 18; it++) {
    float iscale = div_rn(__fadd_rn(__fsub_rn(nm, 1.0f), __fmul_rn(0.1f, (float)it)), span);
    if (iscale <= 0.0f) continue;
    float sl = 0.0f, sl2 = 0.0f, sx = 0.0f, slx = 0.0f;
    for (int k = 0; k < 32; k++) {
      float v = x[k];
      float l = (float)clampi(sat_i32(roundf(__fmul_rn(iscale, __fsub_rn(v, mn)))), 0, nmax);
      sl = __fadd_rn(sl, l);
      sl2 = __fadd_rn(sl2, __fmul_rn(l, l));
      sx = __fadd_rn(sx, v);
      slx = __fadd_rn(slx, __fmul_rn(l, v));
    }
    float denom = __fsub_rn(__fmul_rn(nf, sl2), __fmul_rn(sl, sl));
    float scale, min;
    if (denom > 0.0f) {
      float s = div_rn(__fsub_rn(__fmul_rn(nf, slx), __fmul_rn(sl, sx)), denom);
      float b = div_rn(__fsub_rn(sx, __fmul_rn(s, sl)), nf);
      if (s > 0.0f) {
        scale = s;
        min = fmaxf(-b, 0.0f);
      } else {
        scale = div_rn(span, nm);
        min = -mn;
      }
    } else {
      scale = div_rn(span, nm);
      min = -mn;
    }
    float inv = div_rn(1.0f, scale);
    float err = 0.0f;
    for (int k = 0; k < 32; k++) {
      float v = x[k];
      float l = (float)clampi(sat_i32(roundf(__fmul_rn(__fadd_rn(v, min), inv))), 0, nmax);
      float dd = __fsub_rn(__fsub_rn(__fmul_rn(scale, l), min), v);
      err = __fadd_rn(err, __fmul_rn(dd, dd));
    }
    if (err < best_err) {
      best_err = err;
      best_s = scale;
      best_m = min;
    }
  }
  *out_s = best_s;
  *out_m = best_m;
}

// quantize_qx_k (nmax 15), src/gguf_write.rs:355-412. One thread per super-block.
__global__ void quantize_q4_k_kernel(const float* __restrict__ x, uint8_t* __restrict__ out, long long nsb) {
#pragma clang fp contract(off)
  long long b = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= nsb) return;
  const float* sb = x + b * 256;
  float scales[8], mins[8];
  for (int j = 0; j < 8; j++) qkx_scale_min(sb + 32 * j, 15, &scales[j], &mins[j]);
  float max_scale = 0.0f, max_min = 0.0f;
  for (int j = 0; j < 8; j++) max_scale = fmaxf(max_scale, scales[j]);
  for (int j = 0; j < 8; j++) max_min = fmaxf(max_min, mins[j]);
  float d = div_rn(max_scale, 63.0f), dmin = div_rn(max_min, 63.0f);
  float id = d > 0.0f ? div_rn(1.0f, d) : 0.0f;
  float idm = dmin > 0.0f ? div_rn(1.0f, dmin) : 0.0f;
  uint32_t ls[8], lm[8];
  for (int j = 0; j < 8; j++) {
    ls[j] = (uint32_t)clampi(sat_i32(roundf(__fmul_rn(scales[j], id))), 0, 63);
    lm[j] = (uint32_t)clampi(sat_i32(roundf(__fmul_rn(mins[j], idm))), 0, 63);
  }
  uint8_t* o = out + b * 144;
  uint16_t hd = f32_to_f16bits(d), hdm = f32_to_f16bits(dmin);
  o[0] = (uint8_t)(hd & 0xff);
  o[1] = (uint8_t)(hd >> 8);
  o[2] = (uint8_t)(hdm & 0xff);
  o[3] = (uint8_t)(hdm >> 8);
  uint8_t pk[12] = {0};
  for (int j = 0; j < 8; j++) {  // pack_scales_mins, src/gguf_write.rs:270-285
    if (j < 4) {
      pk[j] = (uint8_t)ls[j];
      pk[j + 4] = (uint8_t)lm[j];
    } else {
      pk[j + 4] = (uint8_t)((ls[j] & 0xF) | ((lm[j] & 0xF) << 4));
      pk[j - 4] |= (uint8_t)((ls[j] >> 4) << 6);
      pk[j] |= (uint8_t)((lm[j] >> 4) << 6);
    }
  }
  for (int i = 0; i < 12; i++) o[4 + i] = pk[i];
  for (int g = 0; g < 4; g++) {
    float dq0 = __fmul_rn(d, (float)ls[2 * g]), mq0 = __fmul_rn(dmin, (float)lm[2 * g]);
    float dq1 = __fmul_rn(d, (float)ls[2 * g + 1]), mq1 = __fmul_rn(dmin, (float)lm[2 * g + 1]);
    for (int l = 0; l < 32; l++) {
      float v0 = sb[g * 64 + l], v1 = sb[g * 64 + 32 + l];
      uint32_t q0 = dq0 > 0.0f ? (uint32_t)clampi(sat_i32(roundf(div_rn(__fadd_rn(v0, mq0), dq0))), 0, 15) : 0u;
      uint32_t q1 = dq1 > 0.0f ? (uint32_t)clampi(sat_i32(roundf(div_rn(__fadd_rn(v1, mq1), dq1))), 0, 15) : 0u;
      o[16 + g * 32 + l] = (uint8_t)((q0 & 15u) | ((q1 & 15u) << 4));
    }
  }
}

// quantize_q6_k, src/gguf_write.rs:426-495. One thread per super-block.
__global__ void quantize_q6_k_kernel(const float* __restrict__ x, uint8_t* __restrict__ out, long long nsb) {
#pragma clang fp contract(off)
  long long b = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= nsb) return;
  const float* sb = x + b * 256;
  float subscale[16];
  for (int s = 0; s < 16; s++) {
    float mx = 0.0f, amax = 0.0f;
    for (int i = 0; i < 16; i++) {
      float v = sb[s * 16 + i];
      if (fabsf(v) > amax) {
        amax = fabsf(v);
        mx = v;
      }
    }
    subscale[s] = amax > 0.0f ? div_rn(mx, -32.0f) : 0.0f;
  }
  float max_scale = 0.0f;
  for (int s = 0; s < 16; s++)
    if (fabsf(subscale[s]) > fabsf(max_scale)) max_scale = subscale[s];
  float d = 0.0f, idd = 0.0f;
  if (max_scale != 0.0f) {
    d = div_rn(max_scale, -128.0f);
    idd = div_rn(-128.0f, max_scale);
  }
  int sc[16];
  for (int s = 0; s < 16; s++) sc[s] = clampi(sat_i32(roundf(__fmul_rn(subscale[s], idd))), -128, 127);
  uint8_t* o = out + b * 210;
  for (int i = 0; i < 128 + 64; i++) o[i] = 0;
  for (int e = 0; e < 256; e++) {
    float scale = __fmul_rn(d, (float)sc[e >> 4]);
    int q = scale != 0.0f ? clampi(sat_i32(roundf(div_rn(sb[e], scale))), -32, 31) : 0;
    uint32_t u = (uint32_t)(q + 32) & 63u;
    int n128 = e >> 7, r = e & 127, qq = r >> 5, l = r & 31;
    o[64 * n128 + l + 32 * (qq & 1)] |= (uint8_t)((u & 15u) << (4 * (qq >> 1)));
    o[128 + 32 * n128 + l] |= (uint8_t)((u >> 4) << (2 * qq));
  }
  for (int s = 0; s < 16; s++) o[192 + s] = (uint8_t)(int8_t)sc[s];
  uint16_t hd = f32_to_f16bits(d);
  o[208] = (uint8_t)(hd & 0xff);
  o[209] = (uint8_t)(hd >> 8);
}

// ---------------------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------------------

size_t gguf_bytes_for(uint32_t t, size_t n) {
  switch (t) {
    case GGUF_F32: return n * 4;
    case GGUF_F16:
    case GGUF_BF16: return n * 2;
    case GGUF_Q4_0: return n / 32 * 18;
    case GGUF_Q5_0: return n / 32 * 22;
    case GGUF_Q8_0: return n / 32 * 34;
    case GGUF_Q4_K: return n / 256 * 144;
    case GGUF_Q5_K: return n / 256 * 176;
    case GGUF_Q6_K: return n / 256 * 210;
    default: return 0;
  }
}

// Elements per GGUF block of a matrix type the GEMMs read (0: not a weight encoding the GEMMs read).
size_t block_elems(uint32_t t) {
  switch (t) {
    case GGUF_F32:
    case GGUF_F16:
    case GGUF_BF16: return 1;
    case GGUF_Q4_0:
    case GGUF_Q5_0:
    case GGUF_Q8_0: return 32;
    case GGUF_Q4_K:
    case GGUF_Q5_K:
    case GGUF_Q6_K: return 256;
    default: return 0;
  }
}

uint32_t storage_type(uint32_t t) { return (t == GGUF_Q4_0 || t == GGUF_Q5_0) ? GGUF_Q8_0 : t; }

void repack_weight(const uint8_t* src_dev, uint32_t src_type, QWeight& w, hipStream_t st) {
  long long n = w.rows * w.cols;
  switch (src_type) {
    case GGUF_Q4_0: {
      long long nb = n / 32;
      repack_q4_0<<<ceil_div(nb, 256), 256, 0, st>>>(src_dev, (int8_t*)w.q, w.s, nb);
      break;
    }
    case GGUF_Q5_0: {
      long long nb = n / 32;
      repack_q5_0<<<ceil_div(nb, 256), 256, 0, st>>>(src_dev, (int8_t*)w.q, w.s, nb);
      break;
    }
    case GGUF_Q5_K: {
      long long ns = n / 32;
      repack_q5_k<<<ceil_div(ns, 256), 256, 0, st>>>(src_dev, (uint8_t*)w.q, (float2*)w.s, ns);
      break;
    }
    case GGUF_F32:
    case GGUF_F16:
    case GGUF_BF16:  // stored as the file holds them
      HOS_HIP_CHECK(hipMemcpyAsync(w.q, src_dev, w.q_bytes, hipMemcpyDeviceToDevice, st));
      break;
    case GGUF_Q8_0: {
      long long nb = n / 32;
      repack_q8_0<<<ceil_div(nb, 256), 256, 0, st>>>(src_dev, (int8_t*)w.q, w.s, nb);
      break;
    }
    case GGUF_Q4_K: {
      long long ns = n / 32;
      repack_q4_k<<<ceil_div(ns, 256), 256, 0, st>>>(src_dev, (uint8_t*)w.q, (float2*)w.s, ns);
      break;
    }
    case GGUF_Q6_K: {
      long long ng = n / 16;
      repack_q6_k<<<ceil_div(ng, 256), 256, 0, st>>>(src_dev, (int8_t*)w.q, w.s, ng);
      break;
    }
    default:
      throw Error(HOS_E_UNSUPPORTED_QUANT, "repack: unsupported quant type " + std::to_string(w.type));
  }
  HOS_HIP_CHECK(hipGetLastError());
}

void qweight_sizes(uint32_t type, long long rows, long long cols, size_t* q_bytes, size_t* s_bytes) {
  long long n = rows * cols;
  switch (type) {
    case GGUF_Q8_0: *q_bytes = n; *s_bytes = n / 32 * 4; break;
    case GGUF_Q4_K: *q_bytes = n / 2; *s_bytes = n / 32 * 8; break;
    case GGUF_Q6_K: *q_bytes = n; *s_bytes = n / 16 * 4; break;
    case GGUF_Q5_K: *q_bytes = n; *s_bytes = n / 32 * 8; break;
    case GGUF_F16:
    case GGUF_BF16: *q_bytes = 2 * n; *s_bytes = 0; break;
    case GGUF_F32: *q_bytes = 4 * n; *s_bytes = 0; break;
    default: throw Error(HOS_E_UNSUPPORTED_QUANT, "unsupported quant type " + std::to_string(type));
  }
}

void launch_dequant(const QWeight& w, float* out_dev, hipStream_t st) {
  long long n = w.rows * w.cols;
  dequant_kernel<<<ceil_div(n, 256), 256, 0, st>>>(view(w), out_dev, n);
  HOS_HIP_CHECK(hipGetLastError());
}

void launch_quantize(const float* x_dev, size_t n, uint32_t type, uint8_t* out_dev, hipStream_t st) {
  switch (type) {
    case GGUF_Q8_0: {
      long long nb = n / 32;
      quantize_q8_0_kernel<<<ceil_div(nb, 128), 128, 0, st>>>(x_dev, out_dev, nb);
      break;
    }
    case GGUF_Q4_K: {
      long long nb = n / 256;
      quantize_q4_k_kernel<<<ceil_div(nb, 64), 64, 0, st>>>(x_dev, out_dev, nb);
      break;
    }
    case GGUF_Q6_K: {
      long long nb = n / 256;
      quantize_q6_k_kernel<<<ceil_div(nb, 64), 64, 0, st>>>(x_dev, out_dev, nb);
      break;
    }
    default:
      throw Error(HOS_E_UNSUPPORTED_QUANT, "quantize: unsupported type " + std::to_string(type));
  }
  HOS_HIP_CHECK(hipGetLastError());
}

}  // namespace hos
