// ORACLE — test infrastructure only. CPU restatement of HOS's GGUF block codec
// (dequantizers and quantizers) used as the parity checker for the HIP backend.
// Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.
//
// Follows, function by function:
//   f16 decode          half 2.7.1 f16::to_f32 (exact IEEE binary16 -> binary32)
//   f16 encode          half 2.7.1 f16::from_f32 (IEEE round-to-nearest-even)
//   scale_min_k4        src/gguf.rs:43-51
//   dequant_into        src/gguf.rs:330-505 (F32 :333, F16 :343, BF16 :349, Q8_0 :354-367,
//                       Q4_0 :369-384, Q4_K :385-413, Q5_K :414-448, Q6_K :449-477, Q5_0 :478-501)
//   bytes_for           src/gguf.rs:548-561
//   quantize_q8_0       src/gguf_write.rs:178-196
//   quantize_q4_0       src/gguf_write.rs:200-223
//   quantize_q5_0       src/gguf_write.rs:227-258
//   pack_scales_mins    src/gguf_write.rs:270-285
//   qkx_scale_min       src/gguf_write.rs:293-351
//   quantize_qx_k       src/gguf_write.rs:355-412 (Q4_K nmax 15, Q5_K nmax 31)
//   quantize_q6_k       src/gguf_write.rs:426-495
// Compiled with -ffp-contract=off so every a*b+c rounds twice, as Rust does.
#include "oracle.h"

#include <cmath>
#include <cstring>
#include <vector>

namespace orc {

float f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1fu;
  uint32_t man = h & 0x3ffu;
  uint32_t bits;
  if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else {
      float f = (float)man * 5.9604644775390625e-08f;  // man * 2^-24, exact
      std::memcpy(&bits, &f, 4);
      bits |= sign;
    }
  } else if (exp == 31) {
    bits = sign | 0x7f800000u | (man << 13);
  } else {
    bits = sign | ((exp + 112u) << 23) | (man << 13);
  }
  float out;
  std::memcpy(&out, &bits, 4);
  return out;
}

uint16_t f32_to_f16(float f) {
  uint32_t x;
  std::memcpy(&x, &f, 4);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t exp = (x >> 23) & 0xffu;
  uint32_t man = x & 0x7fffffu;
  if (exp == 0xff) return (uint16_t)(sign | 0x7c00u | (man ? (0x200u | (man >> 13)) : 0u));
  int e = (int)exp - 127 + 15;
  if (e >= 31) return (uint16_t)(sign | 0x7c00u);
  if (e <= 0) {
    if (e < -10) return (uint16_t)sign;
    uint32_t m = man | 0x800000u;
    int shift = 14 - e;
    uint32_t hm = m >> shift;
    uint32_t rem = m & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (hm & 1u))) hm++;
    return (uint16_t)(sign | hm);
  }
  uint32_t hm = man >> 13;
  uint32_t rem = man & 0x1fffu;
  uint32_t r = sign | ((uint32_t)e << 10) | hm;
  if (rem > 0x1000u || (rem == 0x1000u && (hm & 1u))) r++;
  return (uint16_t)r;
}

static inline float rd_f16(const uint8_t* b, size_t at) {
  return f16_to_f32((uint16_t)(b[at] | (b[at + 1] << 8)));
}

// Rust `f32 as i32`: saturating, NaN -> 0.
static inline int32_t sat_i32(float v) {
  if (v != v) return 0;
  if (v >= 2147483647.0f) return 2147483647;
  if (v <= -2147483648.0f) return (-2147483647 - 1);
  return (int32_t)v;
}
static inline int32_t clampi(int32_t v, int32_t lo, int32_t hi) { return v < lo ? lo : (v > hi ? hi : v); }
// Rust f32::round: half away from zero (C roundf).
static inline float rround(float v) { return std::roundf(v); }
// Rust f32::max / f32::min (IEEE maxNum/minNum).
static inline float rmax(float a, float b) { return std::fmax(a, b); }
static inline float rmin(float a, float b) { return std::fmin(a, b); }

static inline void scale_min_k4(int j, const uint8_t* q, uint8_t* d, uint8_t* m) {
  if (j < 4) {
    *d = q[j] & 63;
    *m = q[j + 4] & 63;
  } else {
    *d = (uint8_t)((q[j + 4] & 0x0F) | ((q[j - 4] >> 6) << 4));
    *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
  }
}

size_t bytes_for(uint32_t t, size_t n) {
  switch (t) {
    case GGML_F32: return n * 4;
    case GGML_F16: return n * 2;
    case GGML_BF16: return n * 2;
    case GGML_Q8_0: return n / 32 * 34;
    case GGML_Q4_0: return n / 32 * 18;
    case GGML_Q5_0: return n / 32 * 22;
    case GGML_Q4_K: return n / 256 * 144;
    case GGML_Q5_K: return n / 256 * 176;
    case GGML_Q6_K: return n / 256 * 210;
    default: return 0;
  }
}

int dequant_into(const uint8_t* bytes, uint32_t t, size_t n, float* out) {
  switch (t) {
    case GGML_F32:
      for (size_t i = 0; i < n; i++) std::memcpy(&out[i], bytes + 4 * i, 4);
      return 0;
    case GGML_F16:
      for (size_t i = 0; i < n; i++) out[i] = rd_f16(bytes, 2 * i);
      return 0;
    case GGML_BF16:
      for (size_t i = 0; i < n; i++) {
        uint32_t b = (uint32_t)(bytes[2 * i] | (bytes[2 * i + 1] << 8)) << 16;
        std::memcpy(&out[i], &b, 4);
      }
      return 0;
    case GGML_Q8_0: {
      size_t nb = n / 32;
      for (size_t b = 0; b < nb; b++) {
        const uint8_t* blk = bytes + b * 34;
        float d = rd_f16(blk, 0);
        for (int j = 0; j < 32; j++) out[b * 32 + j] = (float)(int8_t)blk[2 + j] * d;
      }
      return 0;
    }
    case GGML_Q4_0: {
      size_t nb = n / 32;
      for (size_t b = 0; b < nb; b++) {
        const uint8_t* blk = bytes + b * 18;
        float d = rd_f16(blk, 0);
        for (int j = 0; j < 16; j++) {
          uint8_t q = blk[2 + j];
          out[b * 32 + j] = (float)((int)(q & 0x0F) - 8) * d;
          out[b * 32 + j + 16] = (float)((int)(q >> 4) - 8) * d;
        }
      }
      return 0;
    }
    case GGML_Q4_K: {
      size_t nb = n / 256;
      for (size_t b = 0; b < nb; b++) {
        const uint8_t* blk = bytes + b * 144;
        float d = rd_f16(blk, 0), dmin = rd_f16(blk, 2);
        const uint8_t* sc = blk + 4;
        const uint8_t* qs = blk + 16;
        size_t y = b * 256;
        int is = 0;
        for (int j = 0; j < 256; j += 64) {
          uint8_t s1, m1, s2, m2;
          scale_min_k4(is, sc, &s1, &m1);
          scale_min_k4(is + 1, sc, &s2, &m2);
          float d1 = d * (float)s1, mn1 = dmin * (float)m1;
          float d2 = d * (float)s2, mn2 = dmin * (float)m2;
          const uint8_t* q = qs + j / 2;
          for (int l = 0; l < 32; l++) out[y + l] = d1 * (float)(q[l] & 0x0F) - mn1;
          for (int l = 0; l < 32; l++) out[y + 32 + l] = d2 * (float)(q[l] >> 4) - mn2;
          y += 64;
          is += 2;
        }
      }
      return 0;
    }
    case GGML_Q5_K: {
      size_t nb = n / 256;
      for (size_t b = 0; b < nb; b++) {
        const uint8_t* blk = bytes + b * 176;
        float d = rd_f16(blk, 0), dmin = rd_f16(blk, 2);
        const uint8_t* sc = blk + 4;
        const uint8_t* qh = blk + 16;
        const uint8_t* qs = blk + 48;
        size_t y = b * 256;
        int is = 0;
        uint8_t u1 = 1, u2 = 2;
        for (int j = 0; j < 256; j += 64) {
          uint8_t s1, m1, s2, m2;
          scale_min_k4(is, sc, &s1, &m1);
          scale_min_k4(is + 1, sc, &s2, &m2);
          float d1 = d * (float)s1, mn1 = dmin * (float)m1;
          float d2 = d * (float)s2, mn2 = dmin * (float)m2;
          const uint8_t* q = qs + j / 2;
          for (int l = 0; l < 32; l++) {
            float hi = (qh[l] & u1) ? 16.0f : 0.0f;
            out[y + l] = d1 * ((float)(q[l] & 0x0F) + hi) - mn1;
          }
          for (int l = 0; l < 32; l++) {
            float hi = (qh[l] & u2) ? 16.0f : 0.0f;
            out[y + 32 + l] = d2 * ((float)(q[l] >> 4) + hi) - mn2;
          }
          y += 64;
          is += 2;
          u1 = (uint8_t)(u1 << 2);
          u2 = (uint8_t)(u2 << 2);
        }
      }
      return 0;
    }
    case GGML_Q6_K: {
      size_t nb = n / 256;
      for (size_t b = 0; b < nb; b++) {
        const uint8_t* blk = bytes + b * 210;
        float d = rd_f16(blk, 208);
        for (int n128 = 0; n128 < 2; n128++) {
          const uint8_t* ql = blk + n128 * 64;
          const uint8_t* qh = blk + 128 + n128 * 32;
          const int8_t* sc = (const int8_t*)(blk + 192 + n128 * 8);
          size_t y0 = b * 256 + n128 * 128;
          for (int l = 0; l < 32; l++) {
            int is = l / 16;
            int q1 = (int)((ql[l] & 0x0F) | ((qh[l] & 3) << 4)) - 32;
            int q2 = (int)((ql[l + 32] & 0x0F) | (((qh[l] >> 2) & 3) << 4)) - 32;
            int q3 = (int)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
            int q4 = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
            out[y0 + l] = d * (float)sc[is] * (float)q1;
            out[y0 + l + 32] = d * (float)sc[is + 2] * (float)q2;
            out[y0 + l + 64] = d * (float)sc[is + 4] * (float)q3;
            out[y0 + l + 96] = d * (float)sc[is + 6] * (float)q4;
          }
        }
      }
      return 0;
    }
    case GGML_Q5_0: {
      size_t nb = n / 32;
      for (size_t b = 0; b < nb; b++) {
        const uint8_t* blk = bytes + b * 22;
        float d = rd_f16(blk, 0);
        uint32_t qh = (uint32_t)blk[2] | ((uint32_t)blk[3] << 8) | ((uint32_t)blk[4] << 16) |
                      ((uint32_t)blk[5] << 24);
        for (int j = 0; j < 16; j++) {
          int xh0 = (int)(((qh >> j) << 4) & 0x10);
          int xh1 = (int)((qh >> (j + 12)) & 0x10);
          uint8_t q = blk[6 + j];
          int x0 = ((int)(q & 0x0F) | xh0) - 16;
          int x1 = ((int)(q >> 4) | xh1) - 16;
          out[b * 32 + j] = (float)x0 * d;
          out[b * 32 + j + 16] = (float)x1 * d;
        }
      }
      return 0;
    }
    default:
      return ORC_E_UNSUPPORTED_QUANT;
  }
}

static void put_f16(std::vector<uint8_t>& o, float v) {
  uint16_t h = f32_to_f16(v);
  o.push_back((uint8_t)(h & 0xff));
  o.push_back((uint8_t)(h >> 8));
}

static void quantize_q8_0(const float* x, size_t n, std::vector<uint8_t>& out) {
  for (size_t b0 = 0; b0 < n; b0 += 32) {
    size_t len = (n - b0 < 32) ? n - b0 : 32;
    float amax = 0.0f;
    for (size_t i = 0; i < len; i++) amax = rmax(amax, std::fabs(x[b0 + i]));
    float d = amax / 127.0f;
    float id = (d != 0.0f) ? 1.0f / d : 0.0f;
    put_f16(out, d);
    for (size_t i = 0; i < len; i++) {
      float r = rround(x[b0 + i] * id);
      r = (r != r) ? r : (r < -127.0f ? -127.0f : (r > 127.0f ? 127.0f : r));
      // Rust `f32 as i8`: saturating, NaN -> 0.
      int8_t q = (r != r) ? 0 : (int8_t)(int)r;
      out.push_back((uint8_t)q);
    }
    for (size_t i = len; i < 32; i++) out.push_back(0);
  }
}

static void quantize_q4_0(const float* x, size_t n, std::vector<uint8_t>& out) {
  for (size_t b0 = 0; b0 < n; b0 += 32) {
    size_t len = (n - b0 < 32) ? n - b0 : 32;
    float mx = 0.0f, amax = 0.0f;
    for (size_t i = 0; i < len; i++) {
      float v = x[b0 + i];
      if (std::fabs(v) > amax) { amax = std::fabs(v); mx = v; }
    }
    float d = mx / -8.0f;
    float id = (d != 0.0f) ? 1.0f / d : 0.0f;
    put_f16(out, d);
    for (int j = 0; j < 16; j++) {
      float lo = ((size_t)j < len ? x[b0 + j] : 0.0f) * id;
      float hi = ((size_t)(j + 16) < len ? x[b0 + j + 16] : 0.0f) * id;
      uint8_t xi0 = (uint8_t)clampi(sat_i32(lo + 8.5f), 0, 15);
      uint8_t xi1 = (uint8_t)clampi(sat_i32(hi + 8.5f), 0, 15);
      out.push_back((uint8_t)(xi0 | (xi1 << 4)));
    }
  }
}

static void quantize_q5_0(const float* x, size_t n, std::vector<uint8_t>& out) {
  for (size_t b0 = 0; b0 < n; b0 += 32) {
    size_t len = (n - b0 < 32) ? n - b0 : 32;
    float mx = 0.0f, amax = 0.0f;
    for (size_t i = 0; i < len; i++) {
      float v = x[b0 + i];
      if (std::fabs(v) > amax) { amax = std::fabs(v); mx = v; }
    }
    float d = mx / -16.0f;
    float id = (d != 0.0f) ? 1.0f / d : 0.0f;
    put_f16(out, d);
    uint32_t qh = 0;
    uint8_t qs[16] = {0};
    for (int j = 0; j < 16; j++) {
      float a = ((size_t)j < len ? x[b0 + j] : 0.0f);
      float b = ((size_t)(j + 16) < len ? x[b0 + j + 16] : 0.0f);
      uint32_t v0 = (uint32_t)clampi(sat_i32(a * id + 16.5f), 0, 31);
      uint32_t v1 = (uint32_t)clampi(sat_i32(b * id + 16.5f), 0, 31);
      qs[j] = (uint8_t)((v0 & 0x0F) | ((v1 & 0x0F) << 4));
      qh |= ((v0 >> 4) & 1u) << j;
      qh |= ((v1 >> 4) & 1u) << (j + 16);
    }
    for (int i = 0; i < 4; i++) out.push_back((uint8_t)(qh >> (8 * i)));
    for (int j = 0; j < 16; j++) out.push_back(qs[j]);
  }
}

void pack_scales_mins(const uint8_t* scales, const uint8_t* mins, uint8_t* q) {
  std::memset(q, 0, 12);
  for (int j = 0; j < 8; j++) {
    uint8_t ls = scales[j] & 63, lm = mins[j] & 63;
    if (j < 4) {
      q[j] = ls;
      q[j + 4] = lm;
    } else {
      q[j + 4] = (uint8_t)((ls & 0xF) | ((lm & 0xF) << 4));
      q[j - 4] |= (uint8_t)((ls >> 4) << 6);
      q[j] |= (uint8_t)((lm >> 4) << 6);
    }
  }
}

void qkx_scale_min(const float* x, int len, int nmax, float* out_scale, float* out_min) {
  float mn = x[0], mx = x[0];
  for (int i = 0; i < len; i++) {
    mn = rmin(mn, x[i]);
    mx = rmax(mx, x[i]);
  }
  if (mn > 0.0f) mn = 0.0f;
  if (mx == mn) {
    *out_scale = 0.0f;
    *out_min = -mn;
    return;
  }
  float nf = (float)len;
  float span = mx - mn;
  float nm = (float)nmax;
  float best_s = span / nm, best_m = -mn;
  float best_err = 3.40282347e+38f;
  for (int i = 0; i <= 18; i++) {
    float iscale = (nm - 1.0f + 0.1f * (float)i) / span;
    if (iscale <= 0.0f) continue;
    float sl = 0.0f, sl2 = 0.0f, sx = 0.0f, slx = 0.0f;
    for (int k = 0; k < len; k++) {
      float v = x[k];
      float l = (float)clampi(sat_i32(rround(iscale * (v - mn))), 0, nmax);
      sl += l;
      sl2 += l * l;
      sx += v;
      slx += l * v;
    }
    float denom = nf * sl2 - sl * sl;
    float scale, min;
    if (denom > 0.0f) {
      float s = (nf * slx - sl * sx) / denom;
      float b = (sx - s * sl) / nf;
      if (s > 0.0f) {
        scale = s;
        min = rmax(-b, 0.0f);
      } else {
        scale = span / nm;
        min = -mn;
      }
    } else {
      scale = span / nm;
      min = -mn;
    }
    float inv = 1.0f / scale;
    float err = 0.0f;
    for (int k = 0; k < len; k++) {
      float v = x[k];
      float l = (float)clampi(sat_i32(rround((v + min) * inv)), 0, nmax);
      float d = scale * l - min - v;
      err += d * d;
    }
    if (err < best_err) {
      best_err = err;
      best_s = scale;
      best_m = min;
    }
  }
  *out_scale = best_s;
  *out_min = best_m;
}

// One 256-element super-block of Q4_K (with_high=false) or Q5_K (with_high=true).
static void quantize_qx_k_block(const float* sb, int nmax, bool with_high, uint8_t* dst) {
  float scales[8], mins[8];
  for (int j = 0; j < 8; j++) qkx_scale_min(sb + j * 32, 32, nmax, &scales[j], &mins[j]);
  float max_scale = 0.0f, max_min = 0.0f;
  for (int j = 0; j < 8; j++) max_scale = rmax(max_scale, scales[j]);
  for (int j = 0; j < 8; j++) max_min = rmax(max_min, mins[j]);
  float d = max_scale / 63.0f;
  float dmin = max_min / 63.0f;
  float id = d > 0.0f ? 1.0f / d : 0.0f;
  float idm = dmin > 0.0f ? 1.0f / dmin : 0.0f;
  uint8_t ls[8], lm[8];
  for (int j = 0; j < 8; j++) {
    ls[j] = (uint8_t)clampi(sat_i32(rround(scales[j] * id)), 0, 63);
    lm[j] = (uint8_t)clampi(sat_i32(rround(mins[j] * idm)), 0, 63);
  }
  uint16_t hd = f32_to_f16(d), hdm = f32_to_f16(dmin);
  dst[0] = (uint8_t)(hd & 0xff);
  dst[1] = (uint8_t)(hd >> 8);
  dst[2] = (uint8_t)(hdm & 0xff);
  dst[3] = (uint8_t)(hdm >> 8);
  pack_scales_mins(ls, lm, dst + 4);
  uint8_t qs[128] = {0};
  uint8_t qh[32] = {0};
  for (int g = 0; g < 4; g++) {
    for (int half = 0; half < 2; half++) {
      int sub = 2 * g + half;
      int nib_shift = half ? 4 : 0;
      float dq = d * (float)ls[sub];
      float mq = dmin * (float)lm[sub];
      int off = half ? 32 : 0;
      for (int l = 0; l < 32; l++) {
        float v = sb[g * 64 + off + l];
        uint32_t q = dq > 0.0f ? (uint32_t)clampi(sat_i32(rround((v + mq) / dq)), 0, nmax) : 0u;
        qs[g * 32 + l] |= (uint8_t)((q & 0x0F) << nib_shift);
        if (with_high && ((q >> 4) & 1u)) qh[l] |= (uint8_t)(1u << (2 * g + half));
      }
    }
  }
  if (with_high) {
    std::memcpy(dst + 16, qh, 32);
    std::memcpy(dst + 48, qs, 128);
  } else {
    std::memcpy(dst + 16, qs, 128);
  }
}

static void quantize_q6_k_block(const float* sb, uint8_t* dst) {
  float subscale[16];
  for (int s = 0; s < 16; s++) {
    const float* blk = sb + s * 16;
    float mx = 0.0f, amax = 0.0f;
    for (int i = 0; i < 16; i++) {
      if (std::fabs(blk[i]) > amax) { amax = std::fabs(blk[i]); mx = blk[i]; }
    }
    subscale[s] = amax > 0.0f ? mx / -32.0f : 0.0f;
  }
  float max_scale = 0.0f;
  for (int s = 0; s < 16; s++)
    if (std::fabs(subscale[s]) > std::fabs(max_scale)) max_scale = subscale[s];
  float d, idd;
  if (max_scale != 0.0f) {
    d = max_scale / -128.0f;
    idd = -128.0f / max_scale;
  } else {
    d = 0.0f;
    idd = 0.0f;
  }
  int8_t sc[16];
  for (int s = 0; s < 16; s++) sc[s] = (int8_t)clampi(sat_i32(rround(subscale[s] * idd)), -128, 127);
  uint8_t q6[256];
  for (int s = 0; s < 16; s++) {
    float scale = d * (float)sc[s];
    for (int i = 0; i < 16; i++) {
      int idx = s * 16 + i;
      int q = scale != 0.0f ? clampi(sat_i32(rround(sb[idx] / scale)), -32, 31) : 0;
      q6[idx] = (uint8_t)(q + 32);
    }
  }
  uint8_t* ql = dst;
  uint8_t* qh = dst + 128;
  for (int n128 = 0; n128 < 2; n128++) {
    int y0 = n128 * 128, qlb = n128 * 64, qhb = n128 * 32;
    for (int l = 0; l < 32; l++) {
      uint8_t b1 = q6[y0 + l] & 63, b2 = q6[y0 + l + 32] & 63;
      uint8_t b3 = q6[y0 + l + 64] & 63, b4 = q6[y0 + l + 96] & 63;
      ql[qlb + l] = (uint8_t)((b1 & 0xF) | ((b3 & 0xF) << 4));
      ql[qlb + l + 32] = (uint8_t)((b2 & 0xF) | ((b4 & 0xF) << 4));
      qh[qhb + l] = (uint8_t)(((b1 >> 4) & 3) | (((b2 >> 4) & 3) << 2) | (((b3 >> 4) & 3) << 4) |
                              (((b4 >> 4) & 3) << 6));
    }
  }
  for (int s = 0; s < 16; s++) dst[192 + s] = (uint8_t)sc[s];
  uint16_t hd = f32_to_f16(d);
  dst[208] = (uint8_t)(hd & 0xff);
  dst[209] = (uint8_t)(hd >> 8);
}

int quantize(const float* x, size_t n, uint32_t t, uint8_t* out) {
  switch (t) {
    case GGML_Q8_0: {
      if (n % 32) return ORC_E_INVALID;
      // blocks are independent: parallel over blocks keeps every byte identical
#pragma omp parallel for schedule(static)
      for (long long b = 0; b < (long long)(n / 32); b++) {
        std::vector<uint8_t> tmp;
        tmp.reserve(34);
        quantize_q8_0(x + b * 32, 32, tmp);
        std::memcpy(out + b * 34, tmp.data(), 34);
      }
      return 0;
    }
    case GGML_Q4_0:
    case GGML_Q5_0: {
      if (n % 32) return ORC_E_INVALID;
      std::vector<uint8_t> tmp;
      if (t == GGML_Q4_0) quantize_q4_0(x, n, tmp); else quantize_q5_0(x, n, tmp);
      std::memcpy(out, tmp.data(), tmp.size());
      return 0;
    }
    case GGML_Q4_K:
    case GGML_Q5_K: {
      if (n % 256) return ORC_E_INVALID;
      size_t bb = t == GGML_Q4_K ? 144 : 176;
#pragma omp parallel for schedule(static)
      for (long long b = 0; b < (long long)(n / 256); b++)
        quantize_qx_k_block(x + b * 256, t == GGML_Q4_K ? 15 : 31, t == GGML_Q5_K, out + b * bb);
      return 0;
    }
    case GGML_Q6_K: {
      if (n % 256) return ORC_E_INVALID;
#pragma omp parallel for schedule(static)
      for (long long b = 0; b < (long long)(n / 256); b++) quantize_q6_k_block(x + b * 256, out + b * 210);
      return 0;
    }
    case GGML_F32:
      std::memcpy(out, x, n * 4);
      return 0;
    case GGML_F16:
      for (size_t i = 0; i < n; i++) {
        uint16_t h = f32_to_f16(x[i]);
        out[2 * i] = (uint8_t)(h & 0xff);
        out[2 * i + 1] = (uint8_t)(h >> 8);
      }
      return 0;
    default:
      return ORC_E_UNSUPPORTED_QUANT;
  }
}

}  // namespace orc
