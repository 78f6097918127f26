// Shared definitions for the MI355X (gfx950) LoRA fine-tune backend.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <stdexcept>
#include <string>

#include "../../include/hos_hip.h"

namespace hos {

typedef _Float16 half_t;
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f16v __attribute__((ext_vector_type(16)));
typedef float f4v __attribute__((ext_vector_type(4)));
typedef __bf16 bf8 __attribute__((ext_vector_type(8)));

// bf16 hi/lo split: x = hi + lo with hi = bf16(x) and lo = bf16(x − hi) (x − hi is exact in f32).
__device__ __forceinline__ void split_bf(float x, bf8& H, bf8& L, int i) {
  const __bf16 h = (__bf16)x;
  H[i] = h;
  L[i] = (__bf16)(x - (float)h);
}
// a·b ≈ a_hi·b_hi + a_hi·b_lo + a_lo·b_hi on v_mfma_f32_32x32x16_bf16: ~2^-16 relative, fp32 range.
__device__ __forceinline__ f16v mma3_bf16(const bf8& ah, const bf8& al, const bf8& bh, const bf8& bl, f16v c) {
  c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al, bh, c, 0, 0, 0);
  c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, bl, c, 0, 0, 0);
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, bh, c, 0, 0, 0);
}

// Two independent three-product updates with their passes interleaved, so consecutive MFMAs never depend on each
// other; each accumulator receives the same products in the same order as two mma3_bf16 calls.
__device__ __forceinline__ void mma3_bf16_x2(const bf8& ah0, const bf8& al0, const bf8& bh0, const bf8& bl0, f16v& c0,
                                             const bf8& ah1, const bf8& al1, const bf8& bh1, const bf8& bl1, f16v& c1) {
  c0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al0, bh0, c0, 0, 0, 0);
  c1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al1, bh1, c1, 0, 0, 0);
  c0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah0, bl0, c0, 0, 0, 0);
  c1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah1, bl1, c1, 0, 0, 0);
  c0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah0, bh0, c0, 0, 0, 0);
  c1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah1, bh1, c1, 0, 0, 0);
}

// Host-side error carrying a HOS_E_* status code across the C ABI.
struct Error : std::runtime_error {
  int code;
  Error(int c, const std::string& m) : std::runtime_error(m), code(c) {}
};

#define HOS_HIP_CHECK(expr)                                                                     \
  do {                                                                                          \
    hipError_t e_ = (expr);                                                                     \
    if (e_ != hipSuccess)                                                                       \
      throw ::hos::Error(HOS_E_DEVICE, std::string(#expr) + ": " + hipGetErrorString(e_));      \
  } while (0)

#define HOS_REQUIRE(cond, code, msg)                \
  do {                                              \
    if (!(cond)) throw ::hos::Error((code), (msg)); \
  } while (0)

inline int ceil_div(long long a, long long b) { return (int)((a + b - 1) / b); }

// Device-resident repacked quantized weight (see quant.hip). rows = N (out), cols = K (in).
//   Q8_0: q = int8 [N][K],     s = f32 d              per (row, 32 cols)
//   Q4_K: q = u8   [N][K/2]    (col 2i low nibble, 2i+1 high), s = f32 {d·sc, dmin·m} per (row, 32)
//   Q6_K: q = int8 [N][K],     s = f32 d·sc           per (row, 16 cols)
struct QWeight {
  uint32_t type = 0;
  int64_t rows = 0, cols = 0;
  void* q = nullptr;
  float* s = nullptr;
  size_t q_bytes = 0, s_bytes = 0;
};

// An fp16 GEMM operand with an exact power-of-two scale per row:
//   data[m][k] = fp16(x[m][k] · 2^e[m]),  rinv[m] = 2^-e[m],
//   lo[m][k]   = fp16(x[m][k] · 2^e[m] − data[m][k])  (the rounding residual; null when not kept).
// data + lo carries x to ~22 bits, which the multi-pass GEMMs use.
struct H16 {
  half_t* data;
  float* rinv;
  half_t* lo = nullptr;
};
inline H16 h16_offset(H16 a, long long cols) {
  return H16{a.data + cols, a.rinv, a.lo ? a.lo + cols : nullptr};
}

}  // namespace hos
