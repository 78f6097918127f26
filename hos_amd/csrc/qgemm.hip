// Dequant-fused quantized-weight GEMMs on fp16 MFMA (v_mfma_f32_32x32x16_f16, fp32 accumulate): the launchers and
// the fp16 operand conversion; the kernel templates and the tile rule are in qgemm_impl.hpp, instantiated per weight
// layout in qgemm_{q8,q4k,q5k,q6k,f16,bf16,f32}.hip.
//
//   fwd: Y[M, N]  = A[M, K] · deq(W)ᵀ   W [N, K]  — the frozen-base forward x·t_const(W)
//   dx : dX[M, K] = dY[M, N] · deq(W)   W [N, K]  — the frozen-base backward g·Bᵀ
//        (src/tensor.rs:316-327 and :347-360; src/peft.rs:24-33 transposes W to [in,out])
//
// The activation operand arrives as fp16 with an exact power-of-two scale per row (to_h16 below, or the row kernel
// that produced it); the epilogue multiplies that scale back out. Precision modes 1-5 are described in
// qgemm_impl.hpp.
#include "kernels.hpp"

namespace hos {


void qgemm_launch_q8(bool dx, int passes, const QWeight& w, H16 a, long long lda, long long M, GemmEpi epi,
                      float* ws, size_t ws_bytes, hipStream_t st);
void qgemm_grouped_q8(bool dx, int passes, const QWeight& w, GroupSched gs, H16 a, long long lda, GemmEpi epi,
                       hipStream_t st);
void qgemm_launch_q4k(bool dx, int passes, const QWeight& w, H16 a, long long lda, long long M, GemmEpi epi,
                      float* ws, size_t ws_bytes, hipStream_t st);
void qgemm_grouped_q4k(bool dx, int passes, const QWeight& w, GroupSched gs, H16 a, long long lda, GemmEpi epi,
                       hipStream_t st);
void qgemm_launch_q6k(bool dx, int passes, const QWeight& w, H16 a, long long lda, long long M, GemmEpi epi,
                      float* ws, size_t ws_bytes, hipStream_t st);
void qgemm_grouped_q6k(bool dx, int passes, const QWeight& w, GroupSched gs, H16 a, long long lda, GemmEpi epi,
                       hipStream_t st);
void qgemm_launch_q5k(bool dx, int passes, const QWeight& w, H16 a, long long lda, long long M, GemmEpi epi,
                      float* ws, size_t ws_bytes, hipStream_t st);
void qgemm_grouped_q5k(bool dx, int passes, const QWeight& w, GroupSched gs, H16 a, long long lda, GemmEpi epi,
                       hipStream_t st);
void qgemm_launch_f16(bool dx, int passes, const QWeight& w, H16 a, long long lda, long long M, GemmEpi epi,
                      float* ws, size_t ws_bytes, hipStream_t st);
void qgemm_grouped_f16(bool dx, int passes, const QWeight& w, GroupSched gs, H16 a, long long lda, GemmEpi epi,
                       hipStream_t st);
void qgemm_launch_bf16(bool dx, int passes, const QWeight& w, H16 a, long long lda, long long M, GemmEpi epi,
                      float* ws, size_t ws_bytes, hipStream_t st);
void qgemm_grouped_bf16(bool dx, int passes, const QWeight& w, GroupSched gs, H16 a, long long lda, GemmEpi epi,
                       hipStream_t st);
void qgemm_launch_f32(bool dx, int passes, const QWeight& w, H16 a, long long lda, long long M, GemmEpi epi,
                      float* ws, size_t ws_bytes, hipStream_t st);
void qgemm_grouped_f32(bool dx, int passes, const QWeight& w, GroupSched gs, H16 a, long long lda, GemmEpi epi,
                       hipStream_t st);

namespace {

// f32 rows -> fp16 (+ residual) with a power-of-two row scale putting the row max-abs in [2^14, 2^15).
__global__ void to_h16_kernel(const float* __restrict__ x, long long ldx, int K, _Float16* __restrict__ out,
                              _Float16* __restrict__ lo, float* __restrict__ rinv) {
  const int row = blockIdx.x;
  block_row_h16(x + (long long)row * ldx, K, out + (long long)row * K, lo ? lo + (long long)row * K : nullptr,
                rinv + row);
}

// The same conversion with the row held in registers (K % 4 == 0, K <= 8192, 16-byte aligned rows, 8-byte
// aligned outputs): one read of the row; the same scale and per-element rounding as block_row_h16.
typedef _Float16 h16x4_t __attribute__((ext_vector_type(4)));
__global__ void __launch_bounds__(256) to_h16_reg_kernel(const float* __restrict__ x, long long ldx, int K,
                                                         _Float16* __restrict__ out, _Float16* __restrict__ lo,
                                                         float* __restrict__ rinv) {
  constexpr int NV = 8;
  __shared__ float red[4];
  const int row = blockIdx.x, K4 = K >> 2;
  const float4* xr = reinterpret_cast<const float4*>(x + (long long)row * ldx);
  float4 v[NV];
  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < NV; j++) {
    const int i = threadIdx.x + 256 * j;
    if (i < K4) {
      v[j] = xr[i];
      amax = fmaxf(fmaxf(amax, fmaxf(fabsf(v[j].x), fabsf(v[j].y))), fmaxf(fabsf(v[j].z), fabsf(v[j].w)));
    }
  }
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
  if (threadIdx.x == 0) rinv[row] = ldexpf(1.0f, -e);
#pragma unroll
  for (int j = 0; j < NV; j++) {
    const int i = threadIdx.x + 256 * j;
    if (i < K4) {
      const float a = v[j].x * sc, b = v[j].y * sc, c = v[j].z * sc, d = v[j].w * sc;
      const h16x4_t h{(_Float16)a, (_Float16)b, (_Float16)c, (_Float16)d};
      *reinterpret_cast<h16x4_t*>(out + (long long)row * K + 4 * i) = h;
      if (lo) {
        const h16x4_t l{(_Float16)(a - (float)h.x), (_Float16)(b - (float)h.y), (_Float16)(c - (float)h.z),
                        (_Float16)(d - (float)h.w)};
        *reinterpret_cast<h16x4_t*>(lo + (long long)row * K + 4 * i) = l;
      }
    }
  }
}

void launch_any(bool dx, const QWeight& w, H16 a, long long lda, long long M, GemmEpi epi, float* ws,
                size_t ws_bytes, int passes, hipStream_t st) {
  if (M <= 0) return;
  HOS_REQUIRE(passes >= 1 && passes <= 5, HOS_E_INVALID, "qgemm: precision mode must be 1 to 5");
  switch (w.type) {
    case GGUF_Q8_0: qgemm_launch_q8(dx, passes, w, a, lda, M, epi, ws, ws_bytes, st); break;
    case GGUF_Q4_K: qgemm_launch_q4k(dx, passes, w, a, lda, M, epi, ws, ws_bytes, st); break;
    case GGUF_Q6_K: qgemm_launch_q6k(dx, passes, w, a, lda, M, epi, ws, ws_bytes, st); break;
    case GGUF_Q5_K: qgemm_launch_q5k(dx, passes, w, a, lda, M, epi, ws, ws_bytes, st); break;
    case GGUF_F16: qgemm_launch_f16(dx, passes, w, a, lda, M, epi, ws, ws_bytes, st); break;
    case GGUF_BF16: qgemm_launch_bf16(dx, passes, w, a, lda, M, epi, ws, ws_bytes, st); break;
    case GGUF_F32: qgemm_launch_f32(dx, passes, w, a, lda, M, epi, ws, ws_bytes, st); break;
    default: throw Error(HOS_E_UNSUPPORTED_QUANT, "qgemm: unsupported quant type");
  }
}

}  // namespace

void launch_qgemm_fwd(const QWeight& w, H16 a, long long lda, long long M, GemmEpi epi, float* ws, size_t ws_bytes,
                      int passes, hipStream_t st) {
  launch_any(false, w, a, lda, M, epi, ws, ws_bytes, passes, st);
}
void launch_qgemm_dx(const QWeight& w, H16 a, long long lda, long long M, GemmEpi epi, float* ws, size_t ws_bytes,
                     int passes, hipStream_t st) {
  launch_any(true, w, a, lda, M, epi, ws, ws_bytes, passes, st);
}
void launch_qgemm_grouped(bool dx, const QWeight& w, GroupSched gs, H16 a, long long lda, GemmEpi epi, int passes,
                          hipStream_t st) {
  HOS_REQUIRE(passes >= 1 && passes <= 5, HOS_E_INVALID, "qgemm: precision mode must be 1 to 5");
  if (gs.max_tiles <= 0) return;
  switch (w.type) {
    case GGUF_Q8_0: qgemm_grouped_q8(dx, passes, w, gs, a, lda, epi, st); break;
    case GGUF_Q4_K: qgemm_grouped_q4k(dx, passes, w, gs, a, lda, epi, st); break;
    case GGUF_Q6_K: qgemm_grouped_q6k(dx, passes, w, gs, a, lda, epi, st); break;
    case GGUF_Q5_K: qgemm_grouped_q5k(dx, passes, w, gs, a, lda, epi, st); break;
    case GGUF_F16: qgemm_grouped_f16(dx, passes, w, gs, a, lda, epi, st); break;
    case GGUF_BF16: qgemm_grouped_bf16(dx, passes, w, gs, a, lda, epi, st); break;
    case GGUF_F32: qgemm_grouped_f32(dx, passes, w, gs, a, lda, epi, st); break;
    default: throw Error(HOS_E_UNSUPPORTED_QUANT, "qgemm: unsupported quant type");
  }
}
void launch_to_h16(const float* x, long long ldx, long long M, long long K, H16 out, hipStream_t st) {
  if (M <= 0) return;
  auto al = [](const void* p, uintptr_t n) { return ((uintptr_t)p % n) == 0; };
  if (K % 4 == 0 && K <= 8192 && ldx % 4 == 0 && al(x, 16) && al(out.data, 8) && al(out.lo, 8))
    to_h16_reg_kernel<<<(unsigned)M, 256, 0, st>>>(x, ldx, (int)K, out.data, out.lo, out.rinv);
  else
    to_h16_kernel<<<(unsigned)M, 256, 0, st>>>(x, ldx, (int)K, out.data, out.lo, out.rinv);
  HOS_HIP_CHECK(hipGetLastError());
}

}  // namespace hos
