// Kernel-facing declarations shared by the .hip translation units.
#pragma once
#include "common.hpp"

namespace hos {

// GGUF type ids (src/gguf.rs). Q4_0 and Q5_0 are repacked exactly into the Q8_0 layout on upload; Q5_K, F16 and
// BF16 matrices keep their own device layouts.
enum : uint32_t {
  GGUF_F32 = 0,
  GGUF_F16 = 1,
  GGUF_Q4_0 = 2,
  GGUF_Q5_0 = 6,
  GGUF_Q8_0 = 8,
  GGUF_Q4_K = 12,
  GGUF_Q5_K = 13,
  GGUF_Q6_K = 14,
  GGUF_BF16 = 30
};

// Plain-old-data view of a QWeight passed to kernels by value.
struct QWeightView {
  uint32_t type;
  long long rows, cols;
  const void* q;
  const float* s;
};
inline QWeightView view(const QWeight& w) { return QWeightView{w.type, w.rows, w.cols, w.q, w.s}; }

// Correctly rounded f32 division and square root (what Rust's f32 `/` and sqrt give): the f64 operation is
// correctly rounded, and rounding its result once more to f32 is exact-safe because 53 >= 2·24 + 2. (HIP's
// __fsqrt_rn is the approximate hardware square root unless OCML rounding mode is enabled.)
// e^d for the row statistics of a softmax folded into the vocabulary head GEMM's epilogue (qgemm_impl.hpp):
// hardware exp2 of d·log2 e (one rounding of the product, ~1 ulp exp2; the exponents that matter are small). The
// cross-entropy pass that consumes those statistics (fused.hip ce_kernel) computes its numerators with the same
// function, so each row's p sums to 1. (expf in the epilogue instead: the step's forward GEMMs 1.3% slower — the
// inlined expf of the statistics branch enlarges every forward instantiation.)
__device__ __forceinline__ float exp_rs(float d) { return __builtin_amdgcn_exp2f(d * 1.4426950408889634f); }
__device__ __forceinline__ float div_rn(float a, float b) { return (float)((double)a / (double)b); }
__device__ __forceinline__ float sqrt_rn(float a) { return (float)__builtin_sqrt((double)a); }

// One dequantized element, bit-identical to Gguf::dequant_into (src/gguf.rs):
//   Q8_0  q·d                 (:354-367)
//   Q4_K  (d·sc)·q − dmin·m   (:385-413; d·sc and dmin·m are precomputed in f32 at repack)
//   Q6_K  (d·sc)·q            (:449-477)
//   Q5_K  (d·sc)·q − dmin·m   (:414-448; q = 5-bit code, one byte per element on the device)
//   F16 / BF16 widened exactly (:342-353)
__device__ __forceinline__ float deq_q8(int8_t q, float d) { return __fmul_rn((float)q, d); }
// (d·sc)·q is exact in f32 (d: 11 significant bits, sc ≤ 63, q ≤ 31 → ≤ 22 bits), so the reference's
// multiply-then-subtract rounds once, at the subtraction — exactly what one fused multiply-add does.
__device__ __forceinline__ float deq_q4k(uint32_t q, float2 dm) { return __builtin_fmaf(dm.x, (float)q, -dm.y); }
__device__ __forceinline__ float deq_q4k_f(float q, float2 dm) { return __builtin_fmaf(dm.x, q, -dm.y); }
__device__ __forceinline__ float deq_q6k(int8_t q, float s) { return __fmul_rn(s, (float)q); }

__device__ __forceinline__ float deq_one(const QWeightView& w, long long r, long long c) {
  long long i = r * w.cols + c;
  if (w.type == GGUF_Q8_0) return deq_q8(((const int8_t*)w.q)[i], w.s[i >> 5]);
  if (w.type == GGUF_Q4_K) {
    uint8_t b = ((const uint8_t*)w.q)[i >> 1];
    uint32_t q = (i & 1) ? (b >> 4) : (b & 15u);
    return deq_q4k(q, ((const float2*)w.s)[i >> 5]);
  }
  if (w.type == GGUF_Q5_K) return deq_q4k((uint32_t)((const uint8_t*)w.q)[i], ((const float2*)w.s)[i >> 5]);
  if (w.type == GGUF_F16) return (float)((const _Float16*)w.q)[i];
  if (w.type == GGUF_BF16) return __uint_as_float((uint32_t)((const uint16_t*)w.q)[i] << 16);
  if (w.type == GGUF_F32) return ((const float*)w.q)[i];
  return deq_q6k(((const int8_t*)w.q)[i], w.s[i >> 4]);
}

// One row (this workgroup's) of f32 -> the fp16 GEMM operand with an exact power-of-two scale putting the row
// max-abs in [2^14, 2^15): out = fp16(x·2^e), lo = fp16(x·2^e − out) (lo may be null), rinv = 2^-e. Every thread
// of the workgroup calls it; it reads only the elements c ≡ threadIdx.x (mod blockDim.x) of xr.
__device__ inline void block_row_h16(const float* xr, int K, _Float16* orow, _Float16* lrow, float* rinv) {
  __shared__ float red[32];
  float amax = 0.0f;
  for (int c = threadIdx.x; c < K; c += blockDim.x) amax = fmaxf(amax, fabsf(xr[c]));
  for (int o = 32; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
  __syncthreads();
  if (threadIdx.x == 0) {
    float a = 0.0f;
    for (int i = 0; i < (int)(blockDim.x >> 6); i++) a = fmaxf(a, red[i]);
    red[0] = a;
  }
  __syncthreads();
  amax = red[0];
  int e = 0;
  if (amax > 0.0f && amax < 3.0e38f) {
    int ex;
    frexpf(amax, &ex);  // amax in [2^(ex-1), 2^ex)
    e = 15 - ex;
    e = e > 100 ? 100 : (e < -100 ? -100 : e);
  }
  const float sc = ldexpf(1.0f, e);
  if (threadIdx.x == 0) *rinv = ldexpf(1.0f, -e);
  for (int c = threadIdx.x; c < K; c += blockDim.x) {
    const float v = xr[c] * sc;
    const _Float16 h = (_Float16)v;
    orow[c] = h;
    if (lrow) lrow[c] = (_Float16)(v - (float)h);
  }
}

// ---- quant.hip ----
size_t gguf_bytes_for(uint32_t t, size_t n);
size_t block_elems(uint32_t t);
// Device layout a GGUF type is kept in (Q4_0 / Q5_0 -> Q8_0, exactly; every other type its own).
uint32_t storage_type(uint32_t t);
void qweight_sizes(uint32_t type, long long rows, long long cols, size_t* q_bytes, size_t* s_bytes);
void repack_weight(const uint8_t* src_dev, uint32_t src_type, QWeight& w, hipStream_t st);
void launch_dequant(const QWeight& w, float* out_dev, hipStream_t st);
void launch_quantize(const float* x_dev, size_t n, uint32_t type, uint8_t* out_dev, hipStream_t st);

// ---- qgemm.hip ----
// Epilogue of the fp16 GEMMs: v = rinv[m]·acc[m][n] (+ bias[n]);
//   accumulate: out += v;  else resid: out = resid + v (resid may alias out);  else out = v.
// Optional rank-r update fused into the epilogue (a LoRA branch): v += scale · Σ_j U[m][j] · L(j, n),
// U row-major with row stride ldu, L(j, n) = L[j·slj + n·sln]. rank 0 = none.
struct GemmEpi {
  float* out;
  long long ldo;
  const float* bias;   // may be null
  int accumulate;      // 1: out += v
  const float* resid;  // may be null; same row stride as out
  const float* U = nullptr;
  long long ldu = 0;
  const float* L = nullptr;
  long long slj = 0, sln = 0;
  int rank = 0;
  float scale = 0.0f;
  // Column segments of a stacked projection (q|k|v, gate|up): output columns n >= ub0 (and >= ub1) take their U
  // block ustep (2·ustep) columns further on — each target's own rank-r factor. 0 = one U for all columns.
  int ustep = 0, ub0 = 0, ub1 = 0;
  // Row statistics of the output for a softmax over each row (forward launches): rstat[row·rstat_ld + col/64] =
  // (max, Σ e^(y − max)) over the 64-column chunk of that row (set: the launch takes unsplit 128-column tiles).
  float2* rstat = nullptr;
  long long rstat_ld = 0;
  // Tile order within each XCD's run of workgroups: 0 = output columns fastest (the tiles that run together share
  // an activation row block), 1 = rows fastest (they share a weight column strip: for outputs many tiles wide,
  // such as the vocabulary head, each strip is then fetched once instead of once per row block).
  int rows_fastest = 0;
  // Deferred reduction (host pointer, may be null): a launch split over the contraction leaves its partials in the
  // workspace, stores the split count here and launches no reduction — the consumer reads the partials (SplitSrc);
  // an unsplit launch writes its output as usual and stores 1.
  int* defer = nullptr;
};
// A row source given as the partials of a split qGEMM whose reduction was deferred to its consumer: row m =
// (Σ_z ws[z·mn + m·n .. ]) · rinv[m] (+ resid[m]), the partials summed in split order and then scaled, exactly as
// splitk_reduce4 forms an unbiased, non-accumulating output. splits = 0: no such source.
struct SplitSrc {
  const float* ws = nullptr;
  int splits = 0;
  long long mn = 0;
  const float* rinv = nullptr;
  const float* resid = nullptr;
};
// The deterministic split-K reduction of a qGEMM's partials into epi.out (what a launch without epi.defer runs).
void launch_qgemm_split_reduce(const float* ws, int splits, long long M, int N, const float* rinv, const GemmEpi& epi,
                               hipStream_t st);
// Grouped (mixture-of-experts) GEMM schedule: W holds n_experts stacked [rows, cols] blocks; workgroup row
// y of the launch computes rows tiles[3y+1] .. +tiles[3y+2] of the operand against expert tiles[3y]
// (−1: nothing to do). Built on the device by the router, so the launch needs no host round trip.
struct GroupSched {
  const int* tiles = nullptr;
  int max_tiles = 0;
  int n_experts = 0;
};
// Row tile height of the grouped GEMMs (the router's schedule is built for it).
constexpr int GROUP_BM = 128;
// out[r] (+)= A[r]·deq(W_e)ᵀ (fwd) or A[r]·deq(W_e) (dx) for the rows r the schedule gives expert e.
void launch_qgemm_grouped(bool dx, const QWeight& w, GroupSched gs, H16 a, long long lda, GemmEpi epi, int passes,
                          hipStream_t st);
// Y[M, W.rows] = A[M, W.cols] · deq(W)ᵀ, A an fp16 row-scaled operand with row stride lda.
void launch_qgemm_fwd(const QWeight& w, H16 a, long long lda, long long M, GemmEpi epi, float* ws, size_t ws_bytes,
                      int passes, hipStream_t st);
// dX[M, W.cols] = dY[M, W.rows] · deq(W), dY an fp16 row-scaled operand with row stride lda.
void launch_qgemm_dx(const QWeight& w, H16 a, long long lda, long long M, GemmEpi epi, float* ws, size_t ws_bytes,
                     int passes, hipStream_t st);
// f32 [M, K] (row stride ldx) -> fp16 row-scaled operand (row stride K); residual too when out.lo is set.
void launch_to_h16(const float* x, long long ldx, long long M, long long K, H16 out, hipStream_t st);
// n samples of N(0, stddev²) from a counter-based hash of (seed, index) (synthetic weights on the device)
void launch_randn(float* out, size_t n, uint64_t seed, float stddev, hipStream_t st);

// ---- gemm_f32.hip ----
// C[M,N] = alpha·Σ_k A(m,k)·B(k,n) + beta·C, A(m,k) = A[m·sam + k·sak], B(k,n) = B[k·sbk + n·sbn].
void launch_gemm_f32(long long M, long long N, long long K, float alpha, const float* A, long long sam,
                     long long sak, const float* B, long long sbk, long long sbn, float beta, float* C, long long ldc,
                     float* ws, size_t ws_bytes, hipStream_t st);

}  // namespace hos
