// Dequant-fused quantized-weight GEMMs on fp16 MFMA (v_mfma_f32_32x32x16_f16, fp32 accumulate).
//
//   fwd: Y[M, N]  = A[M, K] · deq(W)ᵀ   W [N, K]  — the frozen-base forward x·t_const(W)
//   dx : dX[M, K] = dY[M, N] · deq(W)   W [N, K]  — the frozen-base backward g·Bᵀ
//        (src/tensor.rs:316-327 and :347-360; src/peft.rs:24-33 transposes W to [in,out])
//
// Each 32-wide slab of the contraction streams the packed weight from HBM, dequantizes it in
// registers with the bit-exact device functions of kernels.hpp and stores it in LDS in the MFMA
// B-operand layout (contraction-contiguous per output column). The fwd tile is a run of W rows; the
// dx tile is W transposed on the fly (8 rows × 2 columns per thread). The activation operand arrives
// as fp16 with an exact power-of-two scale per row; the epilogue multiplies that scale back out.
//
// Precision passes (NP): one fp16 product rounds both operands to 11 bits (~3e-4 relative per GEMM).
//   NP = 1: A·W                            (fp16 × fp16)
//   NP = 2: A_hi·W + A_lo·W                (activation carried to ~22 bits)
//   NP = 3: A_hi·W_hi + A_lo·W_hi + A_hi·W_lo  (both operands to ~22 bits; dropped A_lo·W_lo ~2^-22)
// where W_hi = fp16(w), W_lo = fp16(w − W_hi) of the f32 dequantized w.
//
// Work decomposition: 256 threads = 4 waves (2×2), workgroup tile BM×BN, wave tile (BM/2)×(BN/2)
// of 32×32 MFMA tiles, double-buffered LDS, optional split-K reduced deterministically.
#include "kernels.hpp"

namespace hos {

namespace {

constexpr int BK = 32;   // contraction slab
constexpr int PADH = 8;  // LDS row padding in halves (row = 80 B)
constexpr int LDSROW = BK + PADH;

template <int BM, int BN>
struct Cfg {
  static constexpr int TM = BM / 64;  // 32×32 tiles per wave along M
  static constexpr int TN = BN / 64;
  static constexpr int A_H8 = BM * BK / 8 / 256;  // h8 vectors of A per thread
};

__device__ __forceinline__ h8 zero_h8() {
  h8 z;
#pragma unroll
  for (int i = 0; i < 8; i++) z[i] = (_Float16)0.0f;
  return z;
}

// Round w to fp16 hi (+ residual lo when SPLIT) into lane i of two h8 vectors.
template <bool SPLIT>
__device__ __forceinline__ void put_v(float w, h8& hv, h8& lv, int i) {
  _Float16 h = (_Float16)w;
  hv[i] = h;
  if constexpr (SPLIT) lv[i] = (_Float16)(w - (float)h);
}

// ---- B-tile loaders. Each thread produces 16 dequantized elements per slab. ----

// fwd: thread -> W row n = n0 + tid/2, contraction cols c0 + 16·(tid&1) .. +16.
struct FwdRaw {
  uint4 q;  // Q8_0/Q6_K: 16 int8; Q4_K: 8 bytes in q.x,q.y
  float2 s;
  bool ok;
};

template <uint32_t QT>
__device__ __forceinline__ void fwd_load(const QWeightView& w, int n0, int c0, int tid, FwdRaw& r) {
  long long n = n0 + (tid >> 1);
  int c = c0 + 16 * (tid & 1);
  r.ok = n < w.rows;
  if (!r.ok) n = w.rows - 1;
  long long e = n * w.cols + c;
  if constexpr (QT == GGUF_Q4_K) {
    uint2 v = *(const uint2*)((const uint8_t*)w.q + (e >> 1));
    r.q.x = v.x;
    r.q.y = v.y;
    r.s = ((const float2*)w.s)[e >> 5];
  } else if constexpr (QT == GGUF_Q8_0) {
    r.q = *(const uint4*)((const int8_t*)w.q + e);
    r.s.x = w.s[e >> 5];
  } else {
    r.q = *(const uint4*)((const int8_t*)w.q + e);
    r.s.x = w.s[e >> 4];
  }
}

template <uint32_t QT, bool SPLIT>
__device__ __forceinline__ void fwd_store(const FwdRaw& r, _Float16* Bs, _Float16* Bl, int tid) {
  h8 v0, v1, l0, l1;
  if (!r.ok) {
    v0 = v1 = l0 = l1 = zero_h8();
  } else if constexpr (QT == GGUF_Q4_K) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      uint32_t b0 = (r.q.x >> (8 * i)) & 0xffu, b1 = (r.q.y >> (8 * i)) & 0xffu;
      put_v<SPLIT>(deq_q4k(b0 & 15u, r.s), v0, l0, 2 * i);
      put_v<SPLIT>(deq_q4k(b0 >> 4, r.s), v0, l0, 2 * i + 1);
      put_v<SPLIT>(deq_q4k(b1 & 15u, r.s), v1, l1, 2 * i);
      put_v<SPLIT>(deq_q4k(b1 >> 4, r.s), v1, l1, 2 * i + 1);
    }
  } else {
    const uint32_t words[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
#pragma unroll
    for (int i = 0; i < 8; i++) {
      int8_t a = (int8_t)((words[i >> 2] >> (8 * (i & 3))) & 0xffu);
      int8_t b = (int8_t)((words[2 + (i >> 2)] >> (8 * (i & 3))) & 0xffu);
      if constexpr (QT == GGUF_Q8_0) {
        put_v<SPLIT>(deq_q8(a, r.s.x), v0, l0, i);
        put_v<SPLIT>(deq_q8(b, r.s.x), v1, l1, i);
      } else {
        put_v<SPLIT>(deq_q6k(a, r.s.x), v0, l0, i);
        put_v<SPLIT>(deq_q6k(b, r.s.x), v1, l1, i);
      }
    }
  }
  int off = (tid >> 1) * LDSROW + 16 * (tid & 1);
  *(h8*)(Bs + off) = v0;
  *(h8*)(Bs + off + 8) = v1;
  if constexpr (SPLIT) {
    *(h8*)(Bl + off) = l0;
    *(h8*)(Bl + off + 8) = l1;
  }
}

// dx: thread -> output cols k0 + 2·(tid&63) (+1), contraction rows n0 + 8·(tid>>6) .. +8.
struct DxRaw {
  uint32_t q[8];  // per row: Q4_K one byte (2 nibbles), Q8_0/Q6_K two int8
  float2 s[8];
  bool ok;
};

template <uint32_t QT>
__device__ __forceinline__ void dx_load(const QWeightView& w, int n0, int k0, int tid, DxRaw& r) {
  int k = k0 + 2 * (tid & 63);
  r.ok = k < w.cols;
  if (!r.ok) k = 0;
  long long nb = n0 + 8 * (tid >> 6);
#pragma unroll
  for (int i = 0; i < 8; i++) {
    long long e = (nb + i) * w.cols + k;
    if constexpr (QT == GGUF_Q4_K) {
      r.q[i] = ((const uint8_t*)w.q)[e >> 1];
      r.s[i] = ((const float2*)w.s)[e >> 5];
    } else if constexpr (QT == GGUF_Q8_0) {
      r.q[i] = *(const uint16_t*)((const int8_t*)w.q + e);
      r.s[i].x = w.s[e >> 5];
    } else {
      r.q[i] = *(const uint16_t*)((const int8_t*)w.q + e);
      r.s[i].x = w.s[e >> 4];
    }
  }
}

template <uint32_t QT, bool SPLIT>
__device__ __forceinline__ void dx_store(const DxRaw& r, _Float16* Bs, _Float16* Bl, int tid) {
  h8 v0, v1, l0, l1;
  if (!r.ok) {
    v0 = v1 = l0 = l1 = zero_h8();
  } else {
#pragma unroll
    for (int i = 0; i < 8; i++) {
      if constexpr (QT == GGUF_Q4_K) {
        put_v<SPLIT>(deq_q4k(r.q[i] & 15u, r.s[i]), v0, l0, i);
        put_v<SPLIT>(deq_q4k((r.q[i] >> 4) & 15u, r.s[i]), v1, l1, i);
      } else if constexpr (QT == GGUF_Q8_0) {
        put_v<SPLIT>(deq_q8((int8_t)(r.q[i] & 0xffu), r.s[i].x), v0, l0, i);
        put_v<SPLIT>(deq_q8((int8_t)(r.q[i] >> 8), r.s[i].x), v1, l1, i);
      } else {
        put_v<SPLIT>(deq_q6k((int8_t)(r.q[i] & 0xffu), r.s[i].x), v0, l0, i);
        put_v<SPLIT>(deq_q6k((int8_t)(r.q[i] >> 8), r.s[i].x), v1, l1, i);
      }
    }
  }
  int col = 2 * (tid & 63), rg = 8 * (tid >> 6);
  *(h8*)(Bs + col * LDSROW + rg) = v0;
  *(h8*)(Bs + (col + 1) * LDSROW + rg) = v1;
  if constexpr (SPLIT) {
    *(h8*)(Bl + col * LDSROW + rg) = l0;
    *(h8*)(Bl + (col + 1) * LDSROW + rg) = l1;
  }
}

// ---- the GEMM ----
// out[m][n] (over n < Nout) = Σ_c A[m][c] · B(n, c); contraction C split over gridDim.z.
template <uint32_t QT, bool DX, int BM, int BN, int NP>
__global__ void __launch_bounds__(256) qgemm_kernel(QWeightView w, const _Float16* __restrict__ A,
                                                    const _Float16* __restrict__ Alo, const float* __restrict__ rinv,
                                                    long long lda, int M, int Nout, int C, int c_per_split,
                                                    GemmEpi epi, float* __restrict__ ws) {
  static_assert(BN == 128, "B loaders assume a 128-wide output tile");
  constexpr bool ALO = NP >= 2, BLO = NP >= 3;
  constexpr int NA = ALO ? 2 : 1, NB = BLO ? 2 : 1;
  using CF = Cfg<BM, BN>;
  // per buffer: NA A tiles then NB B tiles
  constexpr int ATILE = BM * LDSROW, BTILE = BN * LDSROW, BUF = NA * ATILE + NB * BTILE;
  __shared__ __attribute__((aligned(16))) _Float16 smem[2 * BUF];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
  const int cbeg = blockIdx.z * c_per_split;
  const int cend = min(C, cbeg + c_per_split);
  const int nslab = (cend - cbeg) / BK;

  f16v acc[CF::TM][CF::TN];
#pragma unroll
  for (int i = 0; i < CF::TM; i++)
#pragma unroll
    for (int j = 0; j < CF::TN; j++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;

  h8 araw[CF::A_H8], alraw[CF::A_H8];
  using Raw = typename std::conditional<DX, DxRaw, FwdRaw>::type;
  Raw braw;

  auto load_a = [&](int c0) {
#pragma unroll
    for (int v = 0; v < CF::A_H8; v++) {
      int idx = tid + 256 * v;            // h8 index within the BM×BK tile
      int row = idx >> 2, cv = idx & 3;   // 4 h8 per 32-wide row
      int m = m0 + row;
      long long off = (long long)m * lda + c0 + 8 * cv;
      araw[v] = m < M ? *(const h8*)(A + off) : zero_h8();
      if constexpr (ALO) alraw[v] = m < M ? *(const h8*)(Alo + off) : zero_h8();
    }
  };
  auto store_a = [&](_Float16* buf) {
#pragma unroll
    for (int v = 0; v < CF::A_H8; v++) {
      int idx = tid + 256 * v;
      int row = idx >> 2, cv = idx & 3;
      *(h8*)(buf + row * LDSROW + 8 * cv) = araw[v];
      if constexpr (ALO) *(h8*)(buf + ATILE + row * LDSROW + 8 * cv) = alraw[v];
    }
  };
  auto load_b = [&](int c0) {
    if constexpr (DX)
      dx_load<QT>(w, c0, n0, tid, braw);
    else
      fwd_load<QT>(w, n0, c0, tid, braw);
  };
  auto store_b = [&](_Float16* buf) {
    _Float16* bs = buf + NA * ATILE;
    if constexpr (DX)
      dx_store<QT, BLO>(braw, bs, bs + BTILE, tid);
    else
      fwd_store<QT, BLO>(braw, bs, bs + BTILE, tid);
  };

  if (nslab > 0) {
    load_a(cbeg);
    load_b(cbeg);
    store_a(smem);
    store_b(smem);
  }
  __syncthreads();

  for (int s = 0; s < nslab; s++) {
    const int buf = s & 1;
    const bool more = s + 1 < nslab;
    if (more) {
      load_a(cbeg + (s + 1) * BK);
      load_b(cbeg + (s + 1) * BK);
    }
    const _Float16* as = smem + buf * BUF;
    const _Float16* bs = as + NA * ATILE;
#pragma unroll
    for (int kk = 0; kk < BK; kk += 16) {
      h8 af[CF::TM], afl[CF::TM], bf[CF::TN], bfl[CF::TN];
      const int koff = kk + 8 * (lane >> 5);
#pragma unroll
      for (int i = 0; i < CF::TM; i++) {
        int ro = (wm * (BM / 2) + 32 * i + (lane & 31)) * LDSROW + koff;
        af[i] = *(const h8*)(as + ro);
        if constexpr (ALO) afl[i] = *(const h8*)(as + ATILE + ro);
      }
#pragma unroll
      for (int j = 0; j < CF::TN; j++) {
        int ro = (wn * (BN / 2) + 32 * j + (lane & 31)) * LDSROW + koff;
        bf[j] = *(const h8*)(bs + ro);
        if constexpr (BLO) bfl[j] = *(const h8*)(bs + BTILE + ro);
      }
#pragma unroll
      for (int i = 0; i < CF::TM; i++)
#pragma unroll
        for (int j = 0; j < CF::TN; j++) {
          if constexpr (BLO) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bfl[j], acc[i][j], 0, 0, 0);
          if constexpr (ALO) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(afl[i], bf[j], acc[i][j], 0, 0, 0);
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
    }
    if (more) {
      store_a(smem + (buf ^ 1) * BUF);
      store_b(smem + (buf ^ 1) * BUF);
    }
    __syncthreads();
  }

  // epilogue: D[i][j] of a 32×32 tile lives at lane j + 32·((i/4)&1), register (i&3) + 4·(i/8)
  const bool split = gridDim.z > 1;
#pragma unroll
  for (int i = 0; i < CF::TM; i++)
#pragma unroll
    for (int j = 0; j < CF::TN; j++) {
      int col = n0 + wn * (BN / 2) + 32 * j + (lane & 31);
      if (col >= Nout) continue;
#pragma unroll
      for (int r = 0; r < 16; r++) {
        int row = m0 + wm * (BM / 2) + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (row >= M) continue;
        float v = acc[i][j][r];
        if (split) {
          ws[((long long)blockIdx.z * M + row) * Nout + col] = v;
        } else {
          v *= rinv[row];
          if (epi.bias) v += epi.bias[col];
          long long off = (long long)row * epi.ldo + col;
          float* o = epi.out + off;
          *o = epi.accumulate ? *o + v : (epi.resid ? epi.resid[off] + v : v);
        }
      }
    }
}

// Deterministic split-K reduction + the same epilogue.
__global__ void splitk_reduce(const float* __restrict__ ws, int splits, int M, int N, const float* __restrict__ rinv,
                              GemmEpi epi) {
  long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long long)M * N) return;
  int row = (int)(i / N), col = (int)(i % N);
  float v = 0.0f;
  for (int z = 0; z < splits; z++) v += ws[(long long)z * M * N + i];
  v *= rinv[row];
  if (epi.bias) v += epi.bias[col];
  long long off = (long long)row * epi.ldo + col;
  float* o = epi.out + off;
  *o = epi.accumulate ? *o + v : (epi.resid ? epi.resid[off] + v : v);
}

// f32 rows -> fp16 (+ residual) with a power-of-two row scale putting the row max-abs in [2^14, 2^15).
__global__ void to_h16_kernel(const float* __restrict__ x, long long ldx, int K, _Float16* __restrict__ out,
                              _Float16* __restrict__ lo, float* __restrict__ rinv) {
  const int row = blockIdx.x;
  const float* xr = x + (long long)row * ldx;
  float amax = 0.0f;
  for (int c = threadIdx.x; c < K; c += blockDim.x) amax = fmaxf(amax, fabsf(xr[c]));
  __shared__ float red[32];
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
  float sc = ldexpf(1.0f, e);
  if (threadIdx.x == 0) rinv[row] = ldexpf(1.0f, -e);
  _Float16* orow = out + (long long)row * K;
  _Float16* lrow = lo ? lo + (long long)row * K : nullptr;
  for (int c = threadIdx.x; c < K; c += blockDim.x) {
    float v = xr[c] * sc;
    _Float16 h = (_Float16)v;
    orow[c] = h;
    if (lrow) lrow[c] = (_Float16)(v - (float)h);
  }
}

template <uint32_t QT, bool DX, int NP>
void launch_typed(const QWeight& w, H16 a, long long lda, long long M, GemmEpi epi, float* ws, size_t ws_bytes,
                  hipStream_t st) {
  const int Nout = DX ? (int)w.cols : (int)w.rows;
  const int C = DX ? (int)w.rows : (int)w.cols;
  HOS_REQUIRE(C % BK == 0, HOS_E_INVALID, "qgemm: contraction length must be a multiple of 32");
  HOS_REQUIRE((lda % 8) == 0, HOS_E_INVALID, "qgemm: activation row stride must be a multiple of 8");
  HOS_REQUIRE(NP == 1 || a.lo != nullptr, HOS_E_INVALID, "qgemm: multi-pass precision needs the operand residual");
  constexpr int BM = 128, BN = 128;
  int tiles = ceil_div(M, BM) * ceil_div(Nout, BN);
  int nslab = C / BK;
  int splits = 1;
  // fill the 256 CUs: split the contraction while the grid is small and slabs remain
  while (tiles * splits < 512 && nslab / (splits * 2) >= 4 &&
         (size_t)(splits * 2) * M * Nout * sizeof(float) <= ws_bytes)
    splits *= 2;
  int per = ceil_div(nslab, splits) * BK;
  splits = ceil_div(C, per);
  dim3 grid(ceil_div(Nout, BN), ceil_div(M, BM), splits);
  qgemm_kernel<QT, DX, BM, BN, NP>
      <<<grid, 256, 0, st>>>(view(w), a.data, a.lo, a.rinv, lda, (int)M, Nout, C, per, epi, ws);
  HOS_HIP_CHECK(hipGetLastError());
  if (splits > 1) {
    long long n = M * (long long)Nout;
    splitk_reduce<<<ceil_div(n, 256), 256, 0, st>>>(ws, splits, (int)M, Nout, a.rinv, epi);
    HOS_HIP_CHECK(hipGetLastError());
  }
}

template <bool DX, int NP>
void launch_np(const QWeight& w, H16 a, long long lda, long long M, GemmEpi epi, float* ws, size_t ws_bytes,
               hipStream_t st) {
  switch (w.type) {
    case GGUF_Q8_0: launch_typed<GGUF_Q8_0, DX, NP>(w, a, lda, M, epi, ws, ws_bytes, st); break;
    case GGUF_Q4_K: launch_typed<GGUF_Q4_K, DX, NP>(w, a, lda, M, epi, ws, ws_bytes, st); break;
    case GGUF_Q6_K: launch_typed<GGUF_Q6_K, DX, NP>(w, a, lda, M, epi, ws, ws_bytes, st); break;
    default: throw Error(HOS_E_UNSUPPORTED_QUANT, "qgemm: unsupported quant type");
  }
}

template <bool DX>
void launch_any(const QWeight& w, H16 a, long long lda, long long M, GemmEpi epi, float* ws, size_t ws_bytes,
                int passes, hipStream_t st) {
  if (M <= 0) return;
  switch (passes) {
    case 1: launch_np<DX, 1>(w, a, lda, M, epi, ws, ws_bytes, st); break;
    case 2: launch_np<DX, 2>(w, a, lda, M, epi, ws, ws_bytes, st); break;
    case 3: launch_np<DX, 3>(w, a, lda, M, epi, ws, ws_bytes, st); break;
    default: throw Error(HOS_E_INVALID, "qgemm: precision passes must be 1, 2 or 3");
  }
}

}  // namespace

void launch_qgemm_fwd(const QWeight& w, H16 a, long long lda, long long M, GemmEpi epi, float* ws, size_t ws_bytes,
                      int passes, hipStream_t st) {
  launch_any<false>(w, a, lda, M, epi, ws, ws_bytes, passes, st);
}
void launch_qgemm_dx(const QWeight& w, H16 a, long long lda, long long M, GemmEpi epi, float* ws, size_t ws_bytes,
                     int passes, hipStream_t st) {
  launch_any<true>(w, a, lda, M, epi, ws, ws_bytes, passes, st);
}
void launch_to_h16(const float* x, long long ldx, long long M, long long K, H16 out, hipStream_t st) {
  if (M <= 0) return;
  to_h16_kernel<<<(unsigned)M, 256, 0, st>>>(x, ldx, (int)K, out.data, out.lo, out.rinv);
  HOS_HIP_CHECK(hipGetLastError());
}

}  // namespace hos
