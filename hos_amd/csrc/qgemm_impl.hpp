// Dequant-fused quantized-weight GEMM kernel templates on fp16 MFMA (v_mfma_f32_32x32x16_f16, fp32
// accumulate); instantiated per quant type in qgemm_q8 / qgemm_q4k / qgemm_q6k.
//
//   fwd: Y[M, N]  = A[M, K] · deq(W)ᵀ   W [N, K]  — the frozen-base forward x·t_const(W)
//   dx : dX[M, K] = dY[M, N] · deq(W)   W [N, K]  — the frozen-base backward g·Bᵀ
//        (src/tensor.rs:316-327 and :347-360; src/peft.rs:24-33 transposes W to [in,out])
//
// Each BK-deep slab of the contraction streams the packed weight from HBM, dequantizes it in registers to
// the same f32 values as the device functions of kernels.hpp (run_store: codes as fp16 subnormals into
// mixed-precision fmas, or packed fp16 for Q8_0) and stores it row-major in LDS exactly as the rows
// arrive (a run of E consecutive values per thread, one coalesced load, one vector LDS store):
//   fwd: W rows are output columns, runs go along the contraction → B fragments are plain 128-bit reads;
//   dx:  W rows are the contraction, runs go along the output → B fragments are read transposed with
//        ds_read_b64_tr_b16 (in a 16-lane group, lane L addressing row cb + L/4, columns jb + 4·(L%4) .. +3
//        hands lane i the rows cb .. cb+3 of column jb + i; two reads give the 8-deep run an MFMA lane needs).
// The activation operand arrives as fp16 with an exact power-of-two scale per row; the epilogue
// multiplies that scale back out and applies bias / residual / a fused rank-r (LoRA) update.
//
// Precision passes (NP): one fp16 product rounds both operands to 11 bits (~3e-4 relative per GEMM).
//   NP = 1: A·W
//   NP = 2: A_hi·W + A_lo·W                       (activation carried to ~22 bits)
//   NP = 3: A_hi·W_hi + A_lo·W_hi + A_hi·W_lo     (both operands to ~22 bits; dropped A_lo·W_lo ~2^-22)
//   NP = 4: A·W_hi + A·W_lo                       (weight to ~22 bits, activation rounded once)
//   NP = 5: Σ_b s_b·(A_hi·Q_b + A_lo·Q_b)         (forward, Q8_0 layout: the weight exact)
// where W_hi = fp16(w), W_lo = fp16(w − W_hi) of the f32 dequantized w. In mode 5 the B operand is the integer
// code q itself (|q| ≤ 128: exact in fp16), each 32-deep block of the contraction is accumulated on its own and
// added into the output accumulator times its scale d (f32 fma, per output column): w = d·q exactly, so the
// result carries only the activation's ~2^-22 and the fp32 accumulation — the precision of mode 3 from two
// products instead of three.
//
// Work decomposition: 4 waves (2×2), or 8 (4×2) for 256-row tiles; workgroup tile BM×BN, wave tile 64×(BN/2) of
// 32×32 MFMA tiles, LDS double-buffered when both stages fit in 64 KB, register prefetch of the next slab,
// optional split-K reduced deterministically by splitk_reduce.
#pragma once
#include <cstdio>
#include <cstdlib>

#include "kernels.hpp"


namespace hos {
namespace {

typedef short s4v __attribute__((ext_vector_type(4)));


// (exp_rs, the e^x of the softmax statistics folded in the epilogue, is in kernels.hpp: the cross-entropy pass
// that consumes them uses it too.)

// Bytes per element of a device weight layout (Q4_K: two per byte).
template <uint32_t QT>
constexpr int elem_bytes() {
  return QT == GGUF_F32 ? 4 : ((QT == GGUF_F16 || QT == GGUF_BF16) ? 2 : 1);
}

// A run of E consecutive values of one W row (E ∈ {8, 16, 32}; it never leaves a 32-value Q8_0/Q4_K group;
// Q6_K's 16-value groups give a second scale for E = 32).
template <uint32_t QT, int E>
struct Run {
  static constexpr int VPW = QT == GGUF_Q4_K ? 8 : 4 / elem_bytes<QT>();  // values per 32-bit word
  static constexpr int NW = E / VPW;
  uint32_t q[NW];
  float2 s[2];
  bool ok;
};

// Where the run starting at element e (row-major over W) lives: its byte offset in q and its float offset in s.
// Both are linear in e, so a run's address splits into a per-thread part and a slab part (e a multiple of 32 there).
template <uint32_t QT>
__device__ __forceinline__ long long run_qoff(long long e) {
  return QT == GGUF_Q4_K ? (e >> 1) : e * elem_bytes<QT>();
}
template <uint32_t QT>
__device__ __forceinline__ long long run_soff(long long e) {
  if constexpr (QT == GGUF_Q4_K || QT == GGUF_Q5_K) return 2 * (e >> 5);  // a float2 per 32 values
  else if constexpr (QT == GGUF_Q8_0) return e >> 5;
  else if constexpr (QT == GGUF_Q6_K) return e >> 4;
  else return 0;  // unscaled types
}

// Load the run at q bytes qp and scales sp (as run_qoff / run_soff place them).
template <uint32_t QT, int E>
__device__ __forceinline__ void run_load(const uint8_t* qp, const float* sp, Run<QT, E>& r) {
  r.ok = true;
  const uint32_t* src = (const uint32_t*)qp;
  if constexpr (Run<QT, E>::NW == 1) {
    r.q[0] = src[0];
  } else if constexpr (Run<QT, E>::NW == 2) {
    uint2 v = *(const uint2*)src;
    r.q[0] = v.x;
    r.q[1] = v.y;
  } else {
#pragma unroll
    for (int i = 0; i < Run<QT, E>::NW; i += 4) {
      uint4 v = *(const uint4*)(src + i);
      r.q[i] = v.x;
      r.q[i + 1] = v.y;
      r.q[i + 2] = v.z;
      r.q[i + 3] = v.w;
    }
  }
  if constexpr (QT == GGUF_Q4_K || QT == GGUF_Q5_K) {
    r.s[0] = *(const float2*)sp;
  } else if constexpr (QT == GGUF_F16 || QT == GGUF_BF16 || QT == GGUF_F32) {
    // unscaled: the stored value is the weight
  } else if constexpr (QT == GGUF_Q8_0) {
    r.s[0].x = sp[0];
  } else {
    r.s[0].x = sp[0];
    if constexpr (E > 16) r.s[1].x = sp[1];
  }
}

// Dequantize a run and store it as E/8 h8 vectors at dst (hi) and dst + lo_off (lo, when SPLIT).
template <uint32_t QT, int E, bool SPLIT, bool CODES = false>
__device__ __forceinline__ void run_store(const Run<QT, E>& r, _Float16* dst, int lo_off) {
  static_assert(!CODES || (QT == GGUF_Q8_0 && !SPLIT), "integer codes: Q8_0 layout, one plane");
#pragma unroll
  for (int v = 0; v < E / 8; v++) {
    // (a run clamped past the last output column only feeds columns that are never stored)
    h8 hv, lv;
    if constexpr (QT == GGUF_Q8_0) {
      // q is an exact fp16 integer and d came from an fp16 field, so in packed fp16 arithmetic
      // hi = q·d rounds the exact product once (= fp16 of the exact f32 dequantized value) and
      // lo = fma(q, d, −hi) is the exact remainder: the same hi/lo as the f32 route, in ~2 ops/element.
      const _Float16 dh = (_Float16)r.s[0].x;
      const h2 d2 = {dh, dh};
      const h2 bias = {(_Float16)1152.0f, (_Float16)1152.0f};
#pragma unroll
      for (int wv = 0; wv < 2; wv++) {
        const uint32_t u = r.q[2 * v + wv] ^ 0x80808080u;  // bytes q + 128
        // 0x6400 | b is the fp16 1024 + b; minus 1152 gives q exactly
        const uint32_t p0 = (u & 0xFFu) | ((u & 0xFF00u) << 8) | 0x64006400u;
        const uint32_t p1 = ((u >> 16) & 0xFFu) | ((u >> 8) & 0xFF0000u) | 0x64006400u;
        h2 x0, x1;
        __builtin_memcpy(&x0, &p0, 4);
        __builtin_memcpy(&x1, &p1, 4);
        x0 -= bias;
        x1 -= bias;
        if constexpr (CODES) {  // the codes themselves; the block scale is applied to the accumulator
          hv[4 * wv] = x0[0];
          hv[4 * wv + 1] = x0[1];
          hv[4 * wv + 2] = x1[0];
          hv[4 * wv + 3] = x1[1];
          continue;
        }
        const h2 h0 = x0 * d2, h1 = x1 * d2;
        hv[4 * wv] = h0[0];
        hv[4 * wv + 1] = h0[1];
        hv[4 * wv + 2] = h1[0];
        hv[4 * wv + 3] = h1[1];
        if constexpr (SPLIT) {
          const h2 l0 = __builtin_elementwise_fma(x0, d2, -h0), l1 = __builtin_elementwise_fma(x1, d2, -h1);
          lv[4 * wv] = l0[0];
          lv[4 * wv + 1] = l0[1];
          lv[4 * wv + 2] = l1[0];
          lv[4 * wv + 3] = l1[1];
        }
      }
    } else if constexpr (QT == GGUF_F16) {
      // the stored halves are the weight: hi is exact and lo is zero
      __builtin_memcpy(&hv, &r.q[4 * v], 16);
      if constexpr (SPLIT) {
#pragma unroll
        for (int i = 0; i < 8; i++) lv[i] = (_Float16)0.0f;
      }
    } else {
      float f[8];
      if constexpr (QT == GGUF_BF16) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
          f[2 * i] = __uint_as_float(r.q[4 * v + i] << 16);
          f[2 * i + 1] = __uint_as_float(r.q[4 * v + i] & 0xffff0000u);
        }
      } else if constexpr (QT == GGUF_F32) {
#pragma unroll
        for (int i = 0; i < 8; i++) f[i] = __uint_as_float(r.q[8 * v + i]);
      } else {
        const float2 sc = (QT == GGUF_Q6_K && v >= 2) ? r.s[1] : r.s[0];
        if constexpr (QT == GGUF_Q4_K) {
          // Value j of the word sits in bits 4j..4j+3. Masked into the low bits of an fp16 half, a code q is
          // the subnormal q·2^-24 (exact), and (float) of it is exact too, so with d' = d·2^24 (exact)
          // fma(d', q·2^-24, -m) rounds the same real number as fma(d, q, -m): the identical f32 value,
          // from one mixed-precision fma per value and four masks per eight.
          const uint32_t w = r.q[v];
          const float dd = sc.x * 16777216.0f;
#pragma unroll
          for (int j = 0; j < 4; j++) {
            const uint32_t p = (w >> (4 * j)) & 0x000F000Fu;
            h2 x;
            __builtin_memcpy(&x, &p, 4);
            f[j] = __builtin_fmaf(dd, (float)x[0], -sc.y);
            f[j + 4] = __builtin_fmaf(dd, (float)x[1], -sc.y);
          }
        } else {
          // Byte codes, the same way: Q5_K's 0..31 with fma(d', q·2^-24, -m); Q6_K's signed q (-32..31) as
          // u = q + 32 = (byte ^ 0x20) & 0x3F with fma(d', u·2^-24, -32·d), which rounds the real d·q once,
          // as d·q itself does (-32·d is exact).
          const float dd = sc.x * 16777216.0f;
          const float c = QT == GGUF_Q5_K ? -sc.y : -32.0f * sc.x;
#pragma unroll
          for (int wv = 0; wv < 2; wv++) {
            uint32_t w = r.q[2 * v + wv];
            if constexpr (QT == GGUF_Q6_K) w = (w ^ 0x20202020u) & 0x3F3F3F3Fu;
            const uint32_t p0 = w & 0x00FF00FFu, p1 = (w >> 8) & 0x00FF00FFu;  // bytes 0, 2 | 1, 3
            h2 x0, x1;
            __builtin_memcpy(&x0, &p0, 4);
            __builtin_memcpy(&x1, &p1, 4);
            f[4 * wv] = __builtin_fmaf(dd, (float)x0[0], c);
            f[4 * wv + 1] = __builtin_fmaf(dd, (float)x1[0], c);
            f[4 * wv + 2] = __builtin_fmaf(dd, (float)x0[1], c);
            f[4 * wv + 3] = __builtin_fmaf(dd, (float)x1[1], c);
          }
        }
      }
#pragma unroll
      for (int i = 0; i < 8; i += 2) {
        const h2 hp = {(_Float16)f[i], (_Float16)f[i + 1]};
        hv[i] = hp[0];
        hv[i + 1] = hp[1];
        if constexpr (SPLIT) {
          // lo = fp16(f - hi), formed as fma(hi, -1, f) (f - hi is exact in f32, so the same value) by one
          // mixed-precision fma per value that reads hi straight from its half of the packed pair
          uint32_t lp;
          asm("v_fma_mixlo_f16 %0, %1, -1.0, %2 op_sel_hi:[1,0,0]" : "=v"(lp) : "v"(hp), "v"(f[i]));
          asm("v_fma_mixhi_f16 %0, %1, -1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "+v"(lp) : "v"(hp), "v"(f[i + 1]));
          h2 l2;
          __builtin_memcpy(&l2, &lp, 4);
          lv[i] = l2[0];
          lv[i + 1] = l2[1];
        }
      }
    }
    *(h8*)(dst + 8 * v) = hv;
    if constexpr (SPLIT) *(h8*)(dst + lo_off + 8 * v) = lv;
  }
}

// Device-side view of a GroupSched: per-expert strides of the repacked weight (bytes of q, floats of s) and
// the W rows of one expert.
struct GroupKernelArgs {
  const int* tiles = nullptr;
  long long q_stride = 0, s_stride = 0, rows = 0;
};

template <int BM, int BN, int BK, bool DX, int NP>
struct Geo {
  static constexpr int NT = BM >= 256 ? 512 : 256;      // threads: 8 waves for 256-row tiles, else 4
  static constexpr int WGM = NT / 128;                  // waves along M (2 along N)
  static constexpr int TM = BM / (32 * WGM), TN = BN / 64;  // 32×32 tiles per wave
  static constexpr int AROW = BK + 8;                   // A tile row (halves)
  static constexpr int A_H8 = BM * BK / 8 / NT;         // A h8 vectors per thread
  static constexpr int E = BN * BK / NT;                // B values per thread
  // B tile row (halves). DX: 32 halves of padding put the 16-lane groups of a transposed fragment read on
  // disjoint banks (16 halves left half of those reads two-way conflicted).
  static constexpr int BROW = DX ? BN + 32 : BK + 8;
  static constexpr int BROWS = DX ? BK : BN;            // B tile rows
  static constexpr int TPR = (DX ? BN : BK) / E;        // threads per B tile row
  static constexpr int NA = (NP == 2 || NP == 3 || NP == 5) ? 2 : 1, NB = (NP == 3 || NP == 4) ? 2 : 1;
  static constexpr int NSB = NP == 5 ? BK / 32 : 0;  // mode 5: 32-deep scale blocks per slab
  static constexpr int ATILE = BM * AROW, BTILE = BROWS * BROW;
  static constexpr int BUF = NA * ATILE + NB * BTILE;   // halves per stage
  static constexpr int STAGES = BUF * 2 * 2 <= 65536 ? 2 : 1;
  // rank capacity of the fused rank-r staging: the largest multiple of 16 up to 64 whose bf16 hi/lo planes of
  // U [BM][RCAP] and (s·L)ᵀ [BN][RCAP] fit in the LDS the main loop already uses, at least 32
  static constexpr int RFIT = STAGES * BUF / ((BM + BN) * 2) / 16 * 16;
  static constexpr int RCAP = RFIT >= 64 ? 64 : (RFIT >= 32 ? RFIT : 32);
  static constexpr int EPI = (BM + BN) * RCAP * 2;  // halves for the fused rank-r staging
  static constexpr int SMEM = (STAGES * BUF > EPI) ? STAGES * BUF : EPI;
};

#ifndef HOS_QG_PRIO
#define HOS_QG_PRIO 1
#endif
// ---- the GEMM ----
// out[m][n] (over n < Nout) = Σ_c A[m][c] · B(n, c); contraction C split over gridDim.z.
template <uint32_t QT, bool DX, int BM, int BN, int BK, int NP>
// (256-row one-plane tiles: at least 4 waves per SIMD, two workgroups per CU, i.e. at most 128 VGPRs — the
// register file, not the LDS, would otherwise cut their occupancy)
__global__ void __launch_bounds__(BM >= 256 ? 512 : 256, (BM >= 256 && (NP == 1 || NP == 4)) ? 4 : 1) qgemm_kernel(QWeightView w, const _Float16* __restrict__ A,
                                                    const _Float16* __restrict__ Alo, const float* __restrict__ rinv,
                                                    long long lda, int M, int Nout, int C, int c_per_split,
                                                    GemmEpi epi, float* __restrict__ ws, GroupKernelArgs gk) {
  using G = Geo<BM, BN, BK, DX, NP>;
  if (gk.tiles) {  // grouped: this workgroup row is one row tile of one expert
    const int* tl = gk.tiles + 3 * blockIdx.y;
    const int e = tl[0];
    if (e < 0) return;
    const long long r0 = tl[1];
    M = tl[2];
    A += r0 * lda;
    if (Alo) Alo += r0 * lda;
    rinv += r0;
    epi.out += r0 * epi.ldo;
    if (epi.resid) epi.resid += r0 * epi.ldo;
    w.q = (const uint8_t*)w.q + e * gk.q_stride;
    w.s += e * gk.s_stride;
    w.rows = gk.rows;
  }
  static_assert(G::E == 8 || G::E == 16 || G::E == 32, "B run length");
  static_assert(BK % 32 == 0 || (BK == 32), "slab depth");
  constexpr bool ICODE = NP == 5;
  static_assert(!ICODE || (!DX && QT == GGUF_Q8_0), "mode 5: forward, Q8_0 layout");
  constexpr bool ALO = NP == 2 || NP == 3 || ICODE, BLO = NP == 3 || NP == 4;
  // A wave multiplying a slab runs at raised issue priority (s_setprio 1; back to 0 for the loads and LDS stores
  // of the next slab), so the SIMD's other waves do not interleave with its MFMA burst — on the 256-row and the
  // 64-deep tiles, where it measured faster on the MI355X (4096³ 1-pass dX 205 → 190 µs, 3-pass forward 426 → 400 µs,
  // the vocabulary head's dX −3%); the 128×128×32 tiles measured 2–7% slower with it.
  constexpr bool PRIO = HOS_QG_PRIO && (BM >= 256 || BK == 64);
  __shared__ __attribute__((aligned(16))) _Float16 smem[G::SMEM];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  // Workgroup ids are dispatched round-robin over the 8 XCDs, each with its own L2. Give every XCD a contiguous
  // run of tiles — columns fastest, so the tiles that share an A row block share one L2, or rows fastest
  // (epi.rows_fastest) for outputs many tiles wide, so the tiles that share a weight strip run together. (Runs that
  // also keep whole splits of a split contraction on one XCD halved the vocabulary head dX's fetched bytes but
  // made the step's split launches 3% slower on the MI355X: the split index stays blockIdx.z.)
  int wid;
  const int zsp = blockIdx.z;
  if (gk.tiles) {
    wid = blockIdx.x;  // grouped: row tile fixed above, no remap (XCD runs measured 7% slower on OLMoE's step)
  } else {
    const int X = gridDim.x, Y = gridDim.y, T = X * Y, full = T & ~7;
    int t = blockIdx.x + X * blockIdx.y;
    if (t < full) t = (t & 7) * (full >> 3) + (t >> 3);
    wid = epi.rows_fastest ? (t % Y) * X + t / Y : t;
  }
  const int m0 = (wid / gridDim.x) * BM, n0 = (wid % gridDim.x) * BN;
  const int cbeg = zsp * c_per_split;
  const int cend = min(C, cbeg + c_per_split);
  const int nslab = (cend - cbeg) / BK;

  // A wave with fewer than four 32×32 tiles gets several accumulator sets: the passes and k-steps rotate
  // over them, so the MFMA pipe always has independent chains instead of one chain that waits for each
  // previous MFMA's result. They are summed in a fixed order before the epilogue.
  constexpr int NACC = (ICODE || G::TM * G::TN >= 4) ? 1 : (G::TM * G::TN == 2 ? 2 : 4);
  constexpr int NPASS = 1 + (ALO ? 1 : 0) + (BLO ? 1 : 0);
  // mode 5: block accumulators, one set (the hi and lo products of all tiles interleave) or, with fewer than four
  // tiles per wave, one set per product so that consecutive MFMAs never share an accumulator
  constexpr int NBLK = G::TM * G::TN >= 4 ? 1 : 2;
  f16v accs[NACC][G::TM][G::TN];
#pragma unroll
  for (int a = 0; a < NACC; a++)
#pragma unroll
    for (int i = 0; i < G::TM; i++)
#pragma unroll
      for (int j = 0; j < G::TN; j++)
#pragma unroll
        for (int r = 0; r < 16; r++) accs[a][i][j][r] = 0.0f;

  // Raw (still quantized / still in registers) data of the slabs ahead, in flight from HBM while the
  // current slab is multiplied: R0 = slab s+1 (issued one slab ago), R1 = slab s+2 (issued now). Two
  // slabs of lead cover the global-memory latency that one slab's MFMA work cannot.
  struct Regs {
    h8 a[G::A_H8], al[G::A_H8];
    Run<QT, G::E> b;
    float sc[ICODE ? G::TN * G::NSB : 1];  // mode 5: d of this lane's output columns, per 32-block of the slab
  };
  float scur[ICODE ? G::TN * G::NSB : 1];  // the scales of the slab in LDS
  Regs R0, R1;
  // this thread's B run: tile row br, first column bc. Its element index at slab 0, e0, is fixed for the launch; a
  // run past the last output column is clamped into the weight (it only feeds columns that are never stored).
  const int br = tid / G::TPR, bc = G::E * (tid % G::TPR);
  long long e0;
  if constexpr (DX) {
    const int col = n0 + bc;  // output column run; rows are the contraction
    e0 = (long long)br * w.cols + (col < w.cols ? col : 0);
  } else {
    const long long row = n0 + br;  // W row = output column; run along the contraction
    e0 = (row < w.rows ? row : 0) * w.cols + bc;
  }
  const uint8_t* const bq = (const uint8_t*)w.q + run_qoff<QT>(e0);
  const float* const bs_ = w.s + run_soff<QT>(e0);

  auto load = [&](Regs& R, int c0) {
#pragma unroll
    for (int v = 0; v < G::A_H8; v++) {
      int idx = tid + G::NT * v;  // h8 index within the BM×BK tile
      int row = idx / (BK / 8), cv = idx % (BK / 8);
      int m = m0 + row;
      long long off = (long long)m * lda + c0 + 8 * cv;
      // Rows past M re-read row M-1: they only feed output rows past M, which are never stored. No
      // branch, so the compiler counts the loads in flight exactly and waits only for the slab it needs.
      const long long offc = m < M ? off : (long long)(M - 1) * lda + c0 + 8 * cv;
      R.a[v] = *(const h8*)(A + offc);
      if constexpr (ALO) R.al[v] = *(const h8*)(Alo + offc);
    }
    {
      // the slab part of the run's element index: c0 rows further (dX) or c0 columns further (forward)
      const long long se = DX ? (long long)c0 * w.cols : (long long)c0;
      run_load<QT, G::E>(bq + run_qoff<QT>(se), bs_ + run_soff<QT>(se), R.b);
    }
    if constexpr (ICODE) {
#pragma unroll
      for (int j = 0; j < G::TN; j++) {
        const long long n = n0 + wn * (BN / 2) + 32 * j + (lane & 31);
        const long long base = (n < w.rows ? n : 0) * (w.cols >> 5) + (c0 >> 5);
#pragma unroll
        for (int b = 0; b < G::NSB; b++) R.sc[j * G::NSB + b] = w.s[base + b];
      }
    }
  };
  auto store = [&](const Regs& R, _Float16* buf) {
#pragma unroll
    for (int v = 0; v < G::A_H8; v++) {
      int idx = tid + G::NT * v;
      int row = idx / (BK / 8), cv = idx % (BK / 8);
      *(h8*)(buf + row * G::AROW + 8 * cv) = R.a[v];
      if constexpr (ALO) *(h8*)(buf + G::ATILE + row * G::AROW + 8 * cv) = R.al[v];
    }
    _Float16* bs = buf + G::NA * G::ATILE;
    run_store<QT, G::E, BLO, ICODE>(R.b, bs + br * G::BROW + bc, G::BTILE);
  };
  auto take_scales = [&](const Regs& R) {
    if constexpr (ICODE) {
#pragma unroll
      for (int i = 0; i < G::TN * G::NSB; i++) scur[i] = R.sc[i];
    }
  };

  if (nslab > 0) {
    load(R0, cbeg);
    store(R0, smem);
    take_scales(R0);
    load(R0, cbeg + min(1, nslab - 1) * BK);
  }
  __syncthreads();

  for (int s = 0; s < nslab; s++) {
    const int buf = G::STAGES == 2 ? (s & 1) : 0;
    const bool more = s + 1 < nslab;
    load(R1, cbeg + min(s + 2, nslab - 1) * BK);  // past the end: a harmless re-read of the last slab
    const _Float16* as = smem + buf * G::BUF;
    const _Float16* bs = as + G::NA * G::ATILE;
    if constexpr (PRIO) __builtin_amdgcn_s_setprio(1);
    if constexpr (ICODE) {
#pragma unroll
      for (int kb = 0; kb < BK; kb += 32) {
        f16v blk[NBLK][G::TM][G::TN];
#pragma unroll
        for (int k2 = 0; k2 < 32; k2 += 16) {
          h8 af[G::TM], afl[G::TM], bf[G::TN];
          const int koff = kb + k2 + 8 * (lane >> 5);
#pragma unroll
          for (int i = 0; i < G::TM; i++) {
            int ro = (wm * (BM / G::WGM) + 32 * i + (lane & 31)) * G::AROW + koff;
            af[i] = *(const h8*)(as + ro);
            afl[i] = *(const h8*)(as + G::ATILE + ro);
          }
#pragma unroll
          for (int j = 0; j < G::TN; j++) {
            int ro = (wn * (BN / 2) + 32 * j + (lane & 31)) * G::BROW + koff;
            bf[j] = *(const h8*)(bs + ro);
          }
          const f16v z = {};
#pragma unroll
          for (int i = 0; i < G::TM; i++)
#pragma unroll
            for (int j = 0; j < G::TN; j++)
              blk[0][i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], k2 == 0 ? z : blk[0][i][j], 0, 0, 0);
#pragma unroll
          for (int i = 0; i < G::TM; i++)
#pragma unroll
            for (int j = 0; j < G::TN; j++) {
              f16v& t = blk[NBLK - 1][i][j];
              t = __builtin_amdgcn_mfma_f32_32x32x16_f16(afl[i], bf[j], (NBLK == 2 && k2 == 0) ? z : t, 0, 0, 0);
            }
        }
#pragma unroll
        for (int i = 0; i < G::TM; i++)
#pragma unroll
          for (int j = 0; j < G::TN; j++) {
            const float sj = scur[j * G::NSB + kb / 32];
#pragma unroll
            for (int r = 0; r < 16; r++) {
              float v = blk[0][i][j][r];
              if constexpr (NBLK == 2) v += blk[1][i][j][r];
              accs[0][i][j][r] = __builtin_fmaf(sj, v, accs[0][i][j][r]);
            }
          }
      }
    } else
#pragma unroll
    for (int kk = 0; kk < BK; kk += 16) {
      h8 af[G::TM], afl[G::TM], bf[G::TN], bfl[G::TN];
      const int koff = kk + 8 * (lane >> 5);
#pragma unroll
      for (int i = 0; i < G::TM; i++) {
        int ro = (wm * (BM / G::WGM) + 32 * i + (lane & 31)) * G::AROW + koff;
        af[i] = *(const h8*)(as + ro);
        if constexpr (ALO) afl[i] = *(const h8*)(as + G::ATILE + ro);
      }
#pragma unroll
      for (int j = 0; j < G::TN; j++) {
        if constexpr (DX) {
          // 16-lane group g: columns 16·(g%2) .. +15 of this 32-wide tile, contraction kk + 8·(g/2) .. +7
          const int g = lane >> 4, L = lane & 15;
          const int col = wn * (BN / 2) + 32 * j + 16 * (g & 1) + 4 * (L & 3);
          const int row = kk + 8 * (g >> 1) + (L >> 2);
          const _Float16* p = bs + row * G::BROW + col;
          typedef __attribute__((address_space(3))) s4v* lds_s4;
          s4v x0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4)(p));
          s4v x1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4)(p + 4 * G::BROW));
          __builtin_memcpy(&bf[j], &x0, 8);
          __builtin_memcpy((char*)&bf[j] + 8, &x1, 8);
          if constexpr (BLO) {
            s4v y0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4)(p + G::BTILE));
            s4v y1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4)(p + G::BTILE + 4 * G::BROW));
            __builtin_memcpy(&bfl[j], &y0, 8);
            __builtin_memcpy((char*)&bfl[j] + 8, &y1, 8);
          }
        } else {
          int ro = (wn * (BN / 2) + 32 * j + (lane & 31)) * G::BROW + koff;
          bf[j] = *(const h8*)(bs + ro);
          if constexpr (BLO) bfl[j] = *(const h8*)(bs + G::BTILE + ro);
        }
      }
      // chain index of this k-step's first pass; the passes are issued outermost, so consecutive MFMAs go to
      // different tiles (each accumulator receives the same products in the same order as tile-major issue, which
      // put a tile's three dependent passes back to back: the step +0.9%, 4096³ 3-pass dX −2%)
      const int cb = NPASS * (kk / 16);
      auto pass_blo = [&]() {
        if constexpr (BLO)
#pragma unroll
          for (int i = 0; i < G::TM; i++)
#pragma unroll
            for (int j = 0; j < G::TN; j++) {
              f16v& t = accs[(cb + 2) % NACC][i][j];
              t = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bfl[j], t, 0, 0, 0);
            }
      };
      auto pass_alo = [&]() {
        if constexpr (ALO)
#pragma unroll
          for (int i = 0; i < G::TM; i++)
#pragma unroll
            for (int j = 0; j < G::TN; j++) {
              f16v& t = accs[(cb + 1) % NACC][i][j];
              t = __builtin_amdgcn_mfma_f32_32x32x16_f16(afl[i], bf[j], t, 0, 0, 0);
            }
      };
      auto pass_hi = [&]() {
#pragma unroll
        for (int i = 0; i < G::TM; i++)
#pragma unroll
          for (int j = 0; j < G::TN; j++) {
            f16v& t = accs[cb % NACC][i][j];
            t = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], t, 0, 0, 0);
          }
      };
      if constexpr (NACC == 4) {
        // the passes of a k-step go to chains cb, cb + 1, cb + 2 (mod 4), all distinct: issued in that order they
        // cycle through the four sets (the longest distance between dependent MFMAs; the same products per set in
        // the same order either way)
        pass_hi();
        pass_alo();
        pass_blo();
      } else {
        pass_blo();
        pass_alo();
        pass_hi();
      }
    }
    if constexpr (PRIO) __builtin_amdgcn_s_setprio(0);
    if (more) {
      if constexpr (G::STAGES == 1) __syncthreads();  // everyone is done reading the single stage
      store(R0, smem + (G::STAGES == 2 ? (buf ^ 1) : 0) * G::BUF);
      take_scales(R0);
    }
    R0 = R1;
    __syncthreads();
  }

  f16v(&acc)[G::TM][G::TN] = accs[0];
#pragma unroll
  for (int a = 1; a < NACC; a++)
#pragma unroll
    for (int i = 0; i < G::TM; i++)
#pragma unroll
      for (int j = 0; j < G::TN; j++) acc[i][j] += accs[a][i][j];

  // epilogue: D[i][j] of a 32×32 tile lives at lane j + 32·((i/4)&1), register (i&3) + 4·(i/8)
  const bool split = gridDim.z > 1;
  // Fused rank-r update s·U·L on bf16 MFMA, accumulated into acc before the row scale: U [BM][r] (each row
  // divided by its power-of-two rinv, exact) and the transposed (s·L)ᵀ [BN][r] are staged in the (now free)
  // LDS as bf16 hi/lo planes, zero-padded to a multiple of 16, and each 32×32 tile takes three products per
  // 16 ranks (hi·hi + lo·hi + hi·lo: ~2^-16 relative to the rank-r term, fp32 range). A staged row is rpad
  // bf16 long; its 16-byte chunks are XOR-swizzled by the row so that the 32 rows of one fragment read spread
  // over the LDS banks.
  // (split contraction: the first split's workgroups carry the rank-r term in their partial; U is pre-divided by
  // the row's power-of-two rinv, so the reduction's (Σ partials)·rinv is exactly the unsplit result's form)
  // Ranks above the staging's capacity (G::RCAP) run in chunks of that many ranks, one staging and product per chunk.
  const int rank = (split && zsp != 0) ? 0 : epi.rank;
  for (int rc0 = 0; rc0 < rank; rc0 += G::RCAP) {
    const int rn = min(G::RCAP, rank - rc0);
    const int rpad = (rn + 15) & ~15;
    const int nch = rpad >> 3, swz = (nch & (nch - 1)) ? 1 : nch - 1;
    auto sidx = [&](int row, int q) { return row * rpad + ((((q >> 3) ^ (row & swz))) << 3) + (q & 7); };
    __bf16* Uh = (__bf16*)smem;
    __bf16* Ul = Uh + BM * rpad;
    __bf16* Lh = Ul + BM * rpad;
    __bf16* Ll = Lh + BN * rpad;
    if (rc0 > 0) __syncthreads();  // every wave is done reading the previous chunk
    // a tile never straddles a column segment (the launcher picks BN to divide the boundaries)
    const float* Ub = epi.U + (epi.ustep ? epi.ustep * ((n0 >= epi.ub0) + (n0 >= epi.ub1)) : 0) + rc0;
    const float* Lb = epi.L + (long long)rc0 * epi.slj;
    for (int e = tid; e < BM * rpad; e += G::NT) {
      const int rr = e / rpad, jj = e % rpad, row = m0 + rr;
      const float x = (row < M && jj < rn) ? Ub[(long long)row * epi.ldu + jj] / rinv[row] : 0.0f;
      const __bf16 h = (__bf16)x;
      Uh[sidx(rr, jj)] = h;
      Ul[sidx(rr, jj)] = (__bf16)(x - (float)h);
    }
    for (int e = tid; e < rpad * BN; e += G::NT) {
      const int jj = e / BN, cc = e % BN, col = n0 + cc;
      const float x =
          (col < Nout && jj < rn) ? Lb[(long long)jj * epi.slj + (long long)col * epi.sln] * epi.scale : 0.0f;
      const __bf16 h = (__bf16)x;
      Lh[sidx(cc, jj)] = h;
      Ll[sidx(cc, jj)] = (__bf16)(x - (float)h);
    }
    __syncthreads();
    // per 16 ranks: each tile's three products (lo·hi, hi·lo, hi·hi, as mma3_bf16) issued pass by pass across the
    // tiles, the fragments read once for all tiles of their row or column
    for (int k0 = 0; k0 < rpad; k0 += 16) {
      const int k = k0 + 8 * (lane >> 5);
      bf8 ah[G::TM], al[G::TM], bh[G::TN], bl[G::TN];
#pragma unroll
      for (int i = 0; i < G::TM; i++) {
        const int ra = wm * (BM / G::WGM) + 32 * i + (lane & 31);
        ah[i] = *(const bf8*)(Uh + sidx(ra, k));
        al[i] = *(const bf8*)(Ul + sidx(ra, k));
      }
#pragma unroll
      for (int j = 0; j < G::TN; j++) {
        const int rb = wn * (BN / 2) + 32 * j + (lane & 31);
        bh[j] = *(const bf8*)(Lh + sidx(rb, k));
        bl[j] = *(const bf8*)(Ll + sidx(rb, k));
      }
#pragma unroll
      for (int i = 0; i < G::TM; i++)
#pragma unroll
        for (int j = 0; j < G::TN; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al[i], bh[j], acc[i][j], 0, 0, 0);
#pragma unroll
      for (int i = 0; i < G::TM; i++)
#pragma unroll
        for (int j = 0; j < G::TN; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah[i], bl[j], acc[i][j], 0, 0, 0);
#pragma unroll
      for (int i = 0; i < G::TM; i++)
#pragma unroll
        for (int j = 0; j < G::TN; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah[i], bh[j], acc[i][j], 0, 0, 0);
    }
  }
  // Output stores. Each 32×32 tile goes through a per-wave LDS transpose and leaves as row-major float4 runs
  // (8 lanes per 128-byte row piece): a quarter of the store instructions of the MFMA layout's one-float-per-lane
  // stores, and one row scale per lane per pass.
  constexpr int TS = 40;  // f32 row stride of a staged tile (4·TS ≡ 32 banks: the two half-waves' rows are disjoint)
  if constexpr (G::SMEM * 2 >= G::NT / 64 * 32 * TS * 4) {
    __syncthreads();  // every wave is done with the main loop's and the rank term's LDS
    float* tb = reinterpret_cast<float*>(smem) + wave * 32 * TS;
    // row statistics (epi.rstat): this wave's rows over its 64 columns, one (max, exp-sum) per lane per (i, pass)
    // folded over the TN column tiles, then over the 8 lanes of a row
    const bool stats = epi.rstat != nullptr && !split;
    float smx[G::TM][4], ssm[G::TM][4];
#pragma unroll
    for (int i = 0; i < G::TM; i++)
#pragma unroll
      for (int pz = 0; pz < 4; pz++) {
        smx[i][pz] = -INFINITY;
        ssm[i][pz] = 0.0f;
      }
    const bool vec = (Nout & 3) == 0 && (split || ((epi.ldo & 3) == 0 && ((uintptr_t)epi.out & 15) == 0 &&
                                                  (!epi.resid || ((uintptr_t)epi.resid & 15) == 0) &&
                                                  (!epi.bias || ((uintptr_t)epi.bias & 15) == 0)));
#pragma unroll
    for (int i = 0; i < G::TM; i++)
#pragma unroll
      for (int j = 0; j < G::TN; j++) {
#pragma unroll
        for (int r = 0; r < 16; r++) tb[(8 * (r >> 2) + 4 * (lane >> 5) + (r & 3)) * TS + (lane & 31)] = acc[i][j][r];
#pragma unroll
        for (int pz = 0; pz < 4; pz++) {
          const int lr = 8 * pz + (lane >> 3), c4 = 4 * (lane & 7);
          const float4 t4 = *reinterpret_cast<const float4*>(tb + lr * TS + c4);
          const int row = m0 + wm * (BM / G::WGM) + 32 * i + lr, col = n0 + wn * (BN / 2) + 32 * j + c4;
          if (row >= M || col >= Nout) continue;
          float v[4] = {t4.x, t4.y, t4.z, t4.w};
          if (split) {
            float* d = ws + ((long long)zsp * M + row) * Nout + col;
            if (vec) {
              *reinterpret_cast<float4*>(d) = make_float4(v[0], v[1], v[2], v[3]);
            } else {
              for (int e = 0; e < 4 && col + e < Nout; e++) d[e] = v[e];
            }
            continue;
          }
          const float ri = rinv[row];
          const long long off = (long long)row * epi.ldo + col;
          float* o = epi.out + off;
          if (vec) {
            const float4 b4 = epi.bias ? *reinterpret_cast<const float4*>(epi.bias + col) : make_float4(0.f, 0.f, 0.f, 0.f);
            float4 y = make_float4(v[0] * ri + b4.x, v[1] * ri + b4.y, v[2] * ri + b4.z, v[3] * ri + b4.w);
            if (epi.accumulate || epi.resid) {
              const float4 q = *reinterpret_cast<const float4*>(epi.accumulate ? o : epi.resid + off);
              y = make_float4(q.x + y.x, q.y + y.y, q.z + y.z, q.w + y.w);
            }
            *reinterpret_cast<float4*>(o) = y;
            if (stats) {
              const float yv[4] = {y.x, y.y, y.z, y.w};
              float mx = -INFINITY;
#pragma unroll
              for (int e = 0; e < 4; e++)
                if (col + e < Nout) mx = fmaxf(mx, yv[e]);
              float& m = smx[i][pz];
              float& sm = ssm[i][pz];
              if (mx > m) {
                sm = m == -INFINITY ? 0.0f : sm * exp_rs(m - mx);
                m = mx;
              }
#pragma unroll
              for (int e = 0; e < 4; e++)
                if (col + e < Nout) sm += exp_rs(yv[e] - m);
            }
          } else {
            for (int e = 0; e < 4 && col + e < Nout; e++) {
              float x = v[e] * ri;
              if (epi.bias) x += epi.bias[col + e];
              x = epi.accumulate ? o[e] + x : (epi.resid ? epi.resid[off + e] + x : x);
              o[e] = x;
              if (stats) {
                float& m = smx[i][pz];
                float& sm = ssm[i][pz];
                if (x > m) {
                  sm = m == -INFINITY ? 0.0f : sm * exp_rs(m - x);
                  m = x;
                }
                sm += exp_rs(x - m);
              }
            }
          }
        }
      }
    if (stats) {
      // the 8 lanes of a row (lane bits 0-2) merge in a fixed tree order; lane 8·k writes row 8·pz + k
      const long long chunk = (n0 + wn * (BN / 2)) / 64;
#pragma unroll
      for (int i = 0; i < G::TM; i++)
#pragma unroll
        for (int pz = 0; pz < 4; pz++) {
          float m = smx[i][pz], sm = ssm[i][pz];
#pragma unroll
          for (int o = 1; o < 8; o <<= 1) {
            const float m2 = __shfl_xor(m, o), s2 = __shfl_xor(sm, o), mn = fmaxf(m, m2);
            sm = (m == -INFINITY ? 0.0f : sm * exp_rs(m - mn)) + (m2 == -INFINITY ? 0.0f : s2 * exp_rs(m2 - mn));
            m = mn;
          }
          const int row = m0 + wm * (BM / G::WGM) + 32 * i + 8 * pz + (lane >> 3);
          if ((lane & 7) == 0 && row < M && n0 + wn * (BN / 2) < Nout)
            epi.rstat[(long long)row * epi.rstat_ld + chunk] = make_float2(m, sm);
        }
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < G::TM; i++)
#pragma unroll
    for (int j = 0; j < G::TN; j++) {
      const int cc = wn * (BN / 2) + 32 * j + (lane & 31);
      const int col = n0 + cc;
      if (col >= Nout) continue;
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int rr = wm * (BM / G::WGM) + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        const int row = m0 + rr;
        if (row >= M) continue;
        float v = acc[i][j][r];
        if (split) {
          ws[((long long)zsp * M + row) * Nout + col] = v;
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

// Deterministic split-K reduction + the same epilogue (the rank-r term is already in the first split's partial).
// Workgroup = RED_ROWS rows × 1024 columns, a thread per 4 columns (16-byte loads); rows go four at a time with all
// their partial loads issued together; partials are summed in split order.
#ifndef HOS_RED_ROWS
#define HOS_RED_ROWS 4
#endif
constexpr int RED_ROWS = HOS_RED_ROWS;  // 4: one pass of four rows, so the grid spreads over every CU
__global__ void __launch_bounds__(256) splitk_reduce4(const float* __restrict__ ws, int splits, int M, int N,
                                                      const float* __restrict__ rinv, GemmEpi epi) {
  const int r0 = blockIdx.y * RED_ROWS, col = (blockIdx.x * 256 + threadIdx.x) * 4;
  if (col >= N) return;
  const long long MN = (long long)M * N;
  const float4 bias = epi.bias ? *(const float4*)(epi.bias + col) : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int rq = 0; rq < RED_ROWS; rq += 4) {
    float4 v[4];
#pragma unroll
    for (int u = 0; u < 4; u++) v[u] = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int z = 0; z < splits; z++)
#pragma unroll
      for (int u = 0; u < 4; u++) {
        const float4 p = *(const float4*)(ws + z * MN + (long long)min(r0 + rq + u, M - 1) * N + col);
        v[u].x += p.x;
        v[u].y += p.y;
        v[u].z += p.z;
        v[u].w += p.w;
      }
#pragma unroll
    for (int u = 0; u < 4; u++) {
      const int row = r0 + rq + u;
      if (row >= M) return;
      const float ri = rinv[row];
      float4 x = make_float4(v[u].x * ri, v[u].y * ri, v[u].z * ri, v[u].w * ri);
      if (epi.bias) {
        x.x += bias.x;
        x.y += bias.y;
        x.z += bias.z;
        x.w += bias.w;
      }
      const long long off = (long long)row * epi.ldo + col;
      float4* o = (float4*)(epi.out + off);
      if (epi.accumulate) {
        const float4 a = *o;
        x = make_float4(a.x + x.x, a.y + x.y, a.z + x.z, a.w + x.w);
      } else if (epi.resid) {
        const float4 a = *(const float4*)(epi.resid + off);
        x = make_float4(a.x + x.x, a.y + x.y, a.z + x.z, a.w + x.w);
      }
      *o = x;
    }
  }
}
// The same for shapes the 16-byte form does not fit (a thread per column).
__global__ void __launch_bounds__(256) splitk_reduce1(const float* __restrict__ ws, int splits, int M, int N,
                                                      const float* __restrict__ rinv, GemmEpi epi) {
  const int r0 = blockIdx.y * RED_ROWS, col = blockIdx.x * 256 + threadIdx.x;
  if (col >= N) return;
  const long long MN = (long long)M * N;
#pragma unroll
  for (int rq = 0; rq < RED_ROWS; rq += 4) {
    float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int z = 0; z < splits; z++)
#pragma unroll
      for (int u = 0; u < 4; u++) v[u] += ws[z * MN + (long long)min(r0 + rq + u, M - 1) * N + col];
#pragma unroll
    for (int u = 0; u < 4; u++) {
      const int row = r0 + rq + u;
      if (row >= M) return;
      float x = v[u] * rinv[row];
      if (epi.bias) x += epi.bias[col];
      const long long off = (long long)row * epi.ldo + col;
      float* o = epi.out + off;
      *o = epi.accumulate ? *o + x : (epi.resid ? epi.resid[off] + x : x);
    }
  }
}
void launch_splitk_reduce(const float* ws, int splits, long long M, int N, const float* rinv, const GemmEpi& epi,
                          hipStream_t st) {
  auto al16 = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
  const bool v4 = N % 4 == 0 && epi.ldo % 4 == 0 && al16(ws) && al16(epi.out) && (!epi.bias || al16(epi.bias)) &&
                  (!epi.resid || al16(epi.resid));
  if (v4) {
    dim3 rg(ceil_div(N, 1024), ceil_div(M, RED_ROWS));
    splitk_reduce4<<<rg, 256, 0, st>>>(ws, splits, (int)M, N, rinv, epi);
  } else {
    dim3 rg(ceil_div(N, 256), ceil_div(M, RED_ROWS));
    splitk_reduce1<<<rg, 256, 0, st>>>(ws, splits, (int)M, N, rinv, epi);
  }
  HOS_HIP_CHECK(hipGetLastError());
}

template <uint32_t QT, bool DX, int BM, int BN, int BK, int NP>
void launch_shape(const QWeight& w, H16 a, long long lda, long long M, int Nout, int C, int per, int splits,
                  GemmEpi epi, float* ws, hipStream_t st) {
  HOS_REQUIRE(!epi.rstat || (BN == 128 && splits == 1 &&
                             Geo<BM, BN, BK, DX, NP>::SMEM * 2 >= Geo<BM, BN, BK, DX, NP>::NT / 64 * 32 * 40 * 4),
              HOS_E_INVALID, "qgemm: row statistics need the staged epilogue on unsplit 128-column tiles");
  dim3 grid(ceil_div(Nout, BN), ceil_div(M, BM), splits);
  qgemm_kernel<QT, DX, BM, BN, BK, NP>
      <<<grid, Geo<BM, BN, BK, DX, NP>::NT, 0, st>>>(view(w), a.data, a.lo, a.rinv, lda, (int)M, Nout, C, per, epi, ws,
                                                     GroupKernelArgs{});
}

template <uint32_t QT, bool DX, int NP>
void launch_typed(const QWeight& w, H16 a, long long lda, long long M, GemmEpi epi, float* ws, size_t ws_bytes,
                  hipStream_t st) {
  const int Nout = DX ? (int)w.cols : (int)w.rows;
  const int C = DX ? (int)w.rows : (int)w.cols;
  HOS_REQUIRE(C % 32 == 0, HOS_E_INVALID, "qgemm: contraction length must be a multiple of 32");
  HOS_REQUIRE((lda % 8) == 0, HOS_E_INVALID, "qgemm: activation row stride must be a multiple of 8");
  HOS_REQUIRE((NP != 2 && NP != 3 && NP != 5) || a.lo != nullptr, HOS_E_INVALID,
              "qgemm: activation-split precision needs the operand residual");
  HOS_REQUIRE(epi.rank >= 0 && epi.rank <= 128, HOS_E_INVALID, "qgemm: fused rank-r update supports r <= 128");
  // Tile choice: the largest tile that still gives ~1.25 waves of workgroups over the 256 CUs; only when
  // even 64×64 tiles leave the chip idle is the contraction split (deterministic reduction after).
  auto ntiles = [&](int bm, int bn) { return ceil_div(M, bm) * ceil_div(Nout, bn); };
  int bm = 64, bn = 64, bk = 32;
  // A very long contraction (the vocabulary-wide head dX) is bound by re-reading the operands once per
  // tile row / column: take the largest tile and split the contraction instead.
  const bool longc = C >= 16384;
  if (ntiles(128, 128) >= 320 || longc) {
    bm = 128;
    bn = 128;
  } else if (ntiles(64, 128) >= 320) {
    bm = 64;
    bn = 128;
  } else if (ntiles(128, 64) >= 320) {
    bm = 128;
    bn = 64;
  }
  // An f32 weight (the full finetune's trainable weights and its dW, whose "weight" is the f32 activation) costs 4
  // bytes per element, so the weight strip each tile re-reads weighs more: 128×128 tiles from 256 of them on (its
  // dW of a 4864-row weight over 2048 tokens, 896 columns: 116 -> 102 µs on the MI355X).
  const bool f32w = QT == GGUF_F32;
  if (f32w && bm * bn < 128 * 128 && ntiles(128, 128) >= 256) {
    bm = 128;
    bn = 128;
  }
  // A long contraction over a narrow output (the stacked gate|up dX, the FFN down projection forward): big
  // tiles split over the contraction beat small unsplit tiles (measured on the MI355X at M 2048: dX 9728 -> 896
  // 155 vs 210 us, forward 4864 -> 896 81 vs 108 us).
  const bool split_big = !longc && C >= 4096 && ntiles(128, 128) < 320;
  if (split_big) {
    bm = 128;
    bn = 128;
  }
  // 64-deep slabs where the contraction is long enough to amortize the deeper prologue: two-plane forwards from
  // C 2048 on (M 8192, Q4_K: 2048 -> 16384 1788 vs 1811 us, 8192 -> 2048 899 vs 960; at C 896 32-deep slabs win,
  // 163 vs 171 us) and the split forward; two-plane dX launches from C 2048 on with narrow outputs (≤ 4096 columns:
  // Llama-3.2-1B's q|k|v and o dX, the step's dX −2.4%), else 32 (equal or faster at the other step shapes: split
  // 9728 -> 896 148 vs 155 us, 2048 -> 8192 897 vs 912 us).
  const bool deep_fwd = !DX && (NP == 2 || NP == 3) && (C >= 2048 || split_big);
  const bool deep_dx = DX && (NP == 2 || NP == 3) && C >= 2048 && Nout <= 4096 && !split_big && !f32w;
  if (C % 64 == 0 &&
      ((bm == 64 && bn == 64) || ((NP == 1 || longc || deep_fwd || deep_dx) && bm == 128 && bn == 128)))
    bk = 64;
  // Single-pass GEMMs are bound by the weight dequantization (VALU) as much as by MFMA: 8 waves on a
  // 256-row tile dequantize each B slab once for twice the MFMA work.
  // The same holds for the weight-split mode 4 (one activation plane) and for the vocabulary-wide head in either
  // direction (measured at Qwen2.5-0.5B, Q8_0 head, M 2048 × V 151936 × 896, warm: forward 1040-1130 µs vs 1160
  // on 128×128×64, dX in mode 4 1100-1170 µs vs 1430).
  const bool one_plane = NP == 1 || NP == 4;
  if (one_plane && (longc || ntiles(256, 128) >= 256) && (C >= 2048 || Nout >= 16384 || longc)) {
    bm = 256;
    bn = 128;
    bk = 32;
  }
  // A fused rank above 32 (stacked q|k|v dX): no split, and 128×128×64 tiles where they alone give every CU one
  // (OLMoE's q|k|v dX, 2048 × 2048 × 6144 at rank 48: 254 µs on 64×64 tiles), else 64×64 (whose staging holds rank 64
  // in one chunk).
  if (epi.rank > 32) {
    if (C % 64 == 0 && ntiles(128, 128) >= 256) {
      bm = 128;
      bn = 128;
      bk = 64;
    } else {
      bm = 64;
      bn = 64;
      bk = C % 64 == 0 ? 64 : 32;
    }
  }
  // Column-segmented U (stacked projections): tiles must not straddle a segment boundary, and the split-K
  // reduction (which stages one U block for all its columns) is not used.
  const bool useg = epi.rank > 0 && epi.ustep > 0;
  if (useg) {
    auto fits = [&](int b) { return epi.ub0 % b == 0 && (epi.ub1 >= Nout || epi.ub1 % b == 0); };
    if (!fits(bn)) {
      bn = 64;
      if (bm == 256) bm = 128;
      if (bk == 64 && !(bm == 64 || C % 64 == 0)) bk = 32;
    }
    HOS_REQUIRE(fits(bn), HOS_E_INVALID, "qgemm: column segments must be multiples of 64");
  }
  // Row statistics: the epilogue folds them per wave over 64 output columns, i.e. unsplit 128-column tiles.
  if (epi.rstat) {
    HOS_REQUIRE(!DX && !useg, HOS_E_INVALID, "qgemm: row statistics are for plain forward launches");
    bm = one_plane ? 256 : 128;
    bn = 128;
    bk = 32;
  }
  int tiles = ntiles(bm, bn);
  int nslab = C / bk;
  int splits = 1;
  while (!epi.rstat && !useg && epi.rank <= 32 && tiles * splits < 320 && nslab / (splits * 2) >= 8 &&
         (size_t)(splits * 2) * M * Nout * sizeof(float) <= ws_bytes)
    splits *= 2;
#ifdef HOS_QG_ENV_TILE
  if (const char* f = getenv("QG_TILE")) {
    int a1, a2, a3, a4;
    if (sscanf(f, "%d,%d,%d,%d", &a1, &a2, &a3, &a4) == 4) { bm = a1; bn = a2; bk = a3; splits = a4; nslab = C / bk; }
    HOS_REQUIRE(splits == 1 || (size_t)splits * M * Nout * sizeof(float) <= ws_bytes, HOS_E_INVALID,
                "forced tile: split-K partials exceed the workspace");
    HOS_REQUIRE(C % bk == 0 && epi.rank <= 32 && !useg, HOS_E_INVALID, "forced tile: unsupported");
  }
#endif
  int per = ceil_div(nslab, splits) * bk;
  splits = ceil_div(C, per);
  // Outputs many tiles wide (the vocabulary head's forward): rows fastest, so each weight strip is fetched once.
  if (ceil_div(Nout, bn) >= 64 * ceil_div(M, bm)) epi.rows_fastest = 1;
#define HOS_QG(BM_, BN_, BK_) \
  if (bm == BM_ && bn == BN_ && bk == BK_) launch_shape<QT, DX, BM_, BN_, BK_, NP>(w, a, lda, M, Nout, C, per, splits, epi, ws, st)
  HOS_QG(128, 128, 64);
  else HOS_QG(128, 128, 32);
  else HOS_QG(64, 128, 32);
  else HOS_QG(128, 64, 32);
  else HOS_QG(64, 64, 32);
  else HOS_QG(64, 128, 64);
  else HOS_QG(128, 64, 64);
  else HOS_QG(64, 64, 64);
  else HOS_QG(256, 128, 32);
  else throw Error(HOS_E_INVALID, "qgemm: no kernel for the chosen tile");
#undef HOS_QG
  HOS_HIP_CHECK(hipGetLastError());
  if (epi.defer) {
    HOS_REQUIRE(splits == 1 || (!epi.bias && !epi.accumulate), HOS_E_INVALID,
                "qgemm: a deferred reduction takes no bias and no accumulation");
    *epi.defer = splits;
  } else if (splits > 1) {
    launch_splitk_reduce(ws, splits, M, Nout, a.rinv, epi, st);
  }
}

// Grouped launch (mixture-of-experts): W = n_experts stacked blocks, 128×128 tiles, no split.
template <uint32_t QT, bool DX, int NP>
void launch_typed_grouped(const QWeight& w, GroupSched gs, H16 a, long long lda, GemmEpi epi, hipStream_t st) {
  HOS_REQUIRE(gs.n_experts > 0 && w.rows % gs.n_experts == 0, HOS_E_INVALID, "grouped qgemm: bad expert count");
  const long long er = w.rows / gs.n_experts;  // W rows of one expert
  const int Nout = DX ? (int)w.cols : (int)er;
  const int C = DX ? (int)er : (int)w.cols;
  HOS_REQUIRE(C % 32 == 0 && lda % 8 == 0, HOS_E_INVALID, "grouped qgemm: contraction must be a multiple of 32");
  HOS_REQUIRE((NP != 2 && NP != 3 && NP != 5) || a.lo != nullptr, HOS_E_INVALID,
              "grouped qgemm: needs the operand residual");
  HOS_REQUIRE(epi.rank == 0 && !epi.rstat, HOS_E_INVALID, "grouped qgemm: no fused rank-r term or row statistics");
  GroupKernelArgs gk;
  gk.tiles = gs.tiles;
  gk.rows = er;
  const long long n = er * w.cols;  // elements of one expert
  gk.q_stride = QT == GGUF_Q4_K ? n / 2 : n * elem_bytes<QT>();
  gk.s_stride = (QT == GGUF_Q4_K || QT == GGUF_Q5_K) ? n / 16
                : (QT == GGUF_Q8_0 ? n / 32 : (QT == GGUF_Q6_K ? n / 16 : 0));
  dim3 grid(ceil_div(Nout, 128), gs.max_tiles, 1);
  if (C % 64 == 0)
    qgemm_kernel<QT, DX, 128, 128, 64, NP><<<grid, 256, 0, st>>>(view(w), a.data, a.lo, a.rinv, lda, 0, Nout, C, C,
                                                                 epi, nullptr, gk);
  else
    qgemm_kernel<QT, DX, 128, 128, 32, NP><<<grid, 256, 0, st>>>(view(w), a.data, a.lo, a.rinv, lda, 0, Nout, C, C,
                                                                 epi, nullptr, gk);
  HOS_HIP_CHECK(hipGetLastError());
}

// Precision of mode 3, by the faster kernel for the launch: the integer-code kernel (mode 5) where the layout has
// codes and the direction allows it (forward, Q8_0 layout) and the launch is large — its extra block
// accumulators cost occupancy (2 waves per SIMD instead of 3 on 128×128 tiles), which the saved third of the MFMA
// work repays only from about 64 GFLOP per launch on (measured on the MI355X, M 2048: N 8192 × K 2048 −14%,
// N 2048 × K 8192 −15%, 4096³ −15%; N 9728 × K 896 +5%, 2048³ +8%) — else mode 3. Grouped (mixture-of-experts)
// launches stay mode 3 (OLMoE's expert forwards, ~100-200 GFLOP each, measured 27% slower in mode 5).
template <uint32_t QT, bool DX>
void launch_exact(const QWeight& w, H16 a, long long lda, long long M, GemmEpi epi, float* ws, size_t ws_bytes,
                  hipStream_t st) {
  if constexpr (!DX && QT == GGUF_Q8_0) {
    if (2.0 * (double)M * (double)w.rows * (double)w.cols >= 6.4e10) {
      launch_typed<QT, false, 5>(w, a, lda, M, epi, ws, ws_bytes, st);
      return;
    }
  }
  launch_typed<QT, DX, 3>(w, a, lda, M, epi, ws, ws_bytes, st);
}
template <uint32_t QT, bool DX>
void launch_exact_grouped(const QWeight& w, GroupSched gs, H16 a, long long lda, GemmEpi epi, hipStream_t st) {
  launch_typed_grouped<QT, DX, 3>(w, gs, a, lda, epi, st);
}

}  // namespace
}  // namespace hos

// Defines qgemm_launch_<NAME> and qgemm_grouped_<NAME> (declared in qgemm.hip) for one device weight layout:
// every tile shape, both directions, precision modes 1-5. One translation unit per layout keeps builds parallel.
#define HOS_QGEMM_INSTANTIATE(NAME, QT)                                                                          \
  namespace hos {                                                                                                \
  void qgemm_launch_##NAME(bool dx, int passes, const QWeight& w, H16 a, long long lda, long long M, GemmEpi epi, \
                           float* ws, size_t ws_bytes, hipStream_t st) {                                         \
    if (dx) {                                                                                                    \
      if (passes == 1) launch_typed<QT, true, 1>(w, a, lda, M, epi, ws, ws_bytes, st);                           \
      else if (passes == 2) launch_typed<QT, true, 2>(w, a, lda, M, epi, ws, ws_bytes, st);                      \
      else if (passes == 3) launch_typed<QT, true, 3>(w, a, lda, M, epi, ws, ws_bytes, st);                      \
      else if (passes == 4) launch_typed<QT, true, 4>(w, a, lda, M, epi, ws, ws_bytes, st);                      \
      else launch_exact<QT, true>(w, a, lda, M, epi, ws, ws_bytes, st);                                          \
    } else {                                                                                                     \
      if (passes == 1) launch_typed<QT, false, 1>(w, a, lda, M, epi, ws, ws_bytes, st);                          \
      else if (passes == 2) launch_typed<QT, false, 2>(w, a, lda, M, epi, ws, ws_bytes, st);                     \
      else if (passes == 3) launch_typed<QT, false, 3>(w, a, lda, M, epi, ws, ws_bytes, st);                     \
      else if (passes == 4) launch_typed<QT, false, 4>(w, a, lda, M, epi, ws, ws_bytes, st);                     \
      else launch_exact<QT, false>(w, a, lda, M, epi, ws, ws_bytes, st);                                         \
    }                                                                                                            \
  }                                                                                                              \
  void qgemm_grouped_##NAME(bool dx, int passes, const QWeight& w, GroupSched gs, H16 a, long long lda,          \
                            GemmEpi epi, hipStream_t st) {                                                       \
    if (dx) {                                                                                                    \
      if (passes == 1) launch_typed_grouped<QT, true, 1>(w, gs, a, lda, epi, st);                                \
      else if (passes == 2) launch_typed_grouped<QT, true, 2>(w, gs, a, lda, epi, st);                           \
      else if (passes == 3) launch_typed_grouped<QT, true, 3>(w, gs, a, lda, epi, st);                           \
      else if (passes == 4) launch_typed_grouped<QT, true, 4>(w, gs, a, lda, epi, st);                           \
      else launch_exact_grouped<QT, true>(w, gs, a, lda, epi, st);                                               \
    } else {                                                                                                     \
      if (passes == 1) launch_typed_grouped<QT, false, 1>(w, gs, a, lda, epi, st);                               \
      else if (passes == 2) launch_typed_grouped<QT, false, 2>(w, gs, a, lda, epi, st);                          \
      else if (passes == 3) launch_typed_grouped<QT, false, 3>(w, gs, a, lda, epi, st);                          \
      else if (passes == 4) launch_typed_grouped<QT, false, 4>(w, gs, a, lda, epi, st);                          \
      else launch_exact_grouped<QT, false>(w, gs, a, lda, epi, st);                                              \
    }                                                                                                            \
  }                                                                                                              \
  }
