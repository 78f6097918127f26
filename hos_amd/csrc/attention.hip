// Causal GQA softmax attention, forward and backward, on bf16 MFMA with hi/lo-split operands (three
// products per multiply, ~2^-16 relative, fp32 accumulation; softmax and everything elementwise in f32),
// without materialising [H, T, T].
//
// Semantics of PeftModel::forward (src/peft.rs:479-489, 530-553): scores = (q·kᵀ)·(1/√hd), the
// strictly-upper triangle masked (−1e9 there gives exactly zero probability, as skipping does),
// row softmax (src/tensor.rs:2460-2491), ctx = P·v, kv head = h / (n_heads / n_kv_heads)
// (repeat_interleave_dim0, src/tensor.rs:2819-2841). Backward = the bmm/softmax/repeat VJPs
// (src/tensor.rs:2260-2272, :2481-2490, :2831-2840) in flash form: P is recomputed from the saved
// log-sum-exp, dS = P∘(dP − rowsum(dO∘O)), and GQA gradients are summed over the group in head order.
// The scale 1/√hd is folded into q (exactly 2^-3 for hd = 64; the f32 value of 1/√128 for hd = 128).
//
// Data path. A split kernel turns the f32 q (pre-scaled, optionally rotated), k, v into bf16 hi/lo planes,
// head-major ([b][head][t][d], so a 32-row tile of one head is one contiguous 32·hd run); the backward reads
// dO from its f32 rows and splits it as it loads it, the dQ kernel forming D = rowsum(dO∘O) for the dK/dV
// kernel on the way. Every attention kernel is a workgroup of 4 waves over 128
// rows of one (head, sequence) — queries for the forward and dQ, keys for dK/dV — each wave owning 32 of them
// for the whole loop (its accumulators never leave registers, no cross-wave merge). The other axis streams
// through LDS in 32-row tiles, loaded once per workgroup with 16-byte loads and double-buffered (one barrier
// per tile), so every tile feeds four waves.
//
// MFMA layout (v_mfma_f32_32x32x16_bf16): register r of lane l holds D[i][j] with column j = l%32 and row
// i = κ(r, l/32) = 8·(r/4) + 4·(l/32) + r%4. The first product puts
// the streamed tile's rows on i (A operand: 16-byte LDS reads of row-major tiles) and this wave's own rows on j
// (B operand: held in registers), so each lane ends up owning one of its wave's rows: softmax statistics are
// per lane. The second product reads the score registers back as a B operand — register 8t+e of lane l is
// contraction slot 8·(l/32)+e of step t, i.e. streamed row κ(8t+e, l/32) — and the A operand is the streamed
// tile transposed, fetched in that same κ order with ds_read_b64_tr_b16 (two 4-row groups per step), giving
// the output transposed: Oᵀ[d][row] with the row again on the lane.
#include "fused.hpp"

namespace hos {
namespace {

constexpr int TB = 32;        // rows of one MFMA tile
constexpr int NW = 4;         // waves per workgroup
constexpr int BR = TB * NW;   // rows a workgroup owns
// Wave groups splitting the streamed axis of a workgroup. Forward: three at head dim 64 (a third of the key range
// each, 110 KB of LDS; measured 3-6% faster than two), two at 128 (three would need 204 KB). Backward: two, except
// for head dim 128, whose accumulators need more than the 256 registers two waves per SIMD leave (they spill).
#ifndef HOS_ATT_LPT
#define HOS_ATT_LPT 1
#endif
#ifndef HOS_ATT_PRIO
#define HOS_ATT_PRIO 1
#endif
// a wave's products and softmax of one streamed tile run at raised issue priority, its loads and LDS stores not
constexpr bool ATT_PRIO = HOS_ATT_PRIO;
template <int HD>
constexpr int fwd_groups() { return HD == 64 ? 3 : 2; }
template <int HD>
constexpr int bwd_groups() { return HD == 64 ? 2 : 1; }

template <int HD>
struct AC {
  static constexpr int NS = HD / 16;    // contraction steps over the head dims
  static constexpr int NC = HD / 32;    // 32-wide column tiles of one head
  static constexpr int LD = HD + 8;     // LDS row stride (bf16): 16 bytes of padding spread the row reads
  static constexpr int TILE = TB * LD;  // one plane of one 32-row tile
  static constexpr int CH = HD / 8;     // 16-byte chunks per row
};

template <int HD>
__device__ __forceinline__ float qscale() {
  return HD == 64 ? 0.125f : 0.08838834764831845f;  // 1/√128 rounded to f32
}

__device__ __forceinline__ int kap(int s, int h) { return 8 * (s >> 2) + 4 * h + (s & 3); }

// e^(x − m) as 2^(x·log2 e − m·log2 e) on the hardware exp2 (v_exp_f32, ~1 ulp; one fma for the argument):
// the exponentials are the bulk of the VALU work between two MFMA products. e^(−∞) = 0.
constexpr float LOG2E = 1.4426950408889634f;
__device__ __forceinline__ float exp_shift(float x, float m_log2e) {
  return __builtin_amdgcn_exp2f(__builtin_fmaf(x, LOG2E, -m_log2e));
}

typedef short s4v __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s4v* lds_s4;
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));  // a native vector: stays in registers

// A operand of the second product: rows κ(8t + 0..7, hl) of a row-major LDS tile, at column `col` (this lane's
// head dim), as one bf8. In a 16-lane group lane L addresses row r0 + L/4, columns c0 + 4·(L%4) .. +3, and the
// transposing read hands lane i the four rows r0 .. r0+3 of column c0 + i.
template <int HD>
__device__ __forceinline__ bf8 tr_frag(const __bf16* tile, int t, int i, int lane) {
  const int g = lane >> 4, L = lane & 15;
  const int row = 16 * t + 4 * (g >> 1) + (L >> 2);
  const int col = 32 * i + 16 * (g & 1) + 4 * (L & 3);
  const __bf16* p = tile + row * AC<HD>::LD + col;
  const s4v x0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4)(p));
  const s4v x1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4)(p + 8 * AC<HD>::LD));
  bf8 f;
  __builtin_memcpy(&f, &x0, 8);
  __builtin_memcpy((char*)&f + 8, &x1, 8);
  return f;
}

// A operand of the first product: row `lane%32` of a row-major LDS tile, head dims 16t + 8·(lane/32) .. +7.
template <int HD>
__device__ __forceinline__ bf8 row_frag(const __bf16* tile, int t, int lane) {
  return *reinterpret_cast<const bf8*>(tile + (lane & 31) * AC<HD>::LD + 16 * t + 8 * (lane >> 5));
}

// B operand of the first product from a head-major plane: row `row`, head dims 16t + 8·hl .. +7, all steps.
template <int HD>
__device__ __forceinline__ void own_frags(const __bf16* __restrict__ ph, const __bf16* __restrict__ pl, long long row,
                                          int hl, bf8* H, bf8* Lo) {
#pragma unroll
  for (int t = 0; t < AC<HD>::NS; t++) {
    H[t] = *reinterpret_cast<const bf8*>(ph + row * HD + 16 * t + 8 * hl);
    Lo[t] = *reinterpret_cast<const bf8*>(pl + row * HD + 16 * t + 8 * hl);
  }
}

// 8 consecutive f32 -> bf16 hi/lo.
__device__ __forceinline__ void split8(const float* v, float mul, bf8& H, bf8& L) {
#pragma unroll
  for (int e = 0; e < 8; e++) split_bf(v[e] * mul, H, L, e);
}

// Work item of this workgroup: (row block, head, sequence). Workgroup ids are dealt round-robin to the 8 XCDs,
// each with its own L2; remapping so that each XCD gets a contiguous run of work items keeps the row blocks of
// one head (which stream the same K/V or Q/dO tiles) and the heads of one GQA group on one L2.
struct Work {
  int xb, h, b;
};

// The causal mask makes a row block's work linear in its index. The kernels here map xb = 0 to their heaviest block
// (the forward and dQ take query block nqb - 1 - xb, dK/dV key block xb), and each XCD's run is ordered row block
// first: all its (head, sequence) items' block 0, then block 1, ... — heavy and light blocks are then dealt evenly
// over the rounds instead of every head's blocks in one stretch (bit-identical; Llama-3.2-1B's attention, 2048
// workgroups per launch, 14.3 -> 12.2 ms per step; the same run ordered lightest first measured within noise of it).
__device__ __forceinline__ Work work_item() {
  const int nwg = gridDim.x * gridDim.y * gridDim.z, full = nwg & ~7, nb = gridDim.x;
  int L = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
  if (L < full) {
    const int per = full >> 3, x = L & 7, j = L >> 3;  // XCD x, position j in its run
    if (HOS_ATT_LPT && per % nb == 0) {
      // the run covers the same (head, sequence) items as the head-major order below: rest in [x·hper, (x+1)·hper)
      const int hper = per / nb, rest = x * hper + j % hper;
      return Work{j / hper, rest % (int)gridDim.y, rest / (int)gridDim.y};
    }
    L = x * per + j;
  }
  const int rest = L / nb;
  return Work{L % nb, rest % (int)gridDim.y, rest / (int)gridDim.y};
}

// ---- split kernels ----
// q (scaled), k, v of rows [M, ld] into head-major hi/lo planes; one thread per 8 columns.
// tab set: q and k are rotated first (RoPE, the forward rotation of rope_kernel in fused.hip with the same
// separately rounded products and sums; tab holds (sin, cos) per (position, pair)), so the planes hold what
// splitting the rotated rows would give, while qkv itself is left unrotated.
template <int HD>
__global__ void attn_split_qkv(const float* __restrict__ qkv, long long ld, int kcol, int vcol, int T, int nh, int nkv,
                               long long M, __bf16* __restrict__ qh, __bf16* __restrict__ ql, __bf16* __restrict__ kh,
                               __bf16* __restrict__ kl, __bf16* __restrict__ vh, __bf16* __restrict__ vl,
                               const float2* __restrict__ tab, int neox) {
#pragma clang fp contract(off)
  const int per_row = (nh + 2 * nkv) * AC<HD>::CH;
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= M * per_row) return;
  const long long m = i / per_row;
  const int c8 = (int)(i % per_row) * 8, b = (int)(m / T), t = (int)(m % T);
  const float* src;
  __bf16 *dh, *dl;
  float mul = 1.0f;
  long long hrow;  // (b·heads + head)·T + t
  if (c8 < nh * HD) {
    src = qkv + m * ld + c8;
    dh = qh;
    dl = ql;
    mul = qscale<HD>();
    hrow = ((long long)b * nh + c8 / HD) * T + t;
  } else if (c8 < (nh + nkv) * HD) {
    const int c = c8 - nh * HD;
    src = qkv + m * ld + kcol + c;
    dh = kh;
    dl = kl;
    hrow = ((long long)b * nkv + c / HD) * T + t;
  } else {
    const int c = c8 - (nh + nkv) * HD;
    src = qkv + m * ld + vcol + c;
    dh = vh;
    dl = vl;
    hrow = ((long long)b * nkv + c / HD) * T + t;
  }
  const float4 a0 = reinterpret_cast<const float4*>(src)[0], a1 = reinterpret_cast<const float4*>(src)[1];
  float v[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
  if (tab && c8 < (nh + nkv) * HD) {
    constexpr int half = HD / 2;
    const int cc = c8 % HD;  // first head dim of this thread's 8
    const float2* tr = tab + (long long)t * half;
    float r[8];
    if (neox) {
      // pairs (i, i + half): the partner run is the 8 dims half away
      const bool lo_half = cc < half;
      const float* ps = lo_half ? src + half : src - half;
      const float4 b0 = reinterpret_cast<const float4*>(ps)[0], b1 = reinterpret_cast<const float4*>(ps)[1];
      const float w[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
#pragma unroll
      for (int e = 0; e < 8; e++) {
        const float2 sc = tr[(lo_half ? cc : cc - half) + e];
        r[e] = lo_half ? v[e] * sc.y - w[e] * sc.x : w[e] * sc.x + v[e] * sc.y;
      }
    } else {
      // adjacent pairs (2i, 2i + 1), all inside this thread's 8
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        const float2 sc = tr[(cc + e) / 2];
        r[e] = v[e] * sc.y - v[e + 1] * sc.x;
        r[e + 1] = v[e] * sc.x + v[e + 1] * sc.y;
      }
    }
#pragma unroll
    for (int e = 0; e < 8; e++) v[e] = r[e];
  }
  bf8 H, L;
  split8(v, mul, H, L);
  const long long o = hrow * HD + (c8 % HD);
  *reinterpret_cast<bf8*>(dh + o) = H;
  *reinterpret_cast<bf8*>(dl + o) = L;
}

// Cooperative load of 4 planes' 32-row tiles (rows r0 .. r0+31 of head-major planes, clamped to T-1) into
// registers, then into LDS tiles of stride LD. Thread tid moves chunk tid + 256·v of the tile set, so the plane
// and row of every chunk are compile-time functions of v plus tid.
struct Planes4 {
  const __bf16* p[4];
};
template <int HD>
struct TileLoader {
  static constexpr int PER = TB * AC<HD>::CH;   // 16-byte chunks per plane tile (256 or 512)
  static constexpr int VPP = PER / (NW * 64);   // register chunks per plane per thread
  static constexpr int NL = 4 * VPP;
  static_assert(PER % (NW * 64) == 0, "tile chunks");
  u32x4 reg[NL];
  __device__ __forceinline__ void load(const Planes4& P, long long hbase, int r0, int T, int tid) {
#pragma unroll
    for (int v = 0; v < NL; v++) {
      const int rem = (v % VPP) * NW * 64 + tid, row = rem / AC<HD>::CH, ch = rem % AC<HD>::CH;
      const int t = min(r0 + row, T - 1);
      reg[v] = *reinterpret_cast<const u32x4*>(P.p[v / VPP] + (hbase + t) * HD + 8 * ch);
    }
  }
  __device__ __forceinline__ void store(__bf16* lds, int tid) const {
#pragma unroll
    for (int v = 0; v < NL; v++) {
      const int rem = (v % VPP) * NW * 64 + tid, row = rem / AC<HD>::CH, ch = rem % AC<HD>::CH;
      *reinterpret_cast<u32x4*>(lds + (v / VPP) * AC<HD>::TILE + row * AC<HD>::LD + 8 * ch) = reg[v];
    }
  }
};

// The same for the dK/dV kernel's stream: q hi/lo from their head-major planes, dO from its f32 rows ([B·T, ldo],
// head h at column h·HD), split into hi/lo on the way into LDS (split8, the split the planes would hold).
template <int HD>
struct TileLoaderQD {
  static constexpr int PER = TB * AC<HD>::CH;
  static constexpr int VPP = PER / (NW * 64);
  u32x4 q[2 * VPP];
  float4 d[2 * VPP];  // 8 floats of dO per chunk
  __device__ __forceinline__ void load(const __bf16* qh, const __bf16* ql, const float* dout, long long ldo,
                                       long long hbase, long long rbase, int r0, int T, int tid) {
#pragma unroll
    for (int v = 0; v < VPP; v++) {
      const int rem = v * NW * 64 + tid, row = rem / AC<HD>::CH, ch = rem % AC<HD>::CH;
      const int t = min(r0 + row, T - 1);
      q[v] = *reinterpret_cast<const u32x4*>(qh + (hbase + t) * HD + 8 * ch);
      q[VPP + v] = *reinterpret_cast<const u32x4*>(ql + (hbase + t) * HD + 8 * ch);
      const float4* src = reinterpret_cast<const float4*>(dout + (rbase + t) * ldo + 8 * ch);
      d[2 * v] = src[0];
      d[2 * v + 1] = src[1];
    }
  }
  __device__ __forceinline__ void store(__bf16* lds, int tid) const {
#pragma unroll
    for (int v = 0; v < VPP; v++) {
      const int rem = v * NW * 64 + tid, row = rem / AC<HD>::CH, ch = rem % AC<HD>::CH;
      const int o = row * AC<HD>::LD + 8 * ch;
      *reinterpret_cast<u32x4*>(lds + o) = q[v];
      *reinterpret_cast<u32x4*>(lds + AC<HD>::TILE + o) = q[VPP + v];
      const float4 a = d[2 * v], b = d[2 * v + 1];
      const float x[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
      bf8 H, L;
      split8(x, 1.0f, H, L);
      *reinterpret_cast<bf8*>(lds + 2 * AC<HD>::TILE + o) = H;
      *reinterpret_cast<bf8*>(lds + 3 * AC<HD>::TILE + o) = L;
    }
  }
};

// ---- forward: a wave owns 32 queries; K and V tiles stream through LDS ----
// NG wave groups of 4 waves own the same 128 queries and split the key tiles into NG consecutive ranges (the
// causal block's last query rows need every key tile: splitting halves the longest workgroup's loop); each group
// streams its range through its own double-buffered LDS stages, and the groups' (m, l, O) merge in group order
// through LDS at the end.
template <int HD, int NG>
__global__ void __launch_bounds__(256 * NG) attn_fwd_kernel(const __bf16* __restrict__ qh, const __bf16* __restrict__ ql,
                                                            const __bf16* __restrict__ kh, const __bf16* __restrict__ kl,
                                                            const __bf16* __restrict__ vh, const __bf16* __restrict__ vl,
                                                            int T, int nh, int group, float* __restrict__ o,
                                                            long long ldo, float* __restrict__ lse) {
  using C = AC<HD>;
  __shared__ __attribute__((aligned(16))) __bf16 sm[NG][2][4 * C::TILE];  // per group, stage: Kh, Kl, Vh, Vl
  const int nqb = (T + BR - 1) / BR;
  const Work wk = work_item();
  const int qb = nqb - 1 - wk.xb, h = wk.h, b = wk.b, g = h / group, nkv = nh / group;
  const int tid = threadIdx.x, gt = tid & (NW * 64 - 1), grp = __builtin_amdgcn_readfirstlane(tid >> 8);
  const int lane = tid & 63, w = __builtin_amdgcn_readfirstlane((tid >> 6) & (NW - 1)), hl = lane >> 5,
            c = lane & 31;
  const int q0 = qb * BR + w * TB, myq = q0 + c;
  const bool active = q0 < T;
  const long long qrow0 = ((long long)b * nh + h) * T, krow0 = ((long long)b * nkv + g) * T;
  bf8 Qh[C::NS], Ql[C::NS];
  own_frags<HD>(qh, ql, qrow0 + min(myq, T - 1), hl, Qh, Ql);
  f16v O[C::NC];
#pragma unroll
  for (int i = 0; i < C::NC; i++)
#pragma unroll
    for (int r = 0; r < 16; r++) O[i][r] = 0.0f;
  float m = -INFINITY, l = 0.0f;
  const int nkb = (min(qb * BR + BR, T) - 1) / TB + 1;  // key tiles the workgroup needs
  const int per = (nkb + NG - 1) / NG, kbeg = grp * per, kend = min(nkb, kbeg + per);  // this group's range
  const int my_last = active ? (min(q0 + TB, T) - 1) / TB : -1;
  const Planes4 planes{{kh, kl, vh, vl}};
  TileLoader<HD> ld;
  ld.load(planes, krow0, min(kbeg, nkb - 1) * TB, T, gt);
  ld.store(sm[grp][0], gt);
  __syncthreads();
  for (int it = 0; it < per; it++) {
    const int kb = kbeg + it;
    const __bf16* st = sm[grp][it & 1];
    ld.load(planes, krow0, min(kb + 1, nkb - 1) * TB, T, gt);  // past the range: a harmless re-read
    if constexpr (ATT_PRIO) __builtin_amdgcn_s_setprio(1);
    if (kb < kend && kb <= my_last) {
      f16v S;
#pragma unroll
      for (int r = 0; r < 16; r++) S[r] = 0.0f;
#pragma unroll
      for (int t = 0; t < C::NS; t++)
        S = mma3_bf16(row_frag<HD>(st, t, lane), row_frag<HD>(st + C::TILE, t, lane), Qh[t], Ql[t], S);
      // S[r] = score(key k0 + κ(r, hl), query myq)
      const int k0 = kb * TB;
      float mb = -INFINITY;
      if (kb == my_last) {
#pragma unroll
        for (int r = 0; r < 16; r++) {
          const int key = k0 + kap(r, hl);
          if (key > myq || key >= T) S[r] = -INFINITY;
        }
      }
#pragma unroll
      for (int r = 0; r < 16; r++) mb = fmaxf(mb, S[r]);
      mb = fmaxf(mb, __shfl_xor(mb, 32));
      const float mn = fmaxf(m, mb), mn2 = mn * LOG2E;
      const float alpha = m == mn ? 1.0f : exp_shift(m, mn2);  // 0 while m = −∞
      float ps = 0.0f, p[16];
#pragma unroll
      for (int r = 0; r < 16; r++) {
        p[r] = exp_shift(S[r], mn2);
        ps += p[r];
      }
      ps += __shfl_xor(ps, 32);
      l = l * alpha + ps;
      m = mn;
      // rescale the running output only when some row's maximum moved (wave-uniform test)
      if (__builtin_amdgcn_ballot_w64(alpha != 1.0f)) {
#pragma unroll
        for (int i = 0; i < C::NC; i++)
#pragma unroll
          for (int r = 0; r < 16; r++) O[i][r] *= alpha;
      }
      // Oᵀ += Vᵀ·Pᵀ
#pragma unroll
      for (int t = 0; t < 2; t++) {
        bf8 ph, pl;
        split8(p + 8 * t, 1.0f, ph, pl);
#pragma unroll
        for (int i = 0; i < C::NC; i += 2)
          mma3_bf16_x2(tr_frag<HD>(st + 2 * C::TILE, t, i, lane), tr_frag<HD>(st + 3 * C::TILE, t, i, lane), ph, pl,
                       O[i], tr_frag<HD>(st + 2 * C::TILE, t, i + 1, lane), tr_frag<HD>(st + 3 * C::TILE, t, i + 1, lane),
                       ph, pl, O[i + 1]);
      }
    }
    if constexpr (ATT_PRIO) __builtin_amdgcn_s_setprio(0);
    ld.store(sm[grp][(it + 1) & 1], gt);
    __syncthreads();
  }
  if constexpr (NG > 1) {
    // groups 1.. hand (m, l, O) to group 0 through the (now free) stages; group 0 merges them in group order
    constexpr int SL = C::NC * 16 + 2;  // floats per lane
    static_assert((NG - 1) * NW * 64 * SL * 4 <= (int)sizeof(sm), "merge staging");
    float* mg = reinterpret_cast<float*>(&sm[0][0][0]);
    if (grp > 0) {
      float* d = mg + (size_t)(((grp - 1) * NW + w) * 64 + lane) * SL;
      d[0] = m;
      d[1] = l;
#pragma unroll
      for (int i = 0; i < C::NC; i++)
#pragma unroll
        for (int r = 0; r < 16; r++) d[2 + 16 * i + r] = O[i][r];
    }
    __syncthreads();
    if (grp > 0) return;
#pragma unroll
    for (int gg = 1; gg < NG; gg++) {
      const float* d = mg + (size_t)(((gg - 1) * NW + w) * 64 + lane) * SL;
      const float mo = d[0], lo = d[1], mn = fmaxf(m, mo), mn2 = mn * LOG2E;
      const float a = m == mn ? 1.0f : exp_shift(m, mn2);
      const float bo = mo == -INFINITY ? 0.0f : (mo == mn ? 1.0f : exp_shift(mo, mn2));
      l = l * a + lo * bo;
      m = mn;
#pragma unroll
      for (int i = 0; i < C::NC; i++)
#pragma unroll
        for (int r = 0; r < 16; r++) O[i][r] = O[i][r] * a + d[2 + 16 * i + r] * bo;
    }
  }
  if (!active || myq >= T) return;
  const float inv = 1.0f / l;
  float* orow = o + ((long long)b * T + myq) * ldo + h * HD;
#pragma unroll
  for (int i = 0; i < C::NC; i++)
#pragma unroll
    for (int j = 0; j < 4; j++)
      *reinterpret_cast<float4*>(orow + 32 * i + 8 * j + 4 * hl) =
          make_float4(O[i][4 * j] * inv, O[i][4 * j + 1] * inv, O[i][4 * j + 2] * inv, O[i][4 * j + 3] * inv);
  if (hl == 0) lse[((long long)b * nh + h) * T + myq] = m + logf(l);
}

// ---- dQ: a wave owns 32 queries; K and V tiles stream through LDS ----
// NG wave groups split the key tiles as in the forward; their partial dQ sums add in group order at the end.
template <int HD, int NG>
__global__ void __launch_bounds__(256 * NG) attn_dq_kernel(const __bf16* __restrict__ qh, const __bf16* __restrict__ ql,
                                                      const __bf16* __restrict__ kh, const __bf16* __restrict__ kl,
                                                      const __bf16* __restrict__ vh, const __bf16* __restrict__ vl,
                                                      const float* __restrict__ o, const float* __restrict__ dout,
                                                      long long ldo, const float* __restrict__ lse,
                                                      float* __restrict__ dvec, int T, int nh, int group,
                                                      float* __restrict__ dq, long long ldq) {
  using C = AC<HD>;
  __shared__ __attribute__((aligned(16))) __bf16 sm[NG][2][4 * C::TILE];  // per group, stage: Kh, Kl, Vh, Vl
  const int nqb = (T + BR - 1) / BR;
  const Work wk = work_item();
  const int qb = nqb - 1 - wk.xb, h = wk.h, b = wk.b, g = h / group, nkv = nh / group;
  const int tid = threadIdx.x, gt = tid & (NW * 64 - 1), grp = __builtin_amdgcn_readfirstlane(tid >> 8);
  const int lane = tid & 63, w = __builtin_amdgcn_readfirstlane((tid >> 6) & (NW - 1)), hl = lane >> 5,
            c = lane & 31;
  const int q0 = qb * BR + w * TB, myq = q0 + c;
  const bool active = q0 < T;
  const long long qrow0 = ((long long)b * nh + h) * T, krow0 = ((long long)b * nkv + g) * T;
  const long long qr = qrow0 + min(myq, T - 1);
  bf8 Qh[C::NS], Ql[C::NS], Dh[C::NS], Dl[C::NS];
  own_frags<HD>(qh, ql, qr, hl, Qh, Ql);
  // this lane's half of its query's dO row (head dims 16t + 8·hl .. +7) from the f32 rows, split to hi/lo, and
  // D = Σ_d dO·O over the row (the two half-rows of lanes c and c + 32 added)
  float Dq = 0.0f;
  {
    const long long rr = ((long long)b * T + min(myq, T - 1)) * ldo + h * HD + 8 * hl;
#pragma unroll
    for (int t = 0; t < C::NS; t++) {
      const float4* dp = reinterpret_cast<const float4*>(dout + rr + 16 * t);
      const float4* op = reinterpret_cast<const float4*>(o + rr + 16 * t);
      const float4 d0 = dp[0], d1 = dp[1], o0 = op[0], o1 = op[1];
      const float v[8] = {d0.x, d0.y, d0.z, d0.w, d1.x, d1.y, d1.z, d1.w};
      const float ov[8] = {o0.x, o0.y, o0.z, o0.w, o1.x, o1.y, o1.z, o1.w};
      split8(v, 1.0f, Dh[t], Dl[t]);
#pragma unroll
      for (int e = 0; e < 8; e++) Dq = __builtin_fmaf(v[e], ov[e], Dq);
    }
    Dq += __shfl_xor(Dq, 32);
    if (grp == 0 && hl == 0 && active && myq < T) dvec[qr] = Dq;  // for the dK/dV launch that follows
  }
  const float Lq2 = lse[qr] * LOG2E;
  f16v A[C::NC];
#pragma unroll
  for (int i = 0; i < C::NC; i++)
#pragma unroll
    for (int r = 0; r < 16; r++) A[i][r] = 0.0f;
  const int nkb = (min(qb * BR + BR, T) - 1) / TB + 1;
  const int per = (nkb + NG - 1) / NG, kbeg = grp * per, kend = min(nkb, kbeg + per);  // this group's range
  const int my_last = active ? (min(q0 + TB, T) - 1) / TB : -1;
  const Planes4 planes{{kh, kl, vh, vl}};
  TileLoader<HD> ld;
  ld.load(planes, krow0, min(kbeg, nkb - 1) * TB, T, gt);
  ld.store(sm[grp][0], gt);
  __syncthreads();
  for (int it = 0; it < per; it++) {
    const int kb = kbeg + it;
    const __bf16* st = sm[grp][it & 1];
    ld.load(planes, krow0, min(kb + 1, nkb - 1) * TB, T, gt);  // past the range: a harmless re-read
    if constexpr (ATT_PRIO) __builtin_amdgcn_s_setprio(1);
    if (kb < kend && kb <= my_last) {
      f16v S, dP;
#pragma unroll
      for (int r = 0; r < 16; r++) S[r] = dP[r] = 0.0f;
#pragma unroll
      for (int t = 0; t < C::NS; t++)
        mma3_bf16_x2(row_frag<HD>(st, t, lane), row_frag<HD>(st + C::TILE, t, lane), Qh[t], Ql[t], S,
                     row_frag<HD>(st + 2 * C::TILE, t, lane), row_frag<HD>(st + 3 * C::TILE, t, lane), Dh[t], Dl[t], dP);
      const int k0 = kb * TB;
      float ds[16];
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int key = k0 + kap(r, hl);
        const float pv = (key > myq || key >= T || myq >= T) ? 0.0f : exp_shift(S[r], Lq2);
        ds[r] = pv * (dP[r] - Dq);
      }
      // dQᵀ += Kᵀ·dSᵀ
#pragma unroll
      for (int t = 0; t < 2; t++) {
        bf8 sh, sl;
        split8(ds + 8 * t, 1.0f, sh, sl);
#pragma unroll
        for (int i = 0; i < C::NC; i += 2)
          mma3_bf16_x2(tr_frag<HD>(st, t, i, lane), tr_frag<HD>(st + C::TILE, t, i, lane), sh, sl, A[i],
                       tr_frag<HD>(st, t, i + 1, lane), tr_frag<HD>(st + C::TILE, t, i + 1, lane), sh, sl, A[i + 1]);
      }
    }
    if constexpr (ATT_PRIO) __builtin_amdgcn_s_setprio(0);
    ld.store(sm[grp][(it + 1) & 1], gt);
    __syncthreads();
  }
  if constexpr (NG > 1) {
    constexpr int SL = C::NC * 16;
    static_assert((NG - 1) * NW * 64 * SL * 4 <= (int)sizeof(sm), "merge staging");
    float* mg = reinterpret_cast<float*>(&sm[0][0][0]);
    if (grp > 0) {
      float* d = mg + (size_t)(((grp - 1) * NW + w) * 64 + lane) * SL;
#pragma unroll
      for (int i = 0; i < C::NC; i++)
#pragma unroll
        for (int r = 0; r < 16; r++) d[16 * i + r] = A[i][r];
    }
    __syncthreads();
    if (grp > 0) return;
#pragma unroll
    for (int gg = 1; gg < NG; gg++) {
      const float* d = mg + (size_t)(((gg - 1) * NW + w) * 64 + lane) * SL;
#pragma unroll
      for (int i = 0; i < C::NC; i++)
#pragma unroll
        for (int r = 0; r < 16; r++) A[i][r] += d[16 * i + r];
    }
  }
  if (!active || myq >= T) return;
  float* out = dq + ((long long)b * T + myq) * ldq + h * HD;
  const float s = qscale<HD>();
#pragma unroll
  for (int i = 0; i < C::NC; i++)
#pragma unroll
    for (int j = 0; j < 4; j++)
      *reinterpret_cast<float4*>(out + 32 * i + 8 * j + 4 * hl) =
          make_float4(A[i][4 * j] * s, A[i][4 * j + 1] * s, A[i][4 * j + 2] * s, A[i][4 * j + 3] * s);
}

// ---- dK, dV for query head h: a wave owns 32 keys; Q and dO tiles (with their LSE and D) stream through LDS.
// With group > 1 each head's result goes to part[(b·T + key)][h][2·HD] and attn_group_sum adds the group in head
// order; with group == 1 it is written in place. NG wave groups split the query tiles into consecutive ranges;
// their partial dK / dV sums add in group order at the end.
template <int HD, int NG>
__global__ void __launch_bounds__(256 * NG) attn_dkdv_kernel(const __bf16* __restrict__ qh, const __bf16* __restrict__ ql,
                                                        const __bf16* __restrict__ kh, const __bf16* __restrict__ kl,
                                                        const __bf16* __restrict__ vh, const __bf16* __restrict__ vl,
                                                        const float* __restrict__ dout, long long ldo,
                                                        const float* __restrict__ lse, const float* __restrict__ dvec,
                                                        int T, int nh, int group, float* __restrict__ dkv,
                                                        long long ldk, int kcol, int vcol, float* __restrict__ part) {
  using C = AC<HD>;
  __shared__ __attribute__((aligned(16))) __bf16 sm[NG][2][4 * C::TILE];  // per group, stage: Qh, Ql, dOh, dOl
  __shared__ float ld_s[NG][2][2][TB];  // per group, stage: LSE·log2 e, D of the tile's queries
  const Work wk = work_item();
  const int h = wk.h, b = wk.b, g = h / group, nkv = nh / group;
  const int tid = threadIdx.x, gt = tid & (NW * 64 - 1), grp = __builtin_amdgcn_readfirstlane(tid >> 8);
  const int lane = tid & 63, w = __builtin_amdgcn_readfirstlane((tid >> 6) & (NW - 1)), hl = lane >> 5,
            c = lane & 31;
  const int kw0 = wk.xb * BR + w * TB, mykey = kw0 + c;
  const bool active = kw0 < T;
  const long long qrow0 = ((long long)b * nh + h) * T, krow0 = ((long long)b * nkv + g) * T;
  bf8 Kh[C::NS], Kl[C::NS], Vh[C::NS], Vl[C::NS];
  own_frags<HD>(kh, kl, krow0 + min(mykey, T - 1), hl, Kh, Kl);
  own_frags<HD>(vh, vl, krow0 + min(mykey, T - 1), hl, Vh, Vl);
  f16v dK[C::NC], dV[C::NC];
#pragma unroll
  for (int i = 0; i < C::NC; i++)
#pragma unroll
    for (int r = 0; r < 16; r++) dK[i][r] = dV[i][r] = 0.0f;
  const int nqt = (T + TB - 1) / TB;                 // query tiles of the sequence
  const int qt0 = (wk.xb * BR) / TB;                 // the first one that sees any of the workgroup's keys
  const int my_first = active ? kw0 / TB : nqt;      // this wave's first (diagonal) query tile
  const int per = (nqt - qt0 + NG - 1) / NG, qbeg = qt0 + grp * per, qend = min(nqt, qbeg + per);  // group range
  TileLoaderQD<HD> ld;
  const float* dhead = dout + h * HD;
  const long long rrow0 = (long long)b * T;
  float ldv = 0.0f;
  auto load = [&](int qt) {
    ld.load(qh, ql, dhead, ldo, qrow0, rrow0, qt * TB, T, gt);
    if (gt < 2 * TB) {
      const long long r = qrow0 + min(qt * TB + (gt & (TB - 1)), T - 1);
      ldv = gt < TB ? lse[r] * LOG2E : dvec[r];
    }
  };
  auto store = [&](int s) {
    ld.store(sm[grp][s], gt);
    if (gt < 2 * TB) ld_s[grp][s][gt / TB][gt & (TB - 1)] = ldv;
  };
  load(min(qbeg, nqt - 1));
  store(0);
  __syncthreads();
  for (int it = 0; it < per; it++) {
    const int qt = qbeg + it;
    const int s = it & 1;
    const __bf16* st = sm[grp][s];
    load(min(qt + 1, nqt - 1));  // past the range: a harmless re-read
    if constexpr (ATT_PRIO) __builtin_amdgcn_s_setprio(1);
    if (qt < qend && qt >= my_first) {
      f16v S, dP;
#pragma unroll
      for (int r = 0; r < 16; r++) S[r] = dP[r] = 0.0f;
#pragma unroll
      for (int t = 0; t < C::NS; t++)
        mma3_bf16_x2(row_frag<HD>(st, t, lane), row_frag<HD>(st + C::TILE, t, lane), Kh[t], Kl[t], S,
                     row_frag<HD>(st + 2 * C::TILE, t, lane), row_frag<HD>(st + 3 * C::TILE, t, lane), Vh[t], Vl[t], dP);
      // S[r] = score(query q0 + κ(r, hl), key mykey); LSE and D of those queries from LDS (4 runs of 4)
      const int q0 = qt * TB;
      float Lr[16], Dr[16];
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const float4 a = *reinterpret_cast<const float4*>(&ld_s[grp][s][0][8 * j + 4 * hl]);
        const float4 d = *reinterpret_cast<const float4*>(&ld_s[grp][s][1][8 * j + 4 * hl]);
        Lr[4 * j] = a.x, Lr[4 * j + 1] = a.y, Lr[4 * j + 2] = a.z, Lr[4 * j + 3] = a.w;
        Dr[4 * j] = d.x, Dr[4 * j + 1] = d.y, Dr[4 * j + 2] = d.z, Dr[4 * j + 3] = d.w;
      }
      float p[16], ds[16];
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int q = q0 + kap(r, hl);
        const float pv = (mykey > q || q >= T || mykey >= T) ? 0.0f : exp_shift(S[r], Lr[r]);
        p[r] = pv;
        ds[r] = pv * (dP[r] - Dr[r]);
      }
      // dVᵀ += dOᵀ·P, dKᵀ += Qᵀ·dS (Q carries the scale, so this is already dK)
#pragma unroll
      for (int t = 0; t < 2; t++) {
        bf8 ph, pl, sh, sl;
        split8(p + 8 * t, 1.0f, ph, pl);
        split8(ds + 8 * t, 1.0f, sh, sl);
#pragma unroll
        for (int i = 0; i < C::NC; i++)
          mma3_bf16_x2(tr_frag<HD>(st + 2 * C::TILE, t, i, lane), tr_frag<HD>(st + 3 * C::TILE, t, i, lane), ph, pl,
                       dV[i], tr_frag<HD>(st, t, i, lane), tr_frag<HD>(st + C::TILE, t, i, lane), sh, sl, dK[i]);
      }
    }
    if constexpr (ATT_PRIO) __builtin_amdgcn_s_setprio(0);
    store(s ^ 1);
    __syncthreads();
  }
  if constexpr (NG > 1) {
    constexpr int SL = C::NC * 32;
    static_assert((NG - 1) * NW * 64 * SL * 4 <= (int)sizeof(sm), "merge staging");
    float* mg = reinterpret_cast<float*>(&sm[0][0][0]);
    if (grp > 0) {
      float* d = mg + (size_t)(((grp - 1) * NW + w) * 64 + lane) * SL;
#pragma unroll
      for (int i = 0; i < C::NC; i++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
          d[32 * i + r] = dK[i][r];
          d[32 * i + 16 + r] = dV[i][r];
        }
    }
    __syncthreads();
    if (grp > 0) return;
#pragma unroll
    for (int gg = 1; gg < NG; gg++) {
      const float* d = mg + (size_t)(((gg - 1) * NW + w) * 64 + lane) * SL;
#pragma unroll
      for (int i = 0; i < C::NC; i++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
          dK[i][r] += d[32 * i + r];
          dV[i][r] += d[32 * i + 16 + r];
        }
    }
  }
  if (!active || mykey >= T) return;
  const long long row = (long long)b * T + mykey;
  float* kr = group == 1 ? dkv + row * ldk + kcol + g * HD : part + (row * nh + h) * 2 * HD;
  float* vr = group == 1 ? dkv + row * ldk + vcol + g * HD : kr + HD;
#pragma unroll
  for (int i = 0; i < C::NC; i++)
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int d = 32 * i + 8 * j + 4 * hl;
      *reinterpret_cast<float4*>(kr + d) = make_float4(dK[i][4 * j], dK[i][4 * j + 1], dK[i][4 * j + 2], dK[i][4 * j + 3]);
      *reinterpret_cast<float4*>(vr + d) = make_float4(dV[i][4 * j], dV[i][4 * j + 1], dV[i][4 * j + 2], dV[i][4 * j + 3]);
    }
}

// dK/dV of kv head g = Σ over its group's heads, in head order (deterministic).
template <int HD>
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

// Plane pointers inside the caller's scratch: q, k, v, each hi then lo.
struct Planes {
  __bf16 *qh, *ql, *kh, *kl, *vh, *vl;
};
Planes planes_of(void* scratch, int B, int T, int nh, int nkv, int hd) {
  const long long nq = (long long)B * nh * T * hd, nk = (long long)B * nkv * T * hd;
  __bf16* p = (__bf16*)scratch;
  Planes P;
  P.qh = p;
  P.ql = P.qh + nq;
  P.kh = P.ql + nq;
  P.kl = P.kh + nk;
  P.vh = P.kl + nk;
  P.vl = P.vh + nk;
  return P;
}

void check_layout(long long ld, int kcol, int vcol, int hd, const void* scratch) {
  HOS_REQUIRE(hd == 64 || hd == 128, HOS_E_INVALID, "attention: head_dim must be 64 or 128");
  HOS_REQUIRE(ld % 4 == 0 && kcol % 4 == 0 && vcol % 4 == 0, HOS_E_INVALID, "attention: unaligned qkv layout");
  HOS_REQUIRE(scratch != nullptr && ((uintptr_t)scratch & 15) == 0, HOS_E_INVALID, "attention: no plane scratch");
}

template <int HD>
void split_qkv(const float* qkv, long long ld, int kcol, int vcol, int B, int T, int nh, int nkv, const Planes& P,
               hipStream_t st, const float2* rope_tab = nullptr, bool rope_neox = false) {
  const long long M = (long long)B * T, n = M * (nh + 2 * nkv) * AC<HD>::CH;
  attn_split_qkv<HD><<<ceil_div(n, 256), 256, 0, st>>>(qkv, ld, kcol, vcol, T, nh, nkv, M, P.qh, P.ql, P.kh, P.kl,
                                                       P.vh, P.vl, rope_tab, rope_neox ? 1 : 0);
  HOS_HIP_CHECK(hipGetLastError());
}

template <int HD>
void attn_fwd_hd(const float* qkv, long long ld, int kcol, int vcol, int B, int T, int nh, int nkv, float* o,
                 long long ldo, float* lse, void* scratch, hipStream_t st, const float2* rope_tab, bool rope_neox) {
  const Planes P = planes_of(scratch, B, T, nh, nkv, HD);
  split_qkv<HD>(qkv, ld, kcol, vcol, B, T, nh, nkv, P, st, rope_tab, rope_neox);
  dim3 grid(ceil_div(T, BR), nh, B);
  constexpr int NGF = fwd_groups<HD>();
  attn_fwd_kernel<HD, NGF><<<grid, 256 * NGF, 0, st>>>(P.qh, P.ql, P.kh, P.kl, P.vh, P.vl, T, nh, nh / nkv, o,
                                                             ldo, lse);
  HOS_HIP_CHECK(hipGetLastError());
}

template <int HD>
void attn_bwd_hd(const float* qkv, long long ld, int kcol, int vcol, const float* o, const float* dout, long long ldo,
                 const float* lse, float* dvec, int B, int T, int nh, int nkv, float* dqkv, long long ldd, float* part,
                 void* scratch, hipStream_t st, bool qkv_planes, bool defer_group_sum) {
  const Planes P = planes_of(scratch, B, T, nh, nkv, HD);
  if (!qkv_planes) split_qkv<HD>(qkv, ld, kcol, vcol, B, T, nh, nkv, P, st);
  // dO is read from its f32 rows by both kernels (split to hi/lo as it is loaded); the dQ launch also forms
  // D = rowsum(dO∘O) for its queries and leaves it in dvec for the dK/dV launch
  dim3 grid(ceil_div(T, BR), nh, B);
  constexpr int NGB = bwd_groups<HD>();
  attn_dq_kernel<HD, NGB><<<grid, 256 * NGB, 0, st>>>(P.qh, P.ql, P.kh, P.kl, P.vh, P.vl, o, dout, ldo, lse, dvec,
                                                            T, nh, nh / nkv, dqkv, ldd);
  HOS_HIP_CHECK(hipGetLastError());
  attn_dkdv_kernel<HD, NGB><<<grid, 256 * NGB, 0, st>>>(P.qh, P.ql, P.kh, P.kl, P.vh, P.vl, dout, ldo, lse,
                                                              dvec, T, nh, nh / nkv, dqkv, ldd, kcol, vcol, part);
  HOS_HIP_CHECK(hipGetLastError());
  if (nh != nkv && !defer_group_sum) {
    long long ne = (long long)B * T * nkv * 2 * HD;
    attn_group_sum<HD><<<ceil_div(ne, 256), 256, 0, st>>>(part, B * T, nh, nkv, nh / nkv, dqkv, ldd, kcol, vcol);
    HOS_HIP_CHECK(hipGetLastError());
  }
}

}  // namespace

size_t attn_scratch_bytes(int B, int T, int nh, int nkv, int hd) {
  return (size_t)B * T * hd * ((size_t)nh + 2 * (size_t)nkv) * 2 * sizeof(__bf16);
}

void launch_attn_fwd(const float* qkv, long long ld, int kcol, int vcol, int B, int T, int nh, int nkv, int hd,
                     float* o, long long ldo, float* lse, void* scratch, hipStream_t st, const float2* rope_tab,
                     bool rope_neox) {
  check_layout(ld, kcol, vcol, hd, scratch);
  HOS_REQUIRE(ldo % 4 == 0 && nkv > 0 && nh % nkv == 0, HOS_E_INVALID, "attention: bad output layout or heads");
  if (B <= 0 || T <= 0) return;
  if (hd == 64)
    attn_fwd_hd<64>(qkv, ld, kcol, vcol, B, T, nh, nkv, o, ldo, lse, scratch, st, rope_tab, rope_neox);
  else
    attn_fwd_hd<128>(qkv, ld, kcol, vcol, B, T, nh, nkv, o, ldo, lse, scratch, st, rope_tab, rope_neox);
}

void launch_attn_bwd(const float* qkv, long long ld, int kcol, int vcol, const float* o, const float* dout,
                     long long ldo, const float* lse, float* dvec, int B, int T, int nh, int nkv, int hd, float* dqkv,
                     long long ldd, float* part, void* scratch, hipStream_t st, bool qkv_planes,
                     bool defer_group_sum) {
  check_layout(ld, kcol, vcol, hd, scratch);
  HOS_REQUIRE(nh == nkv || part != nullptr, HOS_E_INVALID, "attention: GQA backward needs a partial buffer");
  HOS_REQUIRE(ldo % 4 == 0 && ldd % 4 == 0 && nkv > 0 && nh % nkv == 0, HOS_E_INVALID, "attention: unaligned layout");
  if (B <= 0 || T <= 0) return;
  if (hd == 64)
    attn_bwd_hd<64>(qkv, ld, kcol, vcol, o, dout, ldo, lse, dvec, B, T, nh, nkv, dqkv, ldd, part, scratch, st,
                    qkv_planes, defer_group_sum);
  else
    attn_bwd_hd<128>(qkv, ld, kcol, vcol, o, dout, ldo, lse, dvec, B, T, nh, nkv, dqkv, ldd, part, scratch, st,
                     qkv_planes, defer_group_sum);
}

}  // namespace hos
