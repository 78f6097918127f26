// LoRA factor GEMMs on fp32 MFMA (v_mfma_f32_16x16x4f32), shaped for the skinny products of a
// rank-r adapter (src/peft.rs:508-512 forward; the matmul VJPs of src/tensor.rs:340-391 backward):
//
//   rows:  C[M, n]  = α · X[M, K] · Bᵀ        x·A (down-projection), s·dy·Bᵀ (du)
//   cols:  C(j, c)  = α · Σ_m S[m, j] · G[m, c]   s·uᵀ·dy (dB), xᵀ·du (dA)
//
// One side is the adapter rank (n or j ≤ 96), the other a full activation [M, K] read once from HBM,
// so both kernels are bandwidth-bound: the big operand is streamed with 16-byte loads, the small one
// is read from L2. The contraction order inside an MFMA is free, so a lane's float4 of 4 consecutive
// k (rows kernel) or 4 consecutive output columns (cols kernel) feeds 4 MFMAs directly.
//
// Short rows contractions run in one launch (16 waves per workgroup split K; see lora_rows_wide_kernel).
// The long contraction is split across workgroups for parallelism. Each workgroup reduces its four
// waves in LDS in a fixed order and writes its partial block; a reduce launch sums the partials in
// split order. Deterministic. (An in-kernel "last workgroup reduces" variant with device-scope fences
// measured 3-4x slower here: every release fence writes back the XCD's L2.)
#include <algorithm>
#include <cstdlib>
#include <vector>

#include "lora.hpp"

namespace hos {
namespace {

typedef _Float16 h4v __attribute__((ext_vector_type(4)));
// Four consecutive values of an activation row: f32, or the fp16 operand's hi + lo (exact in f32; the row's rinv is
// applied by the caller).
__device__ __forceinline__ float4 load4h(const HIn& xh, long long off) {
  const h4v a = *reinterpret_cast<const h4v*>(xh.hi + off), b = *reinterpret_cast<const h4v*>(xh.lo + off);
  return make_float4((float)a.x + (float)b.x, (float)a.y + (float)b.y, (float)a.z + (float)b.z,
                     (float)a.w + (float)b.w);
}
__device__ __forceinline__ float4 load4(const float* xf, const HIn& xh, long long off) {
  return xh.hi ? load4h(xh, off) : *reinterpret_cast<const float4*>(xf + off);
}

__device__ __forceinline__ f4v mfma16(float a, float b, f4v c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Four waves hold partial sums of the same E-element block (element ids given by pos()). Sum them in
// the fixed order (w0 + w2) + (w1 + w3) through a [2][E] LDS buffer; the result lands in red[0][·].
template <int NV, class Pos>
__device__ __forceinline__ void wave_reduce(float (&v)[NV], float* red, int E, Pos pos) {
  const int wave = threadIdx.x >> 6;
  if (wave >= 2)
#pragma unroll
    for (int i = 0; i < NV; i++) red[(wave - 2) * E + pos(i)] = v[i];
  __syncthreads();
  if (wave < 2)
#pragma unroll
    for (int i = 0; i < NV; i++) v[i] += red[wave * E + pos(i)];
  __syncthreads();
  if (wave == 1)
#pragma unroll
    for (int i = 0; i < NV; i++) red[pos(i)] = v[i];
  __syncthreads();
  if (wave == 0)
#pragma unroll
    for (int i = 0; i < NV; i++) red[pos(i)] += v[i];
  __syncthreads();
}

// Sum of the S partials of element e of block bx, in split order (4 loads in flight).
__device__ __forceinline__ float sum_parts(const float* part, int S, int gx, int bx, int E, int e) {
  const long long stride = (long long)gx * E;
  const float* p = part + (long long)bx * E + e;
  float v = 0.0f;
  int s = 0;
  for (; s + 4 <= S; s += 4) {
    float a0 = p[s * stride], a1 = p[(s + 1) * stride], a2 = p[(s + 2) * stride], a3 = p[(s + 3) * stride];
    v += a0;
    v += a1;
    v += a2;
    v += a3;
  }
  for (; s < S; s++) v += p[s * stride];
  return v;
}

// ---------------- rows: C[M, n] = α·X·Bᵀ ----------------
// Workgroup: 16·RT rows × all n columns × a k-chunk; wave w takes the chunk's 16-wide k steps w, w+4, …
// Lane (q = lane/16, p = lane%16): rows m0+16t+p, k-slot q (k = step + 4q .. +3 as one float4).
#ifndef HOS_ROWS_UNROLL
#define HOS_ROWS_UNROLL 2
#endif
#ifndef HOS_COLS_UNROLL
#define HOS_COLS_UNROLL 4
#endif

// One rows product of a launch (a launch takes one or two: blockIdx.z picks the job; a job split into S
// contraction chunks writes its partials to part, [chunk][row block][E], for lora_rows_reduce).
struct RowsJobK {
  int K, kchunk, S;
  float alpha;
  const float* X;
  long long ldx;
  const float* Bt;
  long long ldb;
  RowsSeg sg;
  float* C;
  long long ldc;
  float* part;
};
template <int NJ, int RT = 2>
__global__ void __launch_bounds__(256) lora_rows_kernel(int M, RowsJobK j0, RowsJobK j1, HIn xh) {
  const RowsJobK& jb = blockIdx.z ? j1 : j0;
  if ((int)blockIdx.y >= jb.S) return;
  const int K = jb.K, kchunk = jb.kchunk;
  const float* __restrict__ X = jb.X;
  const float* __restrict__ Bt = jb.Bt;
  const long long ldx = jb.ldx, ldb = jb.ldb;
  const RowsSeg& sg = jb.sg;
  constexpr int NC = NJ * 16, E = 16 * RT * NC;
  __shared__ float red[2 * E];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, q = lane >> 4, p = lane & 15;
  const int m0 = blockIdx.x * 16 * RT;
  const int kb = blockIdx.y * kchunk, ke = min(K, kb + kchunk);
  const int n = sg.nt * sg.r;

  const float* bp[NJ];
  int klo[NJ], khi[NJ];
#pragma unroll
  for (int jt = 0; jt < NJ; jt++) {
    const int j = jt * 16 + p;
    if (j < n) {
      const int t = j / sg.r, jj = j - t * sg.r;
      bp[jt] = Bt + sg.boff[t] + (long long)jj * ldb - sg.kbeg[t];
      klo[jt] = sg.kbeg[t];
      khi[jt] = sg.kend[t];
    } else {
      bp[jt] = Bt;
      klo[jt] = 0;
      khi[jt] = 0;
    }
  }
  long long xr[RT];  // row offsets (elements)
  bool rv[RT];
#pragma unroll
  for (int t = 0; t < RT; t++) {
    const int row = m0 + 16 * t + p;
    rv[t] = row < M;
    xr[t] = (long long)(rv[t] ? row : 0) * ldx;
  }

  f4v acc[RT][NJ];
#pragma unroll
  for (int t = 0; t < RT; t++)
#pragma unroll
    for (int jt = 0; jt < NJ; jt++) acc[t][jt] = f4v{0.0f, 0.0f, 0.0f, 0.0f};

  // HOS_ROWS_UNROLL k steps per trip, every load issued before the MFMAs that use them (the compiler does not
  // unroll a loop around convergent MFMA builtins with a runtime trip count). Out-of-range steps load zeros and
  // add exact zeros: each accumulator sums the same products in the same order as one step per trip.
  constexpr int U = HOS_ROWS_UNROLL;
  for (int k0 = kb + 16 * wave; k0 < ke; k0 += 64 * U) {
    float4 xa[U][RT], bv[U][NJ];
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int kk = k0 + 64 * u + 4 * q;
      const bool kin = kk < ke;
#pragma unroll
      for (int t = 0; t < RT; t++)
        xa[u][t] = (rv[t] && kin) ? load4(X, xh, xr[t] + kk) : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
      for (int jt = 0; jt < NJ; jt++)
        bv[u][jt] = (kin && kk >= klo[jt] && kk < khi[jt]) ? *reinterpret_cast<const float4*>(bp[jt] + kk)
                                                           : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int u = 0; u < U; u++)
      if (k0 + 64 * u < ke)  // wave-uniform
#pragma unroll
      for (int t = 0; t < RT; t++)
#pragma unroll
        for (int jt = 0; jt < NJ; jt++) {
          acc[t][jt] = mfma16(xa[u][t].x, bv[u][jt].x, acc[t][jt]);
          acc[t][jt] = mfma16(xa[u][t].y, bv[u][jt].y, acc[t][jt]);
          acc[t][jt] = mfma16(xa[u][t].z, bv[u][jt].z, acc[t][jt]);
          acc[t][jt] = mfma16(xa[u][t].w, bv[u][jt].w, acc[t][jt]);
        }
  }

  if (xh.hi)  // the operand's row scale: element i of tile t is row m0 + 16t + 4q + i
#pragma unroll
    for (int t = 0; t < RT; t++)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int row = m0 + 16 * t + 4 * q + i;
        const float ri = row < M ? xh.rinv[row] : 0.0f;
#pragma unroll
        for (int jt = 0; jt < NJ; jt++) acc[t][jt][i] *= ri;
      }
  // flatten: element (row 16t+4q+i, col 16jt+p) of the 32×NC block
  float v[RT * NJ * 4];
#pragma unroll
  for (int t = 0; t < RT; t++)
#pragma unroll
    for (int jt = 0; jt < NJ; jt++)
#pragma unroll
      for (int i = 0; i < 4; i++) v[(t * NJ + jt) * 4 + i] = acc[t][jt][i];
  wave_reduce(v, red, E, [&](int idx) {
    const int i = idx & 3, tj = idx >> 2, t = tj / NJ, jt = tj % NJ;
    return (16 * t + 4 * q + i) * NC + 16 * jt + p;
  });
  if (jb.S == 1) {
    for (int e = threadIdx.x; e < E; e += 256) {
      const int rr = e / NC, c = e % NC, row = m0 + rr;
      if (row < M && c < n) jb.C[(long long)row * jb.ldc + c] = jb.alpha * red[e];
    }
    return;
  }
  float* mine = jb.part + ((long long)blockIdx.y * gridDim.x + blockIdx.x) * E;
  for (int e = threadIdx.x; e < E; e += 256) mine[e] = red[e];
}

// Short contractions (K <= ROWS_WIDE_KMAX): one 16-row × 16·NJ-column block per workgroup of 16 waves, the waves
// splitting K (wave w takes the 16-wide k steps w, w+16, …), their partial tiles summed in LDS in wave order.
// No split over workgroups, so no partial buffer and no reduction launch; deterministic.
constexpr int ROWS_WIDE_KMAX = 1536, ROWS_WIDE_NW = 16;
template <int NJ>
__global__ void __launch_bounds__(64 * ROWS_WIDE_NW) lora_rows_wide_kernel(int M, int K, float alpha,
                                                                           const float* __restrict__ X, long long ldx,
                                                                           const float* __restrict__ Bt, long long ldb,
                                                                           RowsSeg sg, float* __restrict__ C,
                                                                           long long ldc, HIn xh) {
  constexpr int NW = ROWS_WIDE_NW, NC = NJ * 16, E = 16 * NC, U = 2;
  __shared__ float red[NW * E];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, q = lane >> 4, p = lane & 15;
  const int m0 = blockIdx.x * 16, n = sg.nt * sg.r, j0 = blockIdx.y * NC;  // this workgroup's column tiles
  const float* bp[NJ];
  int klo[NJ], khi[NJ];
#pragma unroll
  for (int jt = 0; jt < NJ; jt++) {
    const int j = j0 + jt * 16 + p;
    if (j < n) {
      const int t = j / sg.r, jj = j - t * sg.r;
      bp[jt] = Bt + sg.boff[t] + (long long)jj * ldb - sg.kbeg[t];
      klo[jt] = sg.kbeg[t];
      khi[jt] = sg.kend[t];
    } else {
      bp[jt] = Bt;
      klo[jt] = 0;
      khi[jt] = 0;
    }
  }
  const int row = m0 + p;
  const bool rv = row < M;
  const long long xr = (long long)(rv ? row : 0) * ldx;
  f4v acc[NJ];
#pragma unroll
  for (int jt = 0; jt < NJ; jt++) acc[jt] = f4v{0.0f, 0.0f, 0.0f, 0.0f};
  // U steps per trip, loads first (zero steps past K add exact zeros)
  for (int k0 = 16 * wave; k0 < K; k0 += 16 * NW * U) {
    float4 xa[U], bv[U][NJ];
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int kk = k0 + 16 * NW * u + 4 * q;
      const bool kin = kk < K;
      xa[u] = (rv && kin) ? load4(X, xh, xr + kk) : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
      for (int jt = 0; jt < NJ; jt++)
        bv[u][jt] = (kin && kk >= klo[jt] && kk < khi[jt]) ? *reinterpret_cast<const float4*>(bp[jt] + kk)
                                                           : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int u = 0; u < U; u++)
      if (k0 + 16 * NW * u < K)  // wave-uniform
#pragma unroll
        for (int jt = 0; jt < NJ; jt++) {
          acc[jt] = mfma16(xa[u].x, bv[u][jt].x, acc[jt]);
          acc[jt] = mfma16(xa[u].y, bv[u][jt].y, acc[jt]);
          acc[jt] = mfma16(xa[u].z, bv[u][jt].z, acc[jt]);
          acc[jt] = mfma16(xa[u].w, bv[u][jt].w, acc[jt]);
        }
  }
  if (xh.hi)  // the operand's row scale: element i is row m0 + 4q + i
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int r2 = m0 + 4 * q + i;
      const float ri = r2 < M ? xh.rinv[r2] : 0.0f;
#pragma unroll
      for (int jt = 0; jt < NJ; jt++) acc[jt][i] *= ri;
    }
  // element (row 4q+i, col 16jt+p) of the 16×NC block
#pragma unroll
  for (int jt = 0; jt < NJ; jt++)
#pragma unroll
    for (int i = 0; i < 4; i++) red[wave * E + (4 * q + i) * NC + 16 * jt + p] = acc[jt][i];
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += 64 * NW) {
    float v = 0.0f;
    for (int w = 0; w < NW; w++) v += red[w * E + e];
    const int rr = e / NC, c = j0 + e % NC, r2 = m0 + rr;
    if (r2 < M && c < n) C[(long long)r2 * ldc + c] = alpha * v;
  }
}

// ---------------- cols: C(j, c) = α·Σ_m S[m, j]·G[m, c] ----------------
// Workgroup: 64 columns of one segment × all j × an m-chunk; wave w takes the chunk's 4-row steps
// w, w+4, … Lane (q, p): m = step + q, columns c0+4p .. +3 (one float4; component e is MFMA tile e).
// bx: the workgroup's column block within its job; red: LDS of at least 2·NS·16·64 floats.
// CW = 8 (GH only): a lane takes 8 consecutive columns (16-byte loads of each plane, 8 MFMA tiles), the block is
// 128 columns wide.
template <int NS, bool GH, int CW = 4, int U = HOS_COLS_UNROLL>
__device__ __forceinline__ void cols_body(const ColsJobDev& jb, int bx, int M, int mchunk, float* red, float* part) {
  static_assert(CW == 4 || (CW == 8 && GH), "column run");
  constexpr int BW = 16 * CW, NJR = NS * 16, E = NJR * BW;
  const ColsSeg& sg = jb.sg;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, q = lane >> 4, p = lane & 15;
  int t = 0;
#pragma unroll
  for (int i = 1; i < 4; i++)
    if (i < sg.nseg && bx >= sg.blk0[i]) t = i;
  const int c0 = (bx - sg.blk0[t]) * BW, len = sg.len[t];
  const int mb = blockIdx.y * mchunk, me = min(M, mb + mchunk);
  const bool cv = c0 + CW * p < len;
  const long long gcol = sg.gbeg[t] + c0 + CW * p;
  const float* scol = jb.Sm + sg.soff[t];
  const long long lds = jb.lds, ldg = jb.ldg;
  const int ns = jb.ns;

  f4v acc[NS][CW];
#pragma unroll
  for (int js = 0; js < NS; js++)
#pragma unroll
    for (int e = 0; e < CW; e++) acc[js][e] = f4v{0.0f, 0.0f, 0.0f, 0.0f};

  // U 4-row steps per trip, loads first (as in the rows kernel; zero steps past the end add
  // exact zeros, so the summation order per accumulator is that of one step per trip).
  for (int m40 = mb + 4 * wave; m40 < me; m40 += 16 * U) {
    float g[U][CW];
    float s[U][NS];
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int m = m40 + 16 * u + q;
      const bool mv = m < me;
      // G given as the fp16 operand (GH): its row scale joins S (Σ_m S[m,j]·rinv[m]·(hi+lo)[m,c])
      float ri = 1.0f;
      if constexpr (CW == 8) {
        const long long off = gcol + (long long)m * ldg;
        const h8 zh = {};
        const h8 a = (mv && cv) ? *reinterpret_cast<const h8*>(jb.gh.hi + off) : zh;
        const h8 b = (mv && cv) ? *reinterpret_cast<const h8*>(jb.gh.lo + off) : zh;
#pragma unroll
        for (int e = 0; e < 8; e++) g[u][e] = (float)a[e] + (float)b[e];
        ri = mv ? jb.gh.rinv[m] : 0.0f;
      } else {
        float4 x;
        if constexpr (GH) {
          x = (mv && cv) ? load4h(jb.gh, gcol + (long long)m * ldg) : make_float4(0.f, 0.f, 0.f, 0.f);
          ri = mv ? jb.gh.rinv[m] : 0.0f;
        } else {
          x = (mv && cv) ? *reinterpret_cast<const float4*>(jb.Gm + gcol + (long long)m * ldg)
                         : make_float4(0.f, 0.f, 0.f, 0.f);
        }
        g[u][0] = x.x;
        g[u][1] = x.y;
        g[u][2] = x.z;
        g[u][3] = x.w;
      }
#pragma unroll
      for (int js = 0; js < NS; js++) {
        const int j = js * 16 + p;
        s[u][js] = (mv && j < ns) ? scol[(long long)m * lds + j] * ri : 0.0f;
      }
    }
#pragma unroll
    for (int u = 0; u < U; u++)
      if (m40 + 16 * u < me)  // wave-uniform
#pragma unroll
      for (int js = 0; js < NS; js++)
#pragma unroll
        for (int e = 0; e < CW; e++) acc[js][e] = mfma16(s[u][js], g[u][e], acc[js][e]);
  }

  // flatten: element (j = 16js+4q+i, column CW·p+e) of the NJR×BW block
  float v[NS * 4 * CW];
#pragma unroll
  for (int js = 0; js < NS; js++)
#pragma unroll
    for (int e = 0; e < CW; e++)
#pragma unroll
      for (int i = 0; i < 4; i++) v[(js * CW + e) * 4 + i] = acc[js][e][i];
  wave_reduce(v, red, E, [&](int idx) {
    const int i = idx & 3, e = (idx >> 2) % CW, js = idx / (4 * CW);
    return (16 * js + 4 * q + i) * BW + CW * p + e;
  });
  if (gridDim.y == 1) {
    const long long ocol = sg.ocol[t];
    for (int e = threadIdx.x; e < E; e += 256) {
      const int j = e / BW, c = c0 + e % BW;
      if (j < ns && c < len) jb.C[(long long)j * jb.scj + (ocol + c) * jb.scc] = jb.alpha * red[e];
    }
    return;
  }
  // this split's partial of the block: job region, then [split][block][E]
  float* mine = part + jb.part_off + ((long long)blockIdx.y * jb.gx + bx) * E;
  for (int e = threadIdx.x; e < E; e += 256) mine[e] = red[e];
}

// Two independent jobs over the same contraction length in one launch: workgroups [0, b.bx0) run job a with
// NSA row tiles, the rest job b with NSB. A single job passes b with bx0 = the grid width. GHA: job a reads G
// as the fp16 operand (job b never does).
template <int NSA, int NSB, bool GHA, int CWA = 4>
__global__ void __launch_bounds__(256) lora_cols_kernel(int M, int mchunk, ColsJobDev a, ColsJobDev b, float* part) {
  constexpr int EA = NSA * 16 * 16 * CWA, EB = NSB * 16 * 64, EMAX = EA > EB ? EA : EB;
  __shared__ float red[2 * EMAX];
  if ((int)blockIdx.x < b.bx0)
    cols_body<NSA, GHA, CWA>(a, (int)blockIdx.x, M, mchunk, red, part);
  else
    cols_body<NSB, false>(b, (int)blockIdx.x - b.bx0, M, mchunk, red, part);
}

// Independent jobs of one kernel shape (NS row tiles, G as f32 or as the fp16 operand in CW-column runs) from a
// device-resident table in one launch, each over all M rows in one workgroup per column block — no split of M, so no
// partials and no reduction launch: the training step's dA / dB products of every layer, queued during the backward
// and run together after it. Workgroup b runs job j with start[j] <= b < start[j + 1] (binary search). U: 4-row steps
// per trip (more loads in flight for the long all-rows loops of large M).
template <int NS, bool GH, int CW, int U>
__global__ void __launch_bounds__(256) lora_cols_table_kernel(int M, const ColsJobDev* __restrict__ jobs,
                                                              const int* __restrict__ start, int n) {
  __shared__ float red[2 * NS * 16 * 16 * CW];
  int lo = 0, hi = n - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if ((int)blockIdx.x >= start[mid]) lo = mid;
    else hi = mid - 1;
  }
  const ColsJobDev jb = jobs[lo];
  cols_body<NS, GH, CW, U>(jb, (int)blockIdx.x - start[lo], M, M, red, nullptr);
}

// Separate-launch reductions of the partials (one thread per output element of every block); blockIdx.y picks
// the job of a two-job rows launch, a job with S = 1 wrote its output itself.
struct RowsRed {
  const float* part;
  int S;
  float alpha;
  float* C;
  long long ldc;
};
__global__ void lora_rows_reduce(int gx, int RB, int NC, int M, int n, RowsRed r0, RowsRed r1) {
  const RowsRed& rd = blockIdx.y ? r1 : r0;
  if (rd.S <= 1) return;
  const int E = RB * NC;
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long long)gx * E) return;
  const int bx = (int)(i / E), e = (int)(i % E), rr = e / NC, c = e % NC, row = bx * RB + rr;
  if (row >= M || c >= n) return;
  rd.C[(long long)row * rd.ldc + c] = rd.alpha * sum_parts(rd.part, rd.S, gx, bx, E, e);
}
// One thread per output element of every block of both jobs (job a's elements first).
__device__ __forceinline__ void cols_reduce_one(const ColsJobDev& jb, const float* part, int S, long long i) {
  const int E = jb.nsr * jb.bw;
  const int bx = (int)(i / E), e = (int)(i % E);
  const ColsSeg& sg = jb.sg;
  int t = 0;
  for (int k = 1; k < sg.nseg; k++)
    if (bx >= sg.blk0[k]) t = k;
  const int j = e / jb.bw, c = (bx - sg.blk0[t]) * jb.bw + e % jb.bw;
  if (j >= jb.ns || c >= sg.len[t]) return;
  jb.C[(long long)j * jb.scj + ((long long)sg.ocol[t] + c) * jb.scc] =
      jb.alpha * sum_parts(part + jb.part_off, S, jb.gx, bx, E, e);
}
struct ColsBatchArgs {
  ColsJobDev jobs[8];
  long long start[9];  // first element of each job in the flattened index space
  int n;
};
__global__ void lora_cols_reduce_batch(const float* __restrict__ base, ColsBatchArgs args) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= args.start[args.n]) return;
  int j = 0;
  while (j + 1 < args.n && i >= args.start[j + 1]) j++;
  cols_reduce_one(args.jobs[j], base, args.jobs[j].S, i - args.start[j]);
}
__global__ void lora_cols_reduce(const float* __restrict__ part, int S, ColsJobDev a, ColsJobDev b) {
  const long long na = (long long)a.gx * a.nsr * a.bw, nb = (long long)b.gx * b.nsr * b.bw;
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < na)
    cols_reduce_one(a, part, S, i);
  else if (i < na + nb)
    cols_reduce_one(b, part, S, i - na);
}


// ---------------- rows on fp16 MFMA ----------------
// C[M, n] = α·rinv[m]·Σ_k (Xh + Xl)[m, k]·(Bh + Bl)(j, k)·sc(j), dropping Xl·Bl (~2^-22): v_mfma_f32_16x16x32_f16,
// one 16-row block × all n columns per workgroup of 16 waves splitting the contraction in 32-deep steps (wave w
// takes steps w, w+16, …), their tiles summed in LDS in wave order; long contractions are also split over
// workgroups (partials reduced by lora_rows_reduce). Lane (q = lane/16, p = lane%16): A row p, B column p, k 8q .. +7.
constexpr int R16_NW = 16;
typedef _Float16 h8l __attribute__((ext_vector_type(8)));
template <int NJ, int RT>
__global__ void __launch_bounds__(64 * R16_NW) lora_rows16_kernel(int M, int K, int kchunk, float alpha, HIn xh,
                                                                  long long ldx, B16 bt, long long ldb, RowsSeg sg,
                                                                  float* __restrict__ C, long long ldc, float* part) {
  constexpr int NC = NJ * 16, E = 16 * RT * NC;
  __shared__ float red[R16_NW * E];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, q = lane >> 4, p = lane & 15;
  const int m0 = blockIdx.x * 16 * RT, n = sg.nt * sg.r;
  const int kb = blockIdx.y * kchunk, ke = min(K, kb + kchunk);
  long long bbase[NJ];
  int klo[NJ], khi[NJ];
  float bsc[NJ];
#pragma unroll
  for (int jt = 0; jt < NJ; jt++) {
    const int j = jt * 16 + p;
    if (j < n) {
      const int t = j / sg.r, jj = j - t * sg.r;
      bbase[jt] = sg.boff[t] + (long long)jj * ldb - sg.kbeg[t];
      klo[jt] = sg.kbeg[t];
      khi[jt] = sg.kend[t];
      bsc[jt] = bt.sc[sg.boff[t] / ldb + jj];
    } else {
      bbase[jt] = 0;
      klo[jt] = khi[jt] = 0;
      bsc[jt] = 0.0f;
    }
  }
  bool rv[RT];
  long long xr[RT];
#pragma unroll
  for (int t = 0; t < RT; t++) {
    const int row = m0 + 16 * t + p;
    rv[t] = row < M;
    xr[t] = (long long)(rv[t] ? row : 0) * ldx;
  }
  f4v acc[RT][NJ];
#pragma unroll
  for (int t = 0; t < RT; t++)
#pragma unroll
    for (int jt = 0; jt < NJ; jt++) acc[t][jt] = f4v{0.0f, 0.0f, 0.0f, 0.0f};
  const h8l z8 = {};
  constexpr int U = NJ * RT <= 2 ? 2 : 1;  // steps per trip, loads first (steps past the end add exact zeros)
  for (int k0 = kb + 32 * wave; k0 < ke; k0 += 32 * R16_NW * U) {
    h8l ah[U][RT], al[U][RT], bh[U][NJ], bl[U][NJ];
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int kk = k0 + 32 * R16_NW * u + 8 * q;
      const bool kin = kk < ke;
#pragma unroll
      for (int t = 0; t < RT; t++) {
        ah[u][t] = (rv[t] && kin) ? *reinterpret_cast<const h8l*>(xh.hi + xr[t] + kk) : z8;
        al[u][t] = (rv[t] && kin) ? *reinterpret_cast<const h8l*>(xh.lo + xr[t] + kk) : z8;
      }
#pragma unroll
      for (int jt = 0; jt < NJ; jt++) {
        const bool in = kin && kk >= klo[jt] && kk < khi[jt];
        bh[u][jt] = in ? *reinterpret_cast<const h8l*>(bt.hi + bbase[jt] + kk) : z8;
        bl[u][jt] = in ? *reinterpret_cast<const h8l*>(bt.lo + bbase[jt] + kk) : z8;
      }
    }
    // the three products of each tile issued pass by pass across the tiles (consecutive MFMAs independent)
#pragma unroll
    for (int u = 0; u < U; u++) {
#pragma unroll
      for (int t = 0; t < RT; t++)
#pragma unroll
        for (int jt = 0; jt < NJ; jt++)
          acc[t][jt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[u][t], bh[u][jt], acc[t][jt], 0, 0, 0);
#pragma unroll
      for (int t = 0; t < RT; t++)
#pragma unroll
        for (int jt = 0; jt < NJ; jt++)
          acc[t][jt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[u][t], bl[u][jt], acc[t][jt], 0, 0, 0);
#pragma unroll
      for (int t = 0; t < RT; t++)
#pragma unroll
        for (int jt = 0; jt < NJ; jt++)
          acc[t][jt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[u][t], bh[u][jt], acc[t][jt], 0, 0, 0);
    }
  }
  // element (row 16t+4q+i, col 16jt+p): the operand's row scale and the factor row's scale
#pragma unroll
  for (int t = 0; t < RT; t++)
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int r2 = m0 + 16 * t + 4 * q + i;
      const float ri = r2 < M ? xh.rinv[r2] : 0.0f;
#pragma unroll
      for (int jt = 0; jt < NJ; jt++)
        red[wave * E + (16 * t + 4 * q + i) * NC + 16 * jt + p] = acc[t][jt][i] * ri * bsc[jt];
    }
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += 64 * R16_NW) {
    float v = 0.0f;
    for (int w = 0; w < R16_NW; w++) v += red[w * E + e];
    const int rr = e / NC, c = e % NC, r2 = m0 + rr;
    if (gridDim.y == 1) {
      if (r2 < M && c < n) C[(long long)r2 * ldc + c] = alpha * v;
    } else {
      part[((long long)blockIdx.y * gridDim.x + blockIdx.x) * E + e] = v;
    }
  }
}

// One workgroup per row: max-abs, the power-of-two scale, fp16 hi/lo.
__global__ void __launch_bounds__(256) split_rows16_kernel(const SplitRow* __restrict__ rows, const float* __restrict__ src,
                                                           _Float16* __restrict__ hi, _Float16* __restrict__ lo,
                                                           float* __restrict__ sc) {
  __shared__ float red[4];
  const SplitRow rw = rows[blockIdx.x];
  const float* x = src + rw.off;
  float amax = 0.0f;
  for (int c = threadIdx.x; c < rw.len; c += 256) amax = fmaxf(amax, fabsf(x[c]));
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
  const float s = ldexpf(1.0f, e);
  if (threadIdx.x == 0) sc[blockIdx.x] = ldexpf(1.0f, -e);
  for (int c = threadIdx.x; c < rw.len; c += 256) {
    const float v = x[c] * s;
    const _Float16 h = (_Float16)v;
    hi[rw.off + c] = h;
    lo[rw.off + c] = (_Float16)(v - (float)h);
  }
}

int ceil_div_i(long long a, long long b) { return (int)((a + b - 1) / b); }

// Workgroups a launch aims for; the long contraction is split until the grid reaches it.
// (measured in the training step: 512 −1.6%, 2048 −1%, 4096 −3% tokens/s against 1024)
int split_target() { return 1024; }

// Split of the contraction of a rows launch (long contractions only): S chunks of kchunk columns.
void rows_split(long long M, long long K, int* S, int* kchunk) {
  const int gx = ceil_div_i(M, 32);
  int s = std::max(1, std::min(ceil_div_i(split_target(), gx), ceil_div_i(K, 64)));
  *kchunk = ceil_div_i(ceil_div_i(K, s), 64) * 64;
  *S = std::max(1, ceil_div_i(K, *kchunk));
}

// Split of the rows of a cols launch over gx column blocks: S chunks of mchunk rows.
void cols_split(long long M, int gx, int* S, int* mchunk) {
  int s = std::max(1, std::min(ceil_div_i(split_target(), gx), ceil_div_i(M, 16)));
  *mchunk = ceil_div_i(ceil_div_i(M, s), 16) * 16;
  *S = std::max(1, ceil_div_i(M, *mchunk));
}

}  // namespace

// Split of an fp16 rows launch: about HOS_R16_TARGET workgroups (16-row blocks × contraction chunks of whole
// 32·16-deep wave rounds; one 16-wave workgroup per CU — measured at Qwen2.5-0.5B: 256 beat 128 and 512, e.g. the
// gate|up du 24.4 µs at 2 splits against 27.7 at 4 and 31.7 at 7), each chunk at least HOS_R16_MINROUNDS rounds
// (the reduction launch costs more than a short chunk saves).
#ifndef HOS_R16_TARGET
#define HOS_R16_TARGET 256
#endif
#ifndef HOS_R16_MINROUNDS
#define HOS_R16_MINROUNDS 4
#endif
// Row tiles of 16 per fp16 rows workgroup: two when the 32-row blocks alone reach the split target and n <= 64 (each
// factor fragment loaded from L2 then feeds two row tiles; at one tile the factors' L2 bytes per workgroup are
// 2·n/16 times the activation's: Llama-3.2-1B's step, M 8192, +1.1%), else one (with fewer row blocks, two tiles per
// workgroup would need more contraction splits: Qwen2.5-0.5B at M 2048 −1.3% with two; above 64 columns the 16
// waves' LDS partial tiles would not fit) — except for contractions from HOS_R16_RT_K on, long enough to be split
// anyway (Qwen2.5-0.5B's gate|up du, K 9728: LoRA classes 3.80 -> 3.72 ms, +0.4% tokens/s; from K 4096 on, which
// adds its FFN down-projection, measured no gain).
#ifndef HOS_R16_RT
#define HOS_R16_RT 2
#endif
#ifndef HOS_R16_RT_K
#define HOS_R16_RT_K 8192
#endif
int rows16_rt(long long M, int n, long long K) {
  return (n <= 64 && ((M + 31) / 32 >= HOS_R16_TARGET || K >= HOS_R16_RT_K)) ? HOS_R16_RT : 1;
}
void rows16_split(long long M, long long K, int* S, int* kchunk, int rb = 16) {
  const int gx = ceil_div_i(M, rb), round = 32 * R16_NW;
  int s = std::max(1, std::min(ceil_div_i(HOS_R16_TARGET, gx), (int)(K / ((long long)round * HOS_R16_MINROUNDS))));
  *kchunk = ceil_div_i(ceil_div_i(K, s), round) * round;
  *S = std::max(1, ceil_div_i(K, *kchunk));
}

size_t lora_rows_ws_bytes(long long M, long long K, int n) {
  if (M <= 0 || n <= 0) return 0;
  int S16 = 0, kc16 = 0;
  const int rb16 = 16 * rows16_rt(M, n, K);
  rows16_split(M, K, &S16, &kc16, rb16);
  const size_t w16 = S16 > 1 ? (size_t)S16 * ceil_div_i(M, rb16) * rb16 * ((n + 15) / 16) * 16 * 4 : 0;
  if (K <= ROWS_WIDE_KMAX) return w16;
  int S = 0, kchunk = 0;
  rows_split(M, K, &S, &kchunk);
  return std::max(w16, S > 1 ? (size_t)S * ceil_div_i(M, 32) * 32 * ((n + 15) / 16) * 16 * 4 : (size_t)0);
}

void launch_split_rows16(const SplitRow* rows, int nrows, const float* src, _Float16* hi, _Float16* lo, float* sc,
                         hipStream_t st) {
  if (nrows <= 0) return;
  split_rows16_kernel<<<nrows, 256, 0, st>>>(rows, src, hi, lo, sc);
  HOS_HIP_CHECK(hipGetLastError());
}

namespace {
bool rows_short(long long K) { return K <= ROWS_WIDE_KMAX; }
// One launch of the f32 rows kernel over njobs jobs (j1 unused for one), then one reduction launch for the split ones.
void launch_rows_jobs(long long M, int NJ, int n, const RowsJobK& j0, const RowsJobK& j1, int njobs, HIn xh,
                      hipStream_t st) {
  const int gx = ceil_div_i(M, 32);
  dim3 grid(gx, std::max(j0.S, njobs > 1 ? j1.S : 1), njobs);
#define ROWS(NJV)                                                                        \
  case NJV:                                                                              \
    lora_rows_kernel<NJV><<<grid, 256, 0, st>>>((int)M, j0, njobs > 1 ? j1 : j0, xh);    \
    break;
  switch (NJ) {
    ROWS(1) ROWS(2) ROWS(3) ROWS(4) ROWS(5) ROWS(6)
    default: throw Error(HOS_E_INVALID, "lora_rows: bad width");
  }
#undef ROWS
  HOS_HIP_CHECK(hipGetLastError());
  if (j0.S > 1 || (njobs > 1 && j1.S > 1)) {
    const long long tot = (long long)gx * 32 * NJ * 16;
    const RowsRed r0{j0.part, j0.S, j0.alpha, j0.C, j0.ldc};
    const RowsRed r1 = njobs > 1 ? RowsRed{j1.part, j1.S, j1.alpha, j1.C, j1.ldc} : r0;
    lora_rows_reduce<<<dim3(ceil_div_i(tot, 256), njobs), 256, 0, st>>>(gx, 32, NJ * 16, (int)M, n, r0, r1);
    HOS_HIP_CHECK(hipGetLastError());
  }
}
}  // namespace

void launch_lora_rows(long long M, long long K, float alpha, const float* X, long long ldx, const float* Bt,
                      long long ldb, const RowsSeg& sg, float* C, long long ldc, float* ws, size_t ws_bytes,
                      hipStream_t st, HIn xh, B16 b16) {
  const int n = sg.nt * sg.r;
  if (M <= 0 || n <= 0) return;
  HOS_REQUIRE(n <= 96 && sg.nt >= 1 && sg.nt <= 4, HOS_E_INVALID, "lora_rows: n = nt·r must be <= 96");
  // fp16 path: 16-byte rows and segments on 8-element bounds (otherwise the f32 kernels, reading xh)
  bool f16 = xh.hi && xh.lo && b16.hi && b16.lo && b16.sc && K % 32 == 0 && ldx % 8 == 0 && ldb % 8 == 0 &&
             ((uintptr_t)xh.hi & 15) == 0 && ((uintptr_t)xh.lo & 15) == 0 && ((uintptr_t)b16.hi & 15) == 0 &&
             ((uintptr_t)b16.lo & 15) == 0;
  for (int t = 0; t < sg.nt; t++)
    f16 = f16 && sg.kbeg[t] % 8 == 0 && sg.kend[t] % 8 == 0 && sg.boff[t] % 8 == 0 && sg.kbeg[t] >= 0 &&
          sg.kend[t] <= K;
  if (f16) {
    HOS_REQUIRE(xh.rinv, HOS_E_INVALID, "lora_rows: the fp16 operand needs its row scales");
    const int RT = rows16_rt(M, n, K), rb = 16 * RT, gx = ceil_div_i(M, rb), NJ = (n + 15) / 16;
    int S = 0, kchunk = 0;
    rows16_split(M, K, &S, &kchunk, rb);
    HOS_REQUIRE(S == 1 || (size_t)S * gx * rb * NJ * 16 * 4 <= ws_bytes, HOS_E_INVALID, "lora_rows: workspace too small");
    dim3 grid(gx, S);
#define ROWS16(NJV, RTV)                                                                                   \
  case NJV * 8 + RTV:                                                                                      \
    lora_rows16_kernel<NJV, RTV><<<grid, 64 * R16_NW, 0, st>>>((int)M, (int)K, kchunk, alpha, xh, ldx, b16, ldb, sg, \
                                                               C, ldc, ws);                                \
    break;
    switch (NJ * 8 + RT) {
      ROWS16(1, 1) ROWS16(2, 1) ROWS16(3, 1) ROWS16(4, 1) ROWS16(5, 1) ROWS16(6, 1)
#if HOS_R16_RT == 2
      ROWS16(1, 2) ROWS16(2, 2) ROWS16(3, 2) ROWS16(4, 2)
#endif
      default: throw Error(HOS_E_INVALID, "lora_rows: bad width");
    }
#undef ROWS16
    HOS_HIP_CHECK(hipGetLastError());
    if (S > 1) {
      const long long tot = (long long)gx * rb * NJ * 16;
      const RowsRed rd{ws, S, alpha, C, ldc};
      lora_rows_reduce<<<ceil_div_i(tot, 256), 256, 0, st>>>(gx, rb, NJ * 16, (int)M, n, rd, rd);
      HOS_HIP_CHECK(hipGetLastError());
    }
    return;
  }
  HOS_REQUIRE(K % 4 == 0 && ldx % 4 == 0 && ldb % 4 == 0 && ((uintptr_t)Bt & 15) == 0 &&
                  (xh.hi ? (((uintptr_t)xh.hi & 7) == 0 && ((uintptr_t)xh.lo & 7) == 0 && xh.rinv)
                         : ((uintptr_t)X & 15) == 0),
              HOS_E_INVALID, "lora_rows: K, strides and pointers must be 16-byte aligned");
  for (int t = 0; t < sg.nt; t++)
    HOS_REQUIRE(sg.kbeg[t] % 4 == 0 && sg.kend[t] % 4 == 0 && sg.boff[t] % 4 == 0 && sg.kbeg[t] >= 0 &&
                    sg.kend[t] <= K,
                HOS_E_INVALID, "lora_rows: segment bounds must be multiples of 4 within K");
  if (rows_short(K) && n <= 96) {
    // one 16-column tile per workgroup (grid.y = tiles): 128-row-block grids alone leave half the CUs idle
    const dim3 gw((unsigned)ceil_div_i(M, 16), (unsigned)((n + 15) / 16));
    lora_rows_wide_kernel<1><<<gw, 64 * ROWS_WIDE_NW, 0, st>>>((int)M, (int)K, alpha, X, ldx, Bt, ldb, sg, C, ldc, xh);
    HOS_HIP_CHECK(hipGetLastError());
    return;
  }
  const int gx = ceil_div_i(M, 32);
  int S = 0, kchunk = 0;
  rows_split(M, K, &S, &kchunk);
  const int NJ = (n + 15) / 16;
  HOS_REQUIRE(S == 1 || (size_t)S * gx * 32 * NJ * 16 * 4 <= ws_bytes, HOS_E_INVALID, "lora_rows: workspace too small");
  const RowsJobK jb{(int)K, kchunk, S, alpha, X, ldx, Bt, ldb, sg, C, ldc, ws};
  launch_rows_jobs(M, NJ, n, jb, jb, 1, xh, st);
}

// Two independent f32 rows products over the same rows (u = x·A and du = s·dy·Bᵀ of the LoRA branch op) in one
// launch and one reduction launch, each job's partials in its own part of ws; shapes the one-job launcher would
// give another kernel (short contractions, other widths) or a too small ws run as two launches.
void launch_lora_rows2(long long M, const RowsCall& a, const RowsCall& b, float* ws, size_t ws_bytes,
                       hipStream_t st) {
  const int n = a.sg.nt * a.sg.r, NJ = (n + 15) / 16, gx = ceil_div_i(M, 32);
  auto plain = [&](const RowsCall& c) {
    bool ok = c.sg.nt * c.sg.r == n && !rows_short(c.K) && n <= 96 && c.sg.nt >= 1 && c.sg.nt <= 4 &&
              c.K % 4 == 0 && c.ldx % 4 == 0 && c.ldb % 4 == 0 && ((uintptr_t)c.Bt & 15) == 0 &&
              ((uintptr_t)c.X & 15) == 0;
    for (int t = 0; t < c.sg.nt; t++)
      ok = ok && c.sg.kbeg[t] % 4 == 0 && c.sg.kend[t] % 4 == 0 && c.sg.boff[t] % 4 == 0 && c.sg.kbeg[t] >= 0 &&
           c.sg.kend[t] <= c.K;
    return ok;
  };
  int Sa = 0, ka = 0, Sb = 0, kb = 0;
  rows_split(M, a.K, &Sa, &ka);
  rows_split(M, b.K, &Sb, &kb);
  const size_t pa = Sa > 1 ? (size_t)Sa * gx * 32 * NJ * 16 : 0, pb = Sb > 1 ? (size_t)Sb * gx * 32 * NJ * 16 : 0;
  if (M <= 0 || n <= 0 || !plain(a) || !plain(b) || (pa + pb) * 4 > ws_bytes) {
    launch_lora_rows(M, a.K, a.alpha, a.X, a.ldx, a.Bt, a.ldb, a.sg, a.C, a.ldc, ws, ws_bytes, st);
    launch_lora_rows(M, b.K, b.alpha, b.X, b.ldx, b.Bt, b.ldb, b.sg, b.C, b.ldc, ws, ws_bytes, st);
    return;
  }
  const RowsJobK ja{(int)a.K, ka, Sa, a.alpha, a.X, a.ldx, a.Bt, a.ldb, a.sg, a.C, a.ldc, ws};
  const RowsJobK jb{(int)b.K, kb, Sb, b.alpha, b.X, b.ldx, b.Bt, b.ldb, b.sg, b.C, b.ldc, ws + pa};
  launch_rows_jobs(M, NJ, n, ja, jb, 2, HIn{}, st);
}

namespace {
// Device form of a job: segment blocks laid out, row tiles (nsr = 16·NS) and partial region assigned.
ColsJobDev prepare(const ColsJob& j, int bx0) {
  ColsJobDev d{};
  HOS_REQUIRE(j.ns > 0 && j.ns <= 96 && j.sg.nseg > 0 && j.sg.nseg <= 4, HOS_E_INVALID,
              "lora_cols: ns must be in 1..96, 1 to 4 segments");
  HOS_REQUIRE(j.ldg % 4 == 0 && (j.gh.hi ? (((uintptr_t)j.gh.hi & 7) == 0 && ((uintptr_t)j.gh.lo & 7) == 0 && j.gh.rinv)
                                          : ((uintptr_t)j.Gm & 15) == 0),
              HOS_E_INVALID, "lora_cols: G must be 16-byte aligned");
  d.Sm = j.Sm;
  d.Gm = j.Gm;
  d.C = j.C;
  d.lds = j.lds;
  d.ldg = j.ldg;
  d.scj = j.scj;
  d.scc = j.scc;
  d.alpha = j.alpha;
  d.ns = j.ns;
  d.nsr = (j.ns + 15) / 16 * 16;
  d.sg = j.sg;
  d.gh = j.gh;
  // the fp16 operand in 16-byte runs where its rows, planes and segments allow (128-column blocks)
  bool wide = j.gh.hi && j.ldg % 8 == 0 && ((uintptr_t)j.gh.hi & 15) == 0 && ((uintptr_t)j.gh.lo & 15) == 0;
  for (int t = 0; t < j.sg.nseg; t++) wide = wide && j.sg.gbeg[t] % 8 == 0 && j.sg.len[t] % 8 == 0;
  d.bw = wide ? 128 : 64;
  int gx = 0;
  for (int t = 0; t < j.sg.nseg; t++) {
    HOS_REQUIRE(j.sg.gbeg[t] % 4 == 0 && j.sg.len[t] % 4 == 0 && j.sg.len[t] > 0, HOS_E_INVALID,
                "lora_cols: segment columns must be multiples of 4");
    d.sg.blk0[t] = gx;
    gx += ceil_div_i(j.sg.len[t], d.bw);
  }
  d.gx = gx;
  d.bx0 = bx0;
  return d;
}
}  // namespace

void launch_lora_cols2(long long M, const ColsJob& ja, const ColsJob* jb, float* ws, size_t ws_bytes, hipStream_t st,
                       ColsBatch* batch) {
  if (M <= 0) return;
  ColsJobDev a = prepare(ja, 0);
  ColsJobDev b{};
  if (jb) {
    b = prepare(*jb, a.gx);
  } else {
    b = a;  // never run: its block range is empty
    b.bx0 = a.gx;
    b.gx = 0;
  }
  const int gx = a.gx + b.gx;
  int S = 0, mchunk = 0;
  cols_split(M, gx, &S, &mchunk);
  a.part_off = 0;
  b.part_off = (long long)S * a.gx * a.nsr * a.bw;
  const long long need = b.part_off + (long long)S * b.gx * b.nsr * b.bw;
  a.S = b.S = S;
  // deferred: the partials go to the batch buffer (offsets relative to its base) and the reduction waits for
  // the flush
  const int njobs = jb ? 2 : 1;
  const bool defer = batch && S > 1 && batch->n + njobs <= 8 && batch->used + (size_t)need <= batch->cap;
  float* part = ws;
  if (defer) {
    a.part_off += (long long)batch->used;
    b.part_off += (long long)batch->used;
    part = batch->base;
  } else {
    HOS_REQUIRE(S == 1 || (size_t)need * 4 <= ws_bytes, HOS_E_INVALID, "lora_cols: workspace too small");
  }
  const int NA = a.nsr / 16, NB = jb ? b.nsr / 16 : NA;
  dim3 grid(gx, S);
#define COLS(X, Y)                                                                          \
  if (NA == X && NB == Y && !bgh) {                                                         \
    if (a.gh.hi && a.bw == 128)                                                             \
      lora_cols_kernel<X, Y, true, 8><<<grid, 256, 0, st>>>((int)M, mchunk, a, b, part);    \
    else if (a.gh.hi)                                                                       \
      lora_cols_kernel<X, Y, true><<<grid, 256, 0, st>>>((int)M, mchunk, a, b, part);       \
    else                                                                                    \
      lora_cols_kernel<X, Y, false><<<grid, 256, 0, st>>>((int)M, mchunk, a, b, part);      \
    launched = true;                                                                        \
  }
  const bool bgh = jb && b.gh.hi;
  bool launched = false;
  COLS(1, 1) COLS(2, 2) COLS(3, 3) COLS(4, 4) COLS(5, 5) COLS(6, 6) COLS(1, 2) COLS(1, 3) COLS(2, 4) COLS(2, 6)
#undef COLS
  if (!launched) {
    // width pair without a combined kernel (or a second job on the fp16 operand): run the jobs one after the other
    HOS_REQUIRE(jb != nullptr, HOS_E_INVALID, "lora_cols: bad width");
    launch_lora_cols2(M, ja, nullptr, ws, ws_bytes, st, batch);
    launch_lora_cols2(M, *jb, nullptr, ws, ws_bytes, st, batch);
    return;
  }
  HOS_HIP_CHECK(hipGetLastError());
  if (defer) {
    batch->jobs[batch->n++] = a;
    if (jb) batch->jobs[batch->n++] = b;
    batch->used += (size_t)need;
    return;
  }
  if (S > 1) {
    const long long tot = (long long)a.gx * a.nsr * a.bw + (long long)b.gx * b.nsr * b.bw;
    lora_cols_reduce<<<ceil_div_i(tot, 256), 256, 0, st>>>(ws, S, a, b);
    HOS_HIP_CHECK(hipGetLastError());
  }
}

size_t lora_cols2_ws_bytes(long long M, const ColsJob& ja, const ColsJob* jb) {
  if (M <= 0) return 0;
  const ColsJobDev a = prepare(ja, 0);
  const ColsJobDev b = jb ? prepare(*jb, a.gx) : ColsJobDev{};
  int S = 0, mchunk = 0;
  cols_split(M, a.gx + (jb ? b.gx : 0), &S, &mchunk);
  size_t need = S > 1 ? (size_t)S * ((size_t)a.gx * a.nsr * a.bw + (jb ? (size_t)b.gx * b.nsr * b.bw : 0)) * 4 : 0;
  if (jb && a.nsr != b.nsr)  // some width pairs have no combined kernel and run as two launches in turn
    need = std::max({need, lora_cols2_ws_bytes(M, ja, nullptr), lora_cols2_ws_bytes(M, *jb, nullptr)});
  return need;
}

void launch_lora_cols_table(long long M, const ColsJob* jobs, int n, ColsTable& tab, hipStream_t st) {
  if (M <= 0 || n <= 0) return;
  HOS_REQUIRE(n <= tab.cap, HOS_E_INVALID, "lora_cols_table: more jobs than the table holds");
  // jobs grouped by kernel shape (stable), each group's jobs and block starts contiguous in the table
  std::vector<int> key(n), order(n);
  std::vector<ColsJobDev> dev(n);
  for (int i = 0; i < n; i++) {
    dev[i] = prepare(jobs[i], 0);
    dev[i].S = 1;
    dev[i].part_off = 0;
    const int ns = dev[i].nsr / 16, v = dev[i].gh.hi ? (dev[i].bw == 128 ? 2 : 1) : 0;
    HOS_REQUIRE(ns >= 1 && ns <= 6, HOS_E_INVALID, "lora_cols_table: bad width");
    key[i] = ns * 3 + v;
    order[i] = i;
  }
  std::stable_sort(order.begin(), order.end(), [&](int a, int b) { return key[a] < key[b]; });
  struct Group {
    int key, first, n, blocks;
  };
  std::vector<Group> groups;
  int* hstart = reinterpret_cast<int*>(tab.host + tab.cap);
  for (int i = 0; i < n; i++) {
    const int k = key[order[i]];
    if (groups.empty() || groups.back().key != k) groups.push_back(Group{k, i, 0, 0});
    Group& g = groups.back();
    tab.host[i] = dev[order[i]];
    hstart[i + (int)groups.size() - 1] = g.blocks;  // a group of n jobs takes n + 1 starts
    g.blocks += dev[order[i]].gx;
    g.n++;
  }
  // each group's closing start
  for (size_t gi = 0; gi < groups.size(); gi++) hstart[groups[gi].first + groups[gi].n + (int)gi] = groups[gi].blocks;
  const size_t bytes = (size_t)tab.cap * sizeof(ColsJobDev) + (size_t)(n + groups.size()) * sizeof(int);
  HOS_HIP_CHECK(hipMemcpyAsync(tab.dev, tab.host, bytes, hipMemcpyHostToDevice, st));
  const int* dstart = reinterpret_cast<const int*>(tab.dev + tab.cap);
  for (size_t gi = 0; gi < groups.size(); gi++) {
    const Group& g = groups[gi];
    const ColsJobDev* dj = tab.dev + g.first;
    const int* ds = dstart + g.first + (int)gi;
    const int ns = g.key / 3, v = g.key % 3;
    // 8 row steps per trip from M 8192 on (Llama-3.2-1B's step: the batch 6.9 -> 6.5 ms, +1.5% tokens/s), else 4
    // (Qwen2.5-0.5B at M 2048: 8 and 2 measured 0.5% slower)
    const bool deep = M >= 8192;
#define CTAB1(NSV, GHV, CWV)                                                                                 \
  if (deep)                                                                                                  \
    lora_cols_table_kernel<NSV, GHV, CWV, 8><<<g.blocks, 256, 0, st>>>((int)M, dj, ds, g.n);                 \
  else                                                                                                       \
    lora_cols_table_kernel<NSV, GHV, CWV, 4><<<g.blocks, 256, 0, st>>>((int)M, dj, ds, g.n);
#define CTAB(NSV)                                                                                            \
  case NSV:                                                                                                  \
    if (v == 2) {                                                                                            \
      CTAB1(NSV, true, 8)                                                                                    \
    } else if (v == 1) {                                                                                     \
      CTAB1(NSV, true, 4)                                                                                    \
    } else {                                                                                                 \
      CTAB1(NSV, false, 4)                                                                                   \
    }                                                                                                        \
    break;
    switch (ns) {
      CTAB(1) CTAB(2) CTAB(3) CTAB(4) CTAB(5) CTAB(6)
      default: break;
    }
#undef CTAB
#undef CTAB1
    HOS_HIP_CHECK(hipGetLastError());
  }
}

size_t lora_cols_table_bytes(int cap) { return (size_t)cap * sizeof(ColsJobDev) + (size_t)2 * cap * sizeof(int); }

void launch_lora_cols_flush(ColsBatch& bt, hipStream_t st) {
  if (bt.n > 0) {
    ColsBatchArgs args{};
    long long tot = 0;
    for (int j = 0; j < bt.n; j++) {
      args.jobs[j] = bt.jobs[j];
      args.start[j] = tot;
      tot += (long long)bt.jobs[j].gx * bt.jobs[j].nsr * bt.jobs[j].bw;
    }
    args.start[bt.n] = tot;
    args.n = bt.n;
    lora_cols_reduce_batch<<<ceil_div_i(tot, 256), 256, 0, st>>>(bt.base, args);
    HOS_HIP_CHECK(hipGetLastError());
  }
  bt.n = 0;
  bt.used = 0;
}

void launch_lora_cols(long long M, int ns, float alpha, const float* Sm, long long lds, const float* Gm, long long ldg,
                      ColsSeg sg, float* C, long long scj, long long scc, float* ws, size_t ws_bytes,
                      hipStream_t st) {
  if (M <= 0 || ns <= 0 || sg.nseg <= 0) return;
  ColsJob j{ns, alpha, Sm, lds, Gm, ldg, sg, C, scj, scc};
  launch_lora_cols2(M, j, nullptr, ws, ws_bytes, st);
}

}  // namespace hos
