// LoRA factor GEMMs (lora.hip): skinny fp32-MFMA products with a deterministic split reduction.
#pragma once
#include <algorithm>

#include "kernels.hpp"

namespace hos {

// An activation given as the fp16 GEMM operand instead of f32: X[m, k] = (hi[m, k] + lo[m, k])·rinv[m] (hi + lo is
// exact in f32 and rinv is a power of two, so this is the operand's ~22-bit value). hi == nullptr: not given.
struct HIn {
  const _Float16* hi = nullptr;
  const _Float16* lo = nullptr;
  const float* rinv = nullptr;
};

// A factor matrix split for fp16 MFMA: Bt(j, k) = (hi + lo)[same index as the f32 Bt]·sc[row], where the scale row of
// output column j (slot t, jj < r) is boff[t] / ldb + jj — the stacked row for x·A (boff = t·r·ldb) and row jj for
// dy·Bᵀ (boff a column offset < ldb). sc are powers of two putting each row's max-abs in [2^14, 2^15).
struct B16 {
  const _Float16* hi = nullptr;
  const _Float16* lo = nullptr;
  const float* sc = nullptr;
};

// Output columns of the rows kernel come in nt slots of r columns (one per adapter target). Slot t
// contracts over X columns [kbeg[t], kend[t]) against Bt[boff[t] + jj·ldb + (k − kbeg[t])], jj < r.
struct RowsSeg {
  int nt = 0, r = 0;
  int kbeg[4] = {0, 0, 0, 0}, kend[4] = {0, 0, 0, 0};
  long long boff[4] = {0, 0, 0, 0};
};
// C[m, j] = α·Σ_k X[m, k]·B(j, k) for m < M, j < nt·r. X rows 16-byte aligned, K % 4 == 0. xh.hi set: X is
// that operand (row stride ldx, 8-byte aligned rows) and the f32 pointer is not read.
void launch_lora_rows(long long M, long long K, float alpha, const float* X, long long ldx, const float* Bt,
                      long long ldb, const RowsSeg& sg, float* C, long long ldc, float* ws, size_t ws_bytes,
                      hipStream_t st, HIn xh = HIn{}, B16 b16 = B16{});
// The arguments of one f32 launch_lora_rows product.
struct RowsCall {
  long long K;
  float alpha;
  const float* X;
  long long ldx;
  const float* Bt;
  long long ldb;
  RowsSeg sg;
  float* C;
  long long ldc;
};
// Two independent f32 rows products over the same M rows in one launch (falls back to two launch_lora_rows calls
// where one launch does not fit); ws holds both jobs' split partials (lora_rows_ws_bytes of each, summed).
void launch_lora_rows2(long long M, const RowsCall& a, const RowsCall& b, float* ws, size_t ws_bytes,
                       hipStream_t st);
// With both xh and b16 given the product runs on fp16 MFMA (three products, hi·hi + lo·hi + hi·lo: ~2^-22 relative
// to the f32 one) — the rows kernel's fp32 MFMA rate bounds the long contractions otherwise.

// Split f32 rows into fp16 hi/lo with a power-of-two scale per row (rows[i] = {offset, length} into src / hi / lo;
// scale of row i to sc[i]): the per-step preparation of the factors a B16 reads.
struct SplitRow {
  long long off;
  int len;
};
void launch_split_rows16(const SplitRow* rows, int nrows, const float* src, _Float16* hi, _Float16* lo, float* sc,
                         hipStream_t st);

// Column segments of the cols kernel: segment t covers G columns [gbeg, gbeg + len), uses S columns
// starting at soff and writes output columns starting at ocol. blk0 is filled in by the launcher.
struct ColsSeg {
  int nseg = 0;
  int gbeg[4] = {0, 0, 0, 0}, len[4] = {0, 0, 0, 0}, soff[4] = {0, 0, 0, 0}, ocol[4] = {0, 0, 0, 0};
  int blk0[4] = {0, 0, 0, 0};
};
// C[j·scj + (ocol + c)·scc] = α·Σ_m S[m, soff + j]·G[m, gbeg + c] for j < ns, c < len, per segment.
void launch_lora_cols(long long M, int ns, float alpha, const float* Sm, long long lds, const float* Gm, long long ldg,
                      ColsSeg sg, float* C, long long scj, long long scc, float* ws, size_t ws_bytes,
                      hipStream_t st);

// One cols product as a job (the arguments of launch_lora_cols).
struct ColsJob {
  int ns = 0;
  float alpha = 1.0f;
  const float* Sm = nullptr;
  long long lds = 0;
  const float* Gm = nullptr;
  long long ldg = 0;
  ColsSeg sg;
  float* C = nullptr;
  long long scj = 0, scc = 0;
  HIn gh;  // gh.hi set: G is that operand (row stride ldg) and Gm is not read
};
// Kernel-side job: the above with its block range and partial-sum region.
struct ColsJobDev {
  const float* Sm;
  const float* Gm;
  float* C;
  long long lds, ldg, scj, scc, part_off;
  float alpha;
  int ns, nsr, gx, bx0;
  int bw;  // columns per workgroup block: 64, or 128 for a G read as 16-byte runs of the fp16 operand's planes
  int S;   // splits of M the partials were written with
  ColsSeg sg;
  HIn gh;
};
// Deferred reductions: cols launches given a batch write their partials into the batch's buffer and leave the
// reduction to one launch_lora_cols_flush for all of them (up to 8 jobs; a job that does not fit is reduced
// at once as without a batch).
struct ColsBatch {
  float* base = nullptr;
  size_t cap = 0, used = 0;  // floats
  ColsJobDev jobs[8];
  int n = 0;
};
void launch_lora_cols_flush(ColsBatch& b, hipStream_t st);
// A job table for launch_lora_cols_table: cap jobs plus 2·cap block starts, a pinned host copy and a device copy
// (lora_cols_table_bytes(cap) bytes each, allocated by the owner before any graph capture). The host copy is
// rewritten and sent with each launch — identical content for the same jobs, so a captured copy of it stays valid.
struct ColsTable {
  ColsJobDev* host = nullptr;
  ColsJobDev* dev = nullptr;
  int cap = 0;
};
size_t lora_cols_table_bytes(int cap);
// Every job, one launch per kernel shape whatever the job count (the jobs go through tab), each output block over all
// M rows in one workgroup (no partials, no reduction launch). Deterministic: each element sums its rows in one fixed
// order.
void launch_lora_cols_table(long long M, const ColsJob* jobs, int n, ColsTable& tab, hipStream_t st);
// Two independent cols products over the same M in one launch (and one reduction launch); b may be null.
// Deterministic: the split of M depends only on M and the combined block count, and every output element sums
// its split partials in split order.
void launch_lora_cols2(long long M, const ColsJob& a, const ColsJob* b, float* ws, size_t ws_bytes, hipStream_t st,
                       ColsBatch* batch = nullptr);

// Workspace bytes the launches above need (no batch) for these shapes: 0 when they do not split.
size_t lora_rows_ws_bytes(long long M, long long K, int n);
size_t lora_cols2_ws_bytes(long long M, const ColsJob& a, const ColsJob* b);

}  // namespace hos
