// Full-parameter finetune step on the device: FtModel (src/finetune.rs) — every weight a trainable f32
// parameter (quantized tensors dequantized once at load, the head an untied copy when the file ties it),
// the Llama-family forward of FtModel::hidden (src/finetune.rs:244-319), cross-entropy per sequence with
// the loss scaled by 1/B (the accumulation of src/main.rs:2834-2855), backward through every weight, and
// AdamW over FtModel::params with decay on the 2-D tensors (src/main.rs:2803-2804).
//
// The weight GEMMs, all on [out, in] weights kept in the GGUF layout and all on the quantized-weight GEMM (3
// precision passes on fp16 MFMA): forward Y = X·Wᵀ and input gradient dX = dY·W with the f32 weight as its layout,
// the weight gradient dW = dYᵀ·X (the matmul_atb of src/metal_be.rs:1212-1234) in its dX form over the tokens, dYᵀ
// the operand and X the f32 "weight" (the f32 GEMM of gemm_f32.hip, fp32 MFMA, when the token count is not a
// multiple of 32). Norm-weight and bias gradients are column sums, in row order within chunks
// of rows and the chunks in order; the embedding gradient adds each token's row into its id's row in token order
// (both deterministic).
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "ctx.hpp"
#include "fused.hpp"

using namespace hos;

namespace {

// out[j] = Σ_r g[r][j]·(x ? x[r][j]·inv[r] : 1): each workgroup row (blockIdx.y) sums one chunk of COLSUM_CH rows in
// row order into part[chunk][j] (one thread per column, coalesced over the columns), then colsum_fold adds the
// chunks in chunk order — deterministic, and the chunks run in parallel (one thread per column over all rows left
// the whole GPU with a few waves, each waiting on one load per row: 0.6 ms per call at M 2048).
constexpr int COLSUM_CH = 32;
__global__ void colsum_part_kernel(const float* __restrict__ g, long long ldg, const float* __restrict__ x,
                                   long long ldx, const float* __restrict__ inv, int M, int n,
                                   float* __restrict__ part) {
#pragma clang fp contract(off)
  const int j = blockIdx.x * blockDim.x + threadIdx.x;
  if (j >= n) return;
  const int r0 = blockIdx.y * COLSUM_CH, r1 = min(M, r0 + COLSUM_CH);
  float s = 0.0f;
  if (x) {
#pragma unroll 8
    for (int r = r0; r < r1; r++) s += g[(long long)r * ldg + j] * x[(long long)r * ldx + j] * inv[r];
  } else {
#pragma unroll 8
    for (int r = r0; r < r1; r++) s += g[(long long)r * ldg + j];
  }
  part[(long long)blockIdx.y * n + j] = s;
}
__global__ void colsum_fold_kernel(const float* __restrict__ part, int nch, int n, float* __restrict__ out) {
  const int j = blockIdx.x * blockDim.x + threadIdx.x;
  if (j >= n) return;
  float s = 0.0f;
#pragma unroll 8
  for (int c = 0; c < nch; c++) s += part[(long long)c * n + j];
  out[j] = s;
}

// The weight gradient dW[o, i] = Σ_m dY[m, o]·X[m, i] runs as the quantized-weight GEMM's dX form with dYᵀ as its
// fp16 row-scaled operand ([o][M]: one row per output column of dY, over the tokens) and X as an f32 "weight" of M
// rows. These two kernels form that operand: the max |dY| of every column over each chunk of COLSUM_CH rows, then
// 64×64 tiles transposed through LDS — each workgroup first folds its 64 columns' chunk maxima (max is
// order-free) — and written as the scaled fp16 hi / lo planes with the row scale of launch_to_h16 (a power of two
// putting the row max in [2^14, 2^15)).
__global__ void colmax_kernel(const float* __restrict__ g, long long ldg, int M, int n, float* __restrict__ cpart) {
  const int j = blockIdx.x * blockDim.x + threadIdx.x;
  if (j >= n) return;
  const int r0 = blockIdx.y * COLSUM_CH, r1 = min(M, r0 + COLSUM_CH);
  float m = 0.0f;
#pragma unroll 8
  for (int r = r0; r < r1; r++) m = fmaxf(m, fabsf(g[(long long)r * ldg + j]));
  cpart[(long long)blockIdx.y * n + j] = m;
}
__device__ __forceinline__ int tr_row_exp(float amax) {  // the row scale exponent of launch_to_h16
  if (!(amax > 0.0f) || amax >= 3.0e38f) return 0;
  int ex;
  frexpf(amax, &ex);
  const int e = 15 - ex;
  return e > 100 ? 100 : (e < -100 ? -100 : e);
}
__global__ void __launch_bounds__(256) transpose_h16_kernel(const float* __restrict__ g, long long ldg, int M, int n,
                                                            const float* __restrict__ cpart, int nch,
                                                            _Float16* __restrict__ hi, _Float16* __restrict__ lo,
                                                            float* __restrict__ rinv) {
  __shared__ float tile[64][65];
  __shared__ float cm[4][64];
  const int c0 = blockIdx.x * 64, m0 = blockIdx.y * 64, tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  {
    float mx = 0.0f;
    if (c0 + tx < n)
      for (int k = ty; k < nch; k += 4) mx = fmaxf(mx, cpart[(long long)k * n + c0 + tx]);
    cm[ty][tx] = mx;
  }
  for (int r = ty; r < 64; r += 4) {
    const int m = m0 + r, c = c0 + tx;
    tile[r][tx] = (m < M && c < n) ? g[(long long)m * ldg + c] : 0.0f;
  }
  __syncthreads();
  if (ty == 0) {
    const int e = tr_row_exp(fmaxf(fmaxf(cm[0][tx], cm[1][tx]), fmaxf(cm[2][tx], cm[3][tx])));
    cm[0][tx] = (float)e;  // exact small integer
    if (blockIdx.y == 0 && c0 + tx < n) rinv[c0 + tx] = ldexpf(1.0f, -e);
  }
  __syncthreads();
  for (int cc = ty; cc < 64; cc += 4) {
    const int c = c0 + cc, m = m0 + tx;
    if (c >= n) break;
    if (m < M) {
      const float v = tile[tx][cc] * ldexpf(1.0f, (int)cm[0][cc]);
      const _Float16 h = (_Float16)v;
      hi[(long long)c * M + m] = h;
      lo[(long long)c * M + m] = (_Float16)(v - (float)h);
    }
  }
}

// dE[ids[t]] = Σ over the tokens with that id, in token order (the first occurrence's workgroup does the row)
__global__ void embed_grad_kernel(const int32_t* __restrict__ ids, int M, const float* __restrict__ dx, int d,
                                  float* __restrict__ dE) {
  const int t = blockIdx.x;
  const int id = ids[t];
  for (int u = 0; u < t; u++)
    if (ids[u] == id) return;  // uniform over the workgroup
  for (int c = threadIdx.x; c < d; c += blockDim.x) {
    float s = 0.0f;
    for (int u = t; u < M; u++)
      if (ids[u] == id) s += dx[(long long)u * d + c];
    dE[(long long)id * d + c] = s;
  }
}

__global__ void add_bias_kernel(float* __restrict__ y, long long ld, int M, int n, const float* __restrict__ b) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long long)M * n) return;
  const int r = (int)(i / n), c = (int)(i % n);
  y[(long long)r * ld + c] += b[c];
}

__global__ void embed_f32_kernel(const float* __restrict__ E, const int32_t* __restrict__ ids, int M, int d,
                                 float* __restrict__ x) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long long)M * d) return;
  const int m = (int)(i / d), c = (int)(i % d);
  x[i] = E[(long long)ids[m] * d + c];
}

enum { WQ, WK, WV, WO, WG, WU, WD, NW };
enum { NA, NF, BQ, BK, BV, NV };  // attn_norm, ffn_norm, biases

}  // namespace

struct hos_ft {
  hos_ctx* ctx = nullptr;
  hipStream_t st = nullptr;
  hos_peft_cfg c{};
  std::string err;
  int d = 0, qd = 0, kvd = 0, W3 = 0, F = 0, V = 0, L = 0, Mmax = 0;
  std::vector<void*> allocs;
  // parameter arena: 2-D tensors first (AdamW decay), then 1-D; per tensor its offset (floats)
  long long n2 = 0, n = 0;
  float *P = nullptr, *G = nullptr, *M1 = nullptr, *V1 = nullptr;
  long long o_tok = -1, o_out = -1, o_onorm = -1;
  std::vector<long long> o_w, o_v;  // [L][NW], [L][NV]
  bool out_set = false, tok_set = false;
  std::map<std::string, bool> seen;
  uint64_t adam_t = 0;
  AdamHyper* hyp = nullptr;
  AdamHyper hyp_host{};
  // activations [Mmax, …] per layer
  struct Act {
    float *x, *xn1, *inv1, *qkv, *o, *lse, *x2, *xn2, *inv2, *gu, *h;
  };
  std::vector<Act> act;
  float *xf = nullptr, *xfn = nullptr, *invf = nullptr, *logits = nullptr, *dl = nullptr, *row_loss = nullptr,
        *loss = nullptr, *dx = nullptr, *dxn = nullptr, *dqkv = nullptr, *dout = nullptr, *dh = nullptr,
        *dgu = nullptr, *dvec = nullptr, *part = nullptr, *ws = nullptr;
  void* attn_planes = nullptr;  // bf16 hi/lo planes of q, k, v (attention scratch)
  size_t ws_bytes = 0;
  H16 hs{};
  H16 ah{};  // fp16 hi/lo operand of a weight GEMM's activation (X forward, dY for the input gradient)
  float* csp = nullptr;  // column-sum partials, one row per chunk of rows
  size_t csp_n = 0;
  size_t ah_n = 0;             // elements of each plane of ah
  float* cpart = nullptr;      // per-chunk column max |dY| for the transposed operand
  size_t cpart_n = 0;
  float* tr_rinv = nullptr;    // its row scales, one per column of dY
  size_t tr_rows = 0;
  float2* rope_tab = nullptr;
  int32_t *ids = nullptr, *tgts = nullptr;

  template <class T>
  T* alloc(size_t count) {
    void* p = nullptr;
    if (count == 0) count = 1;
    hipError_t e = hipMalloc(&p, count * sizeof(T));
    if (e != hipSuccess) throw Error(HOS_E_OOM, "hipMalloc(" + std::to_string(count * sizeof(T)) + ") failed");
    allocs.push_back(p);
    return (T*)p;
  }
  void wdims(int t, int* out, int* in) const {
    switch (t) {
      case WQ: *out = qd; *in = d; break;
      case WK: *out = kvd; *in = d; break;
      case WV: *out = kvd; *in = d; break;
      case WO: *out = d; *in = qd; break;
      case WG: *out = F; *in = d; break;
      case WU: *out = F; *in = d; break;
      default: *out = d; *in = F; break;
    }
  }
  int vdim(int t) const { return t == NA || t == NF ? d : (t == BQ ? qd : kvd); }
  float* W(int l, int t) const { return P + o_w[(size_t)l * NW + t]; }
  float* dW(int l, int t) const { return G + o_w[(size_t)l * NW + t]; }
  float* Vp(int l, int t) const { return o_v[(size_t)l * NV + t] < 0 ? nullptr : P + o_v[(size_t)l * NV + t]; }
  float* dV(int l, int t) const { return G + o_v[(size_t)l * NV + t]; }

  void init(hos_ctx* cx, const hos_peft_cfg* cfg) {
    ctx = cx;
    st = hos_internal_stream(cx);
    c = *cfg;
    HOS_REQUIRE(c.n_layers > 0 && c.dim > 0 && c.n_heads > 0 && c.n_kv_heads > 0 && c.ffn_dim > 0 && c.vocab > 0,
                HOS_E_INVALID, "finetune: bad model dimensions");
    HOS_REQUIRE(c.n_heads % c.n_kv_heads == 0, HOS_E_INVALID, "finetune: n_heads must be a multiple of n_kv_heads");
    HOS_REQUIRE(c.head_dim == 64 || c.head_dim == 128, HOS_E_UNSUPPORTED_ARCH, "finetune: head_dim must be 64 or 128");
    HOS_REQUIRE(c.n_experts == 0 && !c.qk_norm, HOS_E_UNSUPPORTED_ARCH,
                "finetune: FtModel covers the dense Llama family (no experts, no QK-norm), src/finetune.rs:62-75");
    HOS_REQUIRE(c.max_batch > 0 && c.max_seq > 0, HOS_E_INVALID, "finetune: bad batch/seq");
    L = c.n_layers;
    d = c.dim;
    qd = c.n_heads * c.head_dim;
    kvd = c.n_kv_heads * c.head_dim;
    W3 = qd + 2 * kvd;
    F = c.ffn_dim;
    V = c.vocab;
    Mmax = c.max_batch * c.max_seq;
    // arena
    auto pad = [](long long v) { return (v + 63) & ~63LL; };
    long long off = 0;
    o_tok = off;
    off = pad(off + (long long)V * d);
    o_out = off;
    off = pad(off + (long long)V * d);
    o_w.assign((size_t)L * NW, -1);
    o_v.assign((size_t)L * NV, -1);
    for (int l = 0; l < L; l++)
      for (int t = 0; t < NW; t++) {
        int o, i;
        wdims(t, &o, &i);
        o_w[(size_t)l * NW + t] = off;
        off = pad(off + (long long)o * i);
      }
    n2 = off;
    o_onorm = off;
    off = pad(off + d);
    for (int l = 0; l < L; l++)
      for (int t = 0; t < NV; t++) {
        if ((t == BQ || t == BK || t == BV) && !c.attn_bias) continue;
        o_v[(size_t)l * NV + t] = off;
        off = pad(off + vdim(t));
      }
    n = off;
    P = alloc<float>(n);
    G = alloc<float>(n);
    M1 = alloc<float>(n);
    V1 = alloc<float>(n);
    for (float* p : {P, G, M1, V1}) launch_fill(p, n, 0.0f, st);
    const size_t M = (size_t)Mmax;
    act.resize(L);
    for (auto& a : act) {
      a.x = alloc<float>(M * d);
      a.xn1 = alloc<float>(M * d);
      a.inv1 = alloc<float>(M);
      a.qkv = alloc<float>(M * W3);
      a.o = alloc<float>(M * qd);
      a.lse = alloc<float>(M * c.n_heads);
      a.x2 = alloc<float>(M * d);
      a.xn2 = alloc<float>(M * d);
      a.inv2 = alloc<float>(M);
      a.gu = alloc<float>(M * 2 * F);
      a.h = alloc<float>(M * F);
    }
    xf = alloc<float>(M * d);
    xfn = alloc<float>(M * d);
    invf = alloc<float>(M);
    logits = alloc<float>(M * V);
    dl = alloc<float>(M * V);
    row_loss = alloc<float>(M);
    loss = alloc<float>(1);
    dx = alloc<float>(M * d);
    dxn = alloc<float>(M * d);
    dqkv = alloc<float>(M * W3);
    dout = alloc<float>(M * qd);
    dh = alloc<float>(M * F);
    dgu = alloc<float>(M * 2 * F);
    dvec = alloc<float>(M * c.n_heads);
    if (c.n_heads != c.n_kv_heads) part = alloc<float>(M * c.n_heads * 2 * c.head_dim);
    attn_planes = alloc<float>(attn_scratch_bytes(c.max_batch, c.max_seq, c.n_heads, c.n_kv_heads, c.head_dim) / 4);
    const size_t hc = std::max<size_t>({(size_t)d, 2 * (size_t)F});
    hs.data = alloc<half_t>(M * hc);  // fp16 operand the fused norm / SwiGLU kernels also write (unused here)
    hs.rinv = alloc<float>(M);
    const size_t amax = std::max<size_t>({(size_t)d, (size_t)qd, (size_t)F, (size_t)V});
    ah_n = M * amax;
    ah.data = alloc<half_t>(ah_n);
    ah.lo = alloc<half_t>(ah_n);
    ah.rinv = alloc<float>(M);
    tr_rows = amax;
    cpart_n = (size_t)ceil_div((long long)M, COLSUM_CH) * tr_rows;
    cpart = alloc<float>(cpart_n);
    tr_rinv = alloc<float>(tr_rows);
    csp_n = (size_t)ceil_div((long long)M, COLSUM_CH) * std::max<size_t>((size_t)d, (size_t)qd);
    csp = alloc<float>(csp_n);
    ws_bytes = std::max<size_t>(64ull << 20, std::min<size_t>(M * std::max<size_t>(V, 2 * (size_t)F) * 4, 1ull << 30));
    ws = alloc<float>(ws_bytes / 4);
    hyp = alloc<AdamHyper>(1);
    launch_fill((float*)hyp, sizeof(AdamHyper) / 4, 0.0f, st);
    ids = alloc<int32_t>(M);
    tgts = alloc<int32_t>(M);
    const int half = c.head_dim / 2;
    std::vector<float2> tab((size_t)c.max_seq * half);
    for (int p = 0; p < c.max_seq; p++)
      for (int i = 0; i < half; i++) {
        float freq = 1.0f / powf(c.rope_base, 2.0f * (float)i / (float)c.head_dim);
        float ang = (float)p * freq;
        tab[(size_t)p * half + i] = make_float2(sinf(ang), cosf(ang));
      }
    rope_tab = alloc<float2>(tab.size());
    HOS_HIP_CHECK(hipMemcpyAsync(rope_tab, tab.data(), tab.size() * sizeof(float2), hipMemcpyHostToDevice, st));
    HOS_HIP_CHECK(hipStreamSynchronize(st));
  }
  void release() {
    (void)hipStreamSynchronize(st);
    for (void* p : allocs) (void)hipFree(p);
    allocs.clear();
  }

  // ---- tensors ----
  float* slot_of(const std::string& name, size_t* count) {
    if (name == "token_embd.weight") return *count = (size_t)V * d, P + o_tok;
    if (name == "output.weight") return *count = (size_t)V * d, P + o_out;
    if (name == "output_norm.weight") return *count = d, P + o_onorm;
    HOS_REQUIRE(name.rfind("blk.", 0) == 0, HOS_E_INVALID, "unknown tensor '" + name + "'");
    size_t dot = name.find('.', 4);
    HOS_REQUIRE(dot != std::string::npos, HOS_E_INVALID, "unknown tensor '" + name + "'");
    const int l = std::atoi(name.substr(4, dot - 4).c_str());
    HOS_REQUIRE(l >= 0 && l < L, HOS_E_INVALID, "layer index out of range in '" + name + "'");
    const std::string leaf = name.substr(dot + 1);
    const char* wn[NW] = {"attn_q.weight", "attn_k.weight", "attn_v.weight", "attn_output.weight",
                          "ffn_gate.weight", "ffn_up.weight", "ffn_down.weight"};
    for (int t = 0; t < NW; t++)
      if (leaf == wn[t]) {
        int o, i;
        wdims(t, &o, &i);
        *count = (size_t)o * i;
        return W(l, t);
      }
    const char* vn[NV] = {"attn_norm.weight", "ffn_norm.weight", "attn_q.bias", "attn_k.bias", "attn_v.bias"};
    for (int t = 0; t < NV; t++)
      if (leaf == vn[t]) {
        HOS_REQUIRE(Vp(l, t) != nullptr, HOS_E_INVALID, "tensor '" + name + "' not in this model (attn_bias = 0)");
        *count = vdim(t);
        return Vp(l, t);
      }
    throw Error(HOS_E_INVALID, "unknown tensor '" + name + "'");
  }
  void set_tensor(const std::string& name, const uint8_t* bytes, size_t nbytes, uint32_t type, size_t rows,
                  size_t cols) {
    HOS_REQUIRE(bytes != nullptr, HOS_E_INVALID, "null bytes");
    size_t cnt = 0;
    float* dst = slot_of(name, &cnt);
    HOS_REQUIRE(rows * cols == cnt, HOS_E_FORMAT, "tensor '" + name + "' has " + std::to_string(rows * cols) +
                                                      " elements, expected " + std::to_string(cnt));
    if (type == GGUF_F32) {
      HOS_REQUIRE(nbytes == cnt * 4, HOS_E_FORMAT, "tensor '" + name + "' byte count");
      HOS_HIP_CHECK(hipMemcpyAsync(dst, bytes, nbytes, hipMemcpyHostToDevice, st));
    } else {  // dequantized once at load (Weight::to_f32, src/model.rs:251-273)
      QWeight q;
      upload_qweight(st, bytes, nbytes, type, rows, cols, q);
      launch_dequant(q, dst, st);
      HOS_HIP_CHECK(hipStreamSynchronize(st));
      free_qweight(q);
    }
    if (name == "token_embd.weight") {
      tok_set = true;
      if (!out_set)  // FtModel's head: an untied copy of the tied embedding
        HOS_HIP_CHECK(hipMemcpyAsync(P + o_out, dst, cnt * 4, hipMemcpyDeviceToDevice, st));
    }
    if (name == "output.weight") out_set = true;
    seen[name] = true;
    HOS_HIP_CHECK(hipStreamSynchronize(st));
  }
  void check_ready() {
    HOS_REQUIRE(tok_set, HOS_E_MISSING_TENSOR, "missing tensor 'token_embd.weight'");
    HOS_REQUIRE(seen.count("output_norm.weight"), HOS_E_MISSING_TENSOR, "missing tensor 'output_norm.weight'");
    const char* wn[NW] = {"attn_q.weight", "attn_k.weight", "attn_v.weight", "attn_output.weight",
                          "ffn_gate.weight", "ffn_up.weight", "ffn_down.weight"};
    for (int l = 0; l < L; l++)
      for (int t = 0; t < NW; t++) {
        const std::string nm = "blk." + std::to_string(l) + "." + wn[t];
        HOS_REQUIRE(seen.count(nm), HOS_E_MISSING_TENSOR, "missing tensor '" + nm + "'");
      }
  }

  // ---- GEMM helpers (row-major, weights [out, in]) ----
  // The forward and input-gradient GEMMs run on the quantized-weight GEMM with the f32 weight as its (unscaled)
  // layout, in 3 precision passes: the activation (or dY) and the weight each split into fp16 hi + lo (~22 bits,
  // the activation with a power-of-two row scale), A_hi·W_hi + A_lo·W_hi + A_hi·W_lo with fp32 accumulation —
  // the f32 result to ~2^-22 relative per product, on fp16 MFMA (16× the fp32-MFMA rate per pass).
  QWeight wview(const float* Wt, int o, int i) const {
    QWeight w;
    w.type = GGUF_F32;
    w.rows = o;
    w.cols = i;
    w.q = (void*)Wt;
    return w;
  }
  // Y[M, o] (beta: 0 overwrite / 1 accumulate) = X[M, i] · Wᵀ; same_x: X is the previous call's X, unchanged since,
  // so the operand it left in ah is reused
  void fwd(const float* X, long long ldx, const float* Wt, int o, int i, int M, float beta, float* Y, long long ldy,
           bool same_x = false) {
    if (!same_x) launch_to_h16(X, ldx, M, i, ah, st);
    GemmEpi e{Y, ldy, nullptr, beta != 0.0f ? 1 : 0, nullptr};
    launch_qgemm_fwd(wview(Wt, o, i), ah, i, M, e, ws, ws_bytes, 3, st);
  }
  // dX[M, i] (+)= dY[M, o] · W
  void bwd_x(const float* dY, long long ldd, const float* Wt, int o, int i, int M, float beta, float* dX,
             long long ldx) {
    launch_to_h16(dY, ldd, M, o, ah, st);
    GemmEpi e{dX, ldx, nullptr, beta != 0.0f ? 1 : 0, nullptr};
    launch_qgemm_dx(wview(Wt, o, i), ah, o, M, e, ws, ws_bytes, 3, st);
  }
  // dW[o, i] = dY[M, o]ᵀ · X[M, i]: the dX-form GEMM over the tokens (dYᵀ as the operand, X as an f32 weight of M
  // rows), in 3 passes like the others; when the token count is not a multiple of 32 (the GEMM's contraction step)
  // or X is not packed, the f32 GEMM
  void bwd_w(const float* dY, long long ldd, const float* X, long long ldx, int o, int i, int M, float* dWt) {
    if (M % 32 != 0 || ldx != i) {
      launch_gemm_f32(o, i, M, 1.0f, dY, 1, ldd, X, ldx, 1, 0.0f, dWt, i, ws, ws_bytes, st);
      return;
    }
    HOS_REQUIRE((size_t)o <= tr_rows && (size_t)o * M <= ah_n, HOS_E_INVALID, "finetune: dYᵀ operand exceeds its buffer");
    const int nch = ceil_div(M, COLSUM_CH);
    HOS_REQUIRE((size_t)nch * o <= cpart_n, HOS_E_INVALID, "finetune: column maxima exceed their buffer");
    colmax_kernel<<<dim3(ceil_div(o, 256), nch), 256, 0, st>>>(dY, ldd, M, o, cpart);
    HOS_HIP_CHECK(hipGetLastError());
    const H16 at{ah.data, tr_rinv, ah.lo};
    transpose_h16_kernel<<<dim3(ceil_div(o, 64), ceil_div(M, 64)), 256, 0, st>>>(dY, ldd, M, o, cpart, nch, at.data,
                                                                                  at.lo, at.rinv);
    HOS_HIP_CHECK(hipGetLastError());
    GemmEpi e{dWt, i, nullptr, 0, nullptr};
    launch_qgemm_dx(wview(X, M, i), at, M, o, e, ws, ws_bytes, 3, st);
  }
  void colsum(const float* g, long long ldg, const float* x, long long ldx, const float* inv, int M, int nc,
              float* out) {
    const int nch = ceil_div(M, COLSUM_CH);
    HOS_REQUIRE((size_t)nch * nc <= csp_n, HOS_E_INVALID, "finetune: column-sum partials exceed their buffer");
    colsum_part_kernel<<<dim3(ceil_div(nc, 256), nch), 256, 0, st>>>(g, ldg, x, ldx, inv, M, nc, csp);
    HOS_HIP_CHECK(hipGetLastError());
    colsum_fold_kernel<<<ceil_div(nc, 256), 256, 0, st>>>(csp, nch, nc, out);
    HOS_HIP_CHECK(hipGetLastError());
  }
  void add_bias(float* y, long long ld, int M, int nc, const float* b) {
    add_bias_kernel<<<ceil_div((long long)M * nc, 256), 256, 0, st>>>(y, ld, M, nc, b);
    HOS_HIP_CHECK(hipGetLastError());
  }

  // ---- forward (FtModel::hidden + head) ----
  void forward(int B, int T) {
    const int M = B * T;
    embed_f32_kernel<<<ceil_div((long long)M * d, 256), 256, 0, st>>>(P + o_tok, ids, M, d, act[0].x);
    HOS_HIP_CHECK(hipGetLastError());
    for (int l = 0; l < L; l++) {
      Act& a = act[l];
      float* xnext = (l + 1 < L) ? act[l + 1].x : xf;
      launch_rmsnorm_fwd(a.x, Vp(l, NA), c.rms_eps, M, d, a.xn1, hs, a.inv1, st);
      fwd(a.xn1, d, W(l, WQ), qd, d, M, 0.0f, a.qkv, W3);
      fwd(a.xn1, d, W(l, WK), kvd, d, M, 0.0f, a.qkv + qd, W3, true);
      fwd(a.xn1, d, W(l, WV), kvd, d, M, 0.0f, a.qkv + qd + kvd, W3, true);
      if (c.attn_bias) {
        add_bias(a.qkv, W3, M, qd, Vp(l, BQ));
        add_bias(a.qkv + qd, W3, M, kvd, Vp(l, BK));
        add_bias(a.qkv + qd + kvd, W3, M, kvd, Vp(l, BV));
      }
      // the k heads follow the q heads in the row (qd = n_heads·head_dim): one launch rotates both
      launch_rope(a.qkv, W3, 0, c.n_heads + c.n_kv_heads, c.head_dim, T, rope_tab, c.rope_neox, false, M, st);
      launch_attn_fwd(a.qkv, W3, qd, qd + kvd, B, T, c.n_heads, c.n_kv_heads, c.head_dim, a.o, qd, a.lse, attn_planes,
                      st);
      launch_copy_rows(a.x, d, a.x2, d, M, d, st);
      fwd(a.o, qd, W(l, WO), d, qd, M, 1.0f, a.x2, d);
      launch_rmsnorm_fwd(a.x2, Vp(l, NF), c.rms_eps, M, d, a.xn2, hs, a.inv2, st);
      fwd(a.xn2, d, W(l, WG), F, d, M, 0.0f, a.gu, 2LL * F);
      fwd(a.xn2, d, W(l, WU), F, d, M, 0.0f, a.gu + F, 2LL * F, true);
      launch_swiglu_fwd(a.gu, M, F, a.h, hs, st);
      launch_copy_rows(a.x2, d, xnext, d, M, d, st);
      fwd(a.h, F, W(l, WD), d, F, M, 1.0f, xnext, d);
    }
    launch_rmsnorm_fwd(xf, P + o_onorm, c.rms_eps, M, d, xfn, hs, invf, st);
    fwd(xfn, d, P + o_out, V, d, M, 0.0f, logits, V);
  }

  // ---- loss + backward ----
  void loss_backward(int B, int T) {
    const int M = B * T;
    const float gscale = (1.0f / (float)B) / (float)T;
    launch_ce(logits, M, V, tgts, gscale, row_loss, H16{}, st, dl);
    launch_loss_reduce(row_loss, B, T, loss, st);
    bwd_w(dl, V, xfn, d, V, d, M, G + o_out);
    bwd_x(dl, V, P + o_out, V, d, M, 0.0f, dxn, d);
    colsum(dxn, d, xf, d, invf, M, d, G + o_onorm);
    launch_fill(dx, (long long)M * d, 0.0f, st);
    launch_rmsnorm_bwd(dxn, xf, invf, P + o_onorm, M, d, dx, st);
    for (int l = L - 1; l >= 0; l--) {
      Act& a = act[l];
      // FFN: x_{l+1} = x2 + (silu(xn2·Wgᵀ) ⊙ xn2·Wuᵀ)·Wdᵀ
      bwd_w(dx, d, a.h, F, d, F, M, dW(l, WD));
      bwd_x(dx, d, W(l, WD), d, F, M, 0.0f, dh, F);
      launch_swiglu_bwd(a.gu, dh, M, F, dgu, hs, st);
      bwd_w(dgu, 2LL * F, a.xn2, d, F, d, M, dW(l, WG));
      bwd_w(dgu + F, 2LL * F, a.xn2, d, F, d, M, dW(l, WU));
      bwd_x(dgu, 2LL * F, W(l, WG), F, d, M, 0.0f, dxn, d);
      bwd_x(dgu + F, 2LL * F, W(l, WU), F, d, M, 1.0f, dxn, d);
      colsum(dxn, d, a.x2, d, a.inv2, M, d, dV(l, NF));
      launch_rmsnorm_bwd(dxn, a.x2, a.inv2, Vp(l, NF), M, d, dx, st);
      // attention: x2 = x + attn(x)·Woᵀ
      bwd_w(dx, d, a.o, qd, d, qd, M, dW(l, WO));
      bwd_x(dx, d, W(l, WO), d, qd, M, 0.0f, dout, qd);
      launch_attn_bwd(a.qkv, W3, qd, qd + kvd, a.o, dout, qd, a.lse, dvec, B, T, c.n_heads, c.n_kv_heads,
                      c.head_dim, dqkv, W3, part, attn_planes, st);
      // the k heads follow the q heads in the row (qd = n_heads·head_dim): one launch rotates both
      launch_rope(dqkv, W3, 0, c.n_heads + c.n_kv_heads, c.head_dim, T, rope_tab, c.rope_neox, true, M, st);
      if (c.attn_bias) {
        colsum(dqkv, W3, nullptr, 0, nullptr, M, qd, dV(l, BQ));
        colsum(dqkv + qd, W3, nullptr, 0, nullptr, M, kvd, dV(l, BK));
        colsum(dqkv + qd + kvd, W3, nullptr, 0, nullptr, M, kvd, dV(l, BV));
      }
      bwd_w(dqkv, W3, a.xn1, d, qd, d, M, dW(l, WQ));
      bwd_w(dqkv + qd, W3, a.xn1, d, kvd, d, M, dW(l, WK));
      bwd_w(dqkv + qd + kvd, W3, a.xn1, d, kvd, d, M, dW(l, WV));
      bwd_x(dqkv, W3, W(l, WQ), qd, d, M, 0.0f, dxn, d);
      bwd_x(dqkv + qd, W3, W(l, WK), kvd, d, M, 1.0f, dxn, d);
      bwd_x(dqkv + qd + kvd, W3, W(l, WV), kvd, d, M, 1.0f, dxn, d);
      colsum(dxn, d, a.x, d, a.inv1, M, d, dV(l, NA));
      launch_rmsnorm_bwd(dxn, a.x, a.inv1, Vp(l, NA), M, d, dx, st);
    }
    launch_fill(G + o_tok, (long long)V * d, 0.0f, st);
    embed_grad_kernel<<<M, 256, 0, st>>>(ids, M, dx, d, G + o_tok);
    HOS_HIP_CHECK(hipGetLastError());
  }
  void set_hyper(float lr, float wd) {
    hyp_host.lr = lr;
    hyp_host.wd = wd;
    HOS_HIP_CHECK(hipMemcpyAsync(hyp, &hyp_host, 2 * sizeof(float), hipMemcpyHostToDevice, st));
  }
  void adamw_enqueue() {
    adam_t += 1;
    launch_adam_tick(hyp, st);
    launch_adamw_dev(P, G, M1, V1, n2, 0.9f, 0.95f, 1e-8f, hyp, true, st);                 // 2-D: decay
    launch_adamw_dev(P + n2, G + n2, M1 + n2, V1 + n2, n - n2, 0.9f, 0.95f, 1e-8f, hyp, false, st);  // 1-D
  }
  void check_bt(int B, int T) {
    HOS_REQUIRE(B > 0 && T > 0 && T <= c.max_seq && B * T <= Mmax, HOS_E_INVALID,
                "batch " + std::to_string(B) + " x seq " + std::to_string(T) + " exceeds max_batch/max_seq");
  }
};

namespace {
template <class Fn>
int fguard(hos_ft* p, Fn&& f) {
  if (!p) return HOS_E_INVALID;
  try {
    HOS_HIP_CHECK(hipSetDevice(hos_internal_device(p->ctx)));
    f();
    p->err.clear();
    return HOS_OK;
  } catch (const Error& e) {
    p->err = e.what();
    return e.code;
  } catch (const std::bad_alloc&) {
    p->err = "host allocation failed";
    return HOS_E_OOM;
  } catch (const std::exception& e) {
    p->err = e.what();
    return HOS_E_DEVICE;
  }
}
void check_ids(hos_ft* p, const int32_t* v, int cnt) {
  for (int i = 0; i < cnt; i++)
    HOS_REQUIRE(v[i] >= 0 && v[i] < p->V, HOS_E_INVALID, "token id " + std::to_string(v[i]) + " out of range");
}
}  // namespace

extern "C" {

int hos_ft_create(hos_ctx* ctx, const hos_peft_cfg* cfg, hos_ft** out) {
  if (!ctx || !cfg || !out) return HOS_E_INVALID;
  *out = nullptr;
  auto* p = new hos_ft();
  p->ctx = ctx;
  int rc = fguard(p, [&] { p->init(ctx, cfg); });
  if (rc) {
    std::fprintf(stderr, "hos_ft_create: %s\n", p->err.c_str());
    p->release();
    delete p;
    return rc;
  }
  *out = p;
  return HOS_OK;
}
void hos_ft_destroy(hos_ft* p) {
  if (!p) return;
  (void)hipSetDevice(hos_internal_device(p->ctx));
  p->release();
  delete p;
}
const char* hos_ft_last_error(const hos_ft* p) { return p ? p->err.c_str() : "null model"; }
int hos_ft_set_tensor(hos_ft* p, const char* name, const uint8_t* bytes, size_t nbytes, uint32_t type, size_t rows,
                      size_t cols) {
  return fguard(p, [&] {
    HOS_REQUIRE(name != nullptr, HOS_E_INVALID, "null name");
    p->set_tensor(name, bytes, nbytes, type, rows, cols);
  });
}
int hos_ft_get(hos_ft* p, const char* name, float* value, float* grad) {
  return fguard(p, [&] {
    HOS_REQUIRE(name != nullptr, HOS_E_INVALID, "null name");
    size_t cnt = 0;
    float* v = p->slot_of(name, &cnt);
    if (value) HOS_HIP_CHECK(hipMemcpyAsync(value, v, cnt * 4, hipMemcpyDeviceToHost, p->st));
    if (grad) HOS_HIP_CHECK(hipMemcpyAsync(grad, p->G + (v - p->P), cnt * 4, hipMemcpyDeviceToHost, p->st));
    HOS_HIP_CHECK(hipStreamSynchronize(p->st));
  });
}
int hos_ft_loss_grad(hos_ft* p, const int32_t* ids, const int32_t* targets, int B, int T, float* loss) {
  return fguard(p, [&] {
    HOS_REQUIRE(ids && targets && loss, HOS_E_INVALID, "null pointer");
    p->check_ready();
    p->check_bt(B, T);
    check_ids(p, ids, B * T);
    check_ids(p, targets, B * T);
    HOS_HIP_CHECK(hipMemcpyAsync(p->ids, ids, (size_t)B * T * 4, hipMemcpyHostToDevice, p->st));
    HOS_HIP_CHECK(hipMemcpyAsync(p->tgts, targets, (size_t)B * T * 4, hipMemcpyHostToDevice, p->st));
    p->forward(B, T);
    p->loss_backward(B, T);
    HOS_HIP_CHECK(hipMemcpyAsync(loss, p->loss, 4, hipMemcpyDeviceToHost, p->st));
    HOS_HIP_CHECK(hipStreamSynchronize(p->st));
  });
}
int hos_ft_adamw(hos_ft* p, float lr, float wd) {
  return fguard(p, [&] {
    p->set_hyper(lr, wd);
    p->adamw_enqueue();
    HOS_HIP_CHECK(hipStreamSynchronize(p->st));
  });
}
int hos_ft_step_dev(hos_ft* p, const int32_t* ids_dev, const int32_t* targets_dev, int B, int T, float lr, float wd,
                    float* loss_dev) {
  return fguard(p, [&] {
    HOS_REQUIRE(ids_dev && targets_dev, HOS_E_INVALID, "null pointer");
    p->check_ready();
    p->check_bt(B, T);
    HOS_HIP_CHECK(hipMemcpyAsync(p->ids, ids_dev, (size_t)B * T * 4, hipMemcpyDeviceToDevice, p->st));
    HOS_HIP_CHECK(hipMemcpyAsync(p->tgts, targets_dev, (size_t)B * T * 4, hipMemcpyDeviceToDevice, p->st));
    p->forward(B, T);
    p->loss_backward(B, T);
    p->set_hyper(lr, wd);
    p->adamw_enqueue();
    if (loss_dev) HOS_HIP_CHECK(hipMemcpyAsync(loss_dev, p->loss, 4, hipMemcpyDeviceToDevice, p->st));
  });
}

}  // extern "C"
