// Device-resident LoRA training step: PeftModel (src/peft.rs) + AdamW (src/tensor.rs:2923-2976) on gfx950.
//
// The reference builds a dynamic autograd graph per sequence and walks it in reverse
// (src/tensor.rs:2844-2881). Here the graph of PeftModel::forward (src/peft.rs:474-604) is fixed, so
// the forward and its reverse pass are a static schedule of kernels over all B·T rows at once: the
// reference's batch is B sequences accumulated with loss·(1/B) (src/main.rs:2583-2596), which is the
// same sum as one pass over B·T rows with the CE gradient scaled by 1/(B·T) and attention kept
// within each sequence. Everything stays in HBM between kernels; the host only enqueues.
//
// Frozen linear weights: quantized (Q8_0/Q4_K/Q6_K), dequantized inside the fp16-MFMA GEMMs.
// LoRA factors, their gradients and AdamW moments: one flat f32 arena, updated by one kernel.
#include <cmath>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "ctx.hpp"
#include "peft_internal.hpp"
#include "fused.hpp"
#include "lora.hpp"
#include "moe.hpp"
#include "rga.hpp"

using namespace hos;

namespace {
// Precision modes that carry the activation as fp16 hi + lo (the operand's residual plane is needed).
static inline bool alo_mode(int m) { return m == 2 || m == 3 || m == 5; }


// LoRA targets in order: q k v o gate up down.
enum { TQ, TK, TV, TO, TG, TU, TD, NT };

struct LayerW {
  QWeight w[NT];                // base projection per target slot
  float* attn_norm = nullptr;   // [d]
  float* ffn_norm = nullptr;    // [d]
  float* bias[3] = {nullptr, nullptr, nullptr};  // q k v
  float *q_norm = nullptr, *k_norm = nullptr;     // OLMoE QK-norm weights [qd], [kvd]
  float* router = nullptr;                        // MoE router [E][d] (f32, ffn_gate_inp.weight)
  QWeight xg, xu, xd;                             // MoE experts, stacked [E·F][d], [E·F][d], [E·d][F]
  QWeight xgu;  // MoE gate|up interleaved per expert, [E·2F][d]: expert e's gate rows then its up rows
  // q|k|v and gate|up stacked row-wise (same encoding and width), each group one GEMM; the q|k|v biases
  // concatenated. Absent when the parts differ in encoding.
  QWeight qkv, gu;
  float* bias_qkv = nullptr;
};

struct LayerAct {
  float *x, *xn1, *inv1, *qkv, *o, *lse, *x2, *xn2, *inv2, *gu, *h, *u;
  // the SwiGLU output as the down projection's fp16 operand, kept for the layer's backward (replaces h when the
  // precision modes carry the residual plane: the down GEMM, its LoRA down-projection and its dA all read it)
  H16 hd{nullptr, nullptr, nullptr};
  float *qk_pre = nullptr, *qk_inv = nullptr;  // QK-norm: pre-norm q|k [M][qd+kvd], 1/rms [2][M]
  // RGA: residual before the adapter [M][d], gates | relu'd bottlenecks [M][Rp], H ⊙ gate [M][Kbp]
  float *xr = nullptr, *ra = nullptr, *hg = nullptr;
  // MoE: softmax [M][E], selections [M][K] (expert, probability, slot, expert-order row), per-expert
  // counts / offsets, grouped-GEMM schedule, expert pre-activations [P][2F] and outputs [P][d] (P = M·K)
  float *pfull = nullptr, *sel_p = nullptr, *gug = nullptr, *yg = nullptr;
  int *sel_e = nullptr, *slot = nullptr, *pos = nullptr, *counts = nullptr, *offsets = nullptr, *tiles = nullptr;
};

struct ProfRec {
  std::string cls;
  hipEvent_t e0, e1;
  double flops, bytes;
};
struct ProfAcc {
  long long launches = 0;
  double ms = 0, flops = 0, bytes = 0;
};

}  // namespace

struct hos_peft {
  hos_ctx* ctx = nullptr;
  hipStream_t st = nullptr;
  hos_peft_cfg c{};
  std::string err;
  int d = 0, qd = 0, kvd = 0, W3 = 0, F = 0, V = 0, r = 0, L = 0, Mmax = 0, passes = 3;
  int pf = 3, pd = 3, phf = 3, phd = 3;  // precision mode per GEMM site: layer fwd / dX, head fwd / dX
  ColsJob pend_db;       // dB of the group whose backward is in progress, launched with its dA
  ColsBatch cbatch;      // a layer's dA/dB partials, reduced in one launch at the end of the layer
  int pend_group = -1;
  // Whole-backward batching of the LoRA dA / dB products (dense LoRA models with two-plane operands): every layer
  // keeps the inputs those products read — its du, the q|k|v output gradient, the residual gradients at x2 and at
  // x_{l+1}, the fp16 d(gate|up) — and the products of all layers run together after the last layer, in a few
  // launches without a split of M (launch_lora_cols_table) instead of five small launches per layer.
  bool gbatch = false;
  std::vector<float*> du_l, dqkv_l, dxs_l, dx2s_l;  // per layer; dxs_l[l]: gradient at x_{l+1}, dx2s_l[l]: at x2
  std::vector<H16> dgu16_l;                         // per layer: d(gate|up) as the fp16 operand
  std::vector<ColsJob> gjobs;                       // the step's queued dA / dB products
  ColsTable gtab;                                   // their device table (launch_lora_cols_table)
  int tpf[7] = {0, 0, 0, 0, 0, 0, 0}, tpd[7] = {0, 0, 0, 0, 0, 0, 0};  // per-target overrides (0 = site mode)
  float lscale = 0.0f;

  std::vector<LayerW> lw;
  int E = 0, K = 0, max_tiles = 0;  // MoE: experts, experts per token, grouped-GEMM schedule length
  H16 hx{};                         // MoE operand scratch [M·K][max(d, 2F)]
  float *mlogits = nullptr, *mdY = nullptr, *mdH = nullptr, *mdX = nullptr, *mdp = nullptr, *mdl = nullptr;
  QWeight tok, out;
  bool out_set = false;
  float* out_norm = nullptr;
  bool stacks_dirty = true;  // a projection or bias changed since the stacked copies were built

  // LoRA arena offsets (floats): per (layer, group) the stacked At and Bcat blocks; per (layer, target)
  // the first row of A_tᵀ in At and the first column of B_t in Bcat; -1 when not adapted
  std::vector<long long> offAg, offBg, offA, offB;
  long long nparams = 0;
  // RGA (rga_genes > 0): Kg genes of bottleneck bn per layer; stacked factors RT [Rp][d] (W_rᵀ rows, then each
  // down_kᵀ) and Up [Kbp][d] (each up_k) per layer, wg [8][Kg] and the genome [8]; widths padded to 4.
  bool rga = false;
  int Kg = 0, bn = 0, Rp = 0, Kbp = 0;
  float rlambda = 0.0f;
  long long offWg = -1, offGen = -1;
  std::vector<long long> offRT, offUp;
  float *rz = nullptr, *rdg = nullptr, *rgb = nullptr, *rdgb = nullptr, *rgsum = nullptr, *rgm = nullptr;
  float *P = nullptr, *G = nullptr, *M1 = nullptr, *V1 = nullptr;
  // fp16 hi/lo split of the LoRA factors (arena-parallel), one power-of-two scale per factor row: At rows of a
  // group from scA, Bcat rows from scB; written at the start of each forward from the table split_tab.
  _Float16 *P16h = nullptr, *P16l = nullptr;
  float* psc = nullptr;
  std::vector<int> scA, scB;
  SplitRow* split_tab = nullptr;
  int n_split = 0;
  long long nfac = 0;
  uint64_t adam_t = 0;

  std::vector<LayerAct> act;
  float* xfinal = nullptr;  // residual stream after the last layer
  float* invf = nullptr;
  H16 hs{};                 // fp16 operand scratch [Mmax, hs_cols]
  float* logits = nullptr;
  float2* lstat = nullptr;  // (max, exp-sum) of each 64-column chunk of the logit rows, from the head GEMM
  H16 dl{};
  float *row_loss = nullptr, *loss = nullptr;
  float *dx = nullptr, *dxn = nullptr, *dqkv = nullptr, *dout = nullptr, *dh = nullptr, *dgu = nullptr,
        *du = nullptr, *dvec = nullptr, *attn_part = nullptr;
  // bf16 hi/lo planes of q, k, v (attention scratch), one per layer: the backward reuses the q, k, v planes
  // its layer's forward made
  std::vector<void*> attn_planes;
  float* ws = nullptr;
  size_t ws_bytes = 0;
  // Partials of the split GEMMs whose reduction the next row kernel performs (the FFN down projection's forward,
  // the stacked gate|up dX, the vocabulary head's dX): a workspace of their own, so that launches in between (the
  // LoRA dA/dB partials) cannot overwrite them.
  float* ws2 = nullptr;
  SplitSrc xsrc{};  // the residual row source the next forward RMSNorm forms and stores
  float2* rope_tab = nullptr;
  int32_t *ids = nullptr, *tgts = nullptr;
  std::vector<void*> allocs;

  // AdamW hyper-parameters in device memory (lr, wd written before each step; t advanced on the device)
  AdamHyper* hyp = nullptr;
  AdamHyper hyp_host{};
  // Captured optimizer steps, keyed by (B, T, ids, targets, loss) device pointers.
  bool use_graph = true;
  std::map<std::vector<uintptr_t>, hipGraphExec_t> graphs;
  bool prof = false;
  std::string prof_only;  // when set, only this kernel class is timed
  std::vector<ProfRec> recs;
  std::map<std::string, ProfAcc> acc;

  // ---------------- helpers ----------------
  template <class T>
  T* alloc(size_t n) {
    void* p = nullptr;
    if (n == 0) n = 1;
    hipError_t e = hipMalloc(&p, n * sizeof(T));
    if (e != hipSuccess) throw Error(HOS_E_OOM, "hipMalloc(" + std::to_string(n * sizeof(T)) + ") failed");
    allocs.push_back(p);
    return (T*)p;
  }
  bool has(int t) const { return (c.lora_targets >> t) & 1u; }
  void dims(int t, int* in, int* outd) const {
    switch (t) {
      case TQ: *in = d; *outd = qd; break;
      case TK: *in = d; *outd = kvd; break;
      case TV: *in = d; *outd = kvd; break;
      case TO: *in = qd; *outd = d; break;
      case TG: *in = d; *outd = F; break;
      case TU: *in = d; *outd = F; break;
      default: *in = F; *outd = d; break;
    }
  }

  struct Scope {
    hos_peft* p;
    hipEvent_t e0{}, e1{};
    const char* cls;
    double fl, by;
    bool on;
    Scope(hos_peft* p_, const char* cls_, double fl_, double by_)
        : p(p_), cls(cls_), fl(fl_), by(by_), on(p_->prof && (p_->prof_only.empty() || p_->prof_only == cls_)) {
      if (on) {
        HOS_HIP_CHECK(hipEventCreate(&e0));
        HOS_HIP_CHECK(hipEventCreate(&e1));
        HOS_HIP_CHECK(hipEventRecord(e0, p->st));
      }
    }
    ~Scope() {
      if (on) {
        (void)hipEventRecord(e1, p->st);
        p->recs.push_back(ProfRec{cls, e0, e1, fl, by});
      }
    }
  };

  double wbytes(const QWeight& w) const { return (double)(w.q_bytes + w.s_bytes); }

  // fp16 GEMMs on frozen weights
  // `lo` carries an optional fused LoRA rank-r update (GemmEpi U/L fields).
  void qfwd(const QWeight& w, H16 a, long long lda, int M, float* out, long long ldo, const float* bias,
            const float* resid, int accumulate, GemmEpi lo = GemmEpi{}, int np = 0) {
    // algorithmic flops (2·M·N·K), independent of the precision passes
    Scope s(this, "qgemm_fwd", 2.0 * M * w.rows * w.cols,
            2.0 * M * w.cols + wbytes(w) + 4.0 * M * w.rows * (resid || accumulate ? 2 : 1));
    GemmEpi e = lo;
    e.out = out;
    e.ldo = ldo;
    e.bias = bias;
    e.accumulate = accumulate;
    e.resid = resid;
    launch_qgemm_fwd(w, a, lda, M, e, ws, ws_bytes, np ? np : pf, st);
  }
  void qdx(const QWeight& w, H16 a, long long lda, int M, float* out, long long ldo, int accumulate,
           GemmEpi lo = GemmEpi{}, int np = 0) {
    Scope s(this, "qgemm_dx", 2.0 * M * w.rows * w.cols,
            2.0 * M * w.rows + wbytes(w) + 4.0 * M * w.cols * (accumulate ? 2 : 1));
    GemmEpi e = lo;
    e.out = out;
    e.ldo = ldo;
    e.bias = nullptr;
    e.accumulate = accumulate;
    e.resid = nullptr;
    launch_qgemm_dx(w, a, lda, M, e, ws, ws_bytes, np ? np : pd, st);
  }
  // A GEMM whose split-K reduction (if the tile rule splits it) is left to the row kernel that consumes its output:
  // returns the partials as a SplitSrc (splits = 0 when the launch was not split and wrote out itself). The output
  // must be dense (ldo = its width), unbiased and not accumulated.
  SplitSrc deferred(bool dx, const QWeight& w, H16 a, long long lda, int M, float* out, long long ldo,
                    const float* resid, GemmEpi lo, int np) {
    const long long N = dx ? w.cols : w.rows;
    HOS_REQUIRE(ldo == N, HOS_E_INVALID, "peft: a deferred reduction needs a dense output");
    Scope s(this, dx ? "qgemm_dx" : "qgemm_fwd", 2.0 * M * w.rows * w.cols,
            2.0 * M * (dx ? w.rows : w.cols) + wbytes(w) + 4.0 * M * N * (resid ? 2 : 1));
    GemmEpi e = lo;
    e.out = out;
    e.ldo = ldo;
    e.bias = nullptr;
    e.accumulate = 0;
    e.resid = resid;
    int splits = 1;
    e.defer = &splits;
    if (dx)
      launch_qgemm_dx(w, a, lda, M, e, ws2, ws_bytes, np ? np : pd, st);
    else
      launch_qgemm_fwd(w, a, lda, M, e, ws2, ws_bytes, np ? np : pf, st);
    SplitSrc src{};
    if (splits > 1) {
      src.ws = ws2;
      src.splits = splits;
      src.mn = (long long)M * N;
      src.rinv = a.rinv;
      src.resid = resid;
    }
    return src;
  }
  void to16(const float* x, long long ldx, int M, int K) {
    Scope s(this, "convert", 0, 6.0 * M * K);
    launch_to_h16(x, ldx, M, K, hs, st);
  }

  // ---- LoRA pieces (reference factors: A [in, r], B [r, out]) ----
  // Targets sharing an input form a group (q/k/v, o, gate/up, down). Per layer and group the arena
  // holds the adapted targets' A factors transposed and stacked, At [G·r][in] (row slot·r + j is
  // column j of A_t), then their B factors side by side, Bcat [r][Σ out] (B_t at column bcol(t)).
  // One rows-GEMM gives u = x·[A_1 … A_G] for the whole group, one cols-GEMM gives every dA, one
  // cols-GEMM every dB and one rows-GEMM every du. u and du live in [M, 7·r] buffers, target t at
  // column ucol(t).
  static int group_of(int t) { return t <= TV ? 0 : (t == TO ? 1 : (t <= TU ? 2 : 3)); }
  static int group_first(int g) { return g == 0 ? TQ : (g == 1 ? TO : (g == 2 ? TG : TD)); }
  static int group_last(int g) { return g == 0 ? TV : (g == 1 ? TO : (g == 2 ? TU : TD)); }
  int gcount(int g) const {
    int n = 0;
    for (int t = group_first(g); t <= group_last(g); t++) n += has(t);
    return n;
  }
  int slot(int t) const {
    int n = 0;
    for (int u = group_first(group_of(t)); u < t; u++) n += has(u);
    return n;
  }
  int first_adapted(int g) const {
    int t = group_first(g);
    while (t <= group_last(g) && !has(t)) t++;
    return t;
  }
  int ucol(int t) const { return group_first(group_of(t)) * r + slot(t) * r; }
  int out_dim(int t) const {
    int in, o;
    dims(t, &in, &o);
    return o;
  }
  int in_dim(int t) const {
    int in, o;
    dims(t, &in, &o);
    return in;
  }
  // Bcat width of a group and column of target t in it
  int bw(int g) const {
    int w = 0;
    for (int t = group_first(g); t <= group_last(g); t++)
      if (has(t)) w += out_dim(t);
    return w;
  }
  int bcol(int t) const {
    int w = 0;
    for (int u = group_first(group_of(t)); u < t; u++)
      if (has(u)) w += out_dim(u);
    return w;
  }
  // column of target t's output inside the buffer its group's projections write (fused q|k|v, gate|up)
  int ycol(int t) const { return t == TK ? qd : (t == TV ? qd + kvd : (t == TU ? F : 0)); }

  void lora_rows(const char* cls, long long M, long long K, float alpha, const float* X, long long ldx,
                 const float* Bt, long long ldb, const RowsSeg& sg, float* C, long long ldc, HIn xh = HIn{},
                 B16 b16 = B16{}) {
    Scope s(this, cls, 2.0 * M * K * sg.nt * sg.r, 4.0 * (M * K + (double)M * sg.nt * sg.r));
    launch_lora_rows(M, K, alpha, X, ldx, Bt, ldb, sg, C, ldc, ws, ws_bytes, st, xh, b16);
  }
  // The fp16 operand of the activation the current GEMM reads (when it carries the residual plane) and the
  // factor split of a group's At (a) or Bcat: the LoRA rows products then run on fp16 MFMA.
  HIn hs_in() const { return hs.lo ? HIn{hs.data, hs.lo, hs.rinv} : HIn{}; }
  float* du_of(int l) const { return gbatch ? du_l[l] : du; }
  B16 fac16(int l, int g, bool a) const {
    const long long off = a ? offAg[l * 4 + g] : offBg[l * 4 + g];
    return B16{P16h + off, P16l + off, psc + (a ? scA : scB)[l * 4 + g]};
  }
  void split_factors() {
    if (n_split == 0) return;
    Scope s(this, "convert", 0, 8.0 * nfac);
    launch_split_rows16(split_tab, n_split, P, P16h, P16l, psc, st);
  }
  void lora_cols(const char* cls, long long M, int ns, float alpha, const float* Sm, long long lds, const float* Gm,
                 long long ldg, const ColsSeg& sg, float* C, long long scj, long long scc) {
    double cols = 0;
    for (int t = 0; t < sg.nseg; t++) cols += sg.len[t];
    Scope s(this, cls, 2.0 * M * ns * cols, 4.0 * (M * cols + (double)M * ns + ns * cols));
    launch_lora_cols(M, ns, alpha, Sm, lds, Gm, ldg, sg, C, scj, scc, ws, ws_bytes, st);
  }

  // u[:, group columns] = x · [A_1 … A_G]   (forward)
  // xh: x as the fp16 operand (row stride ldx)
  void lora_down(int l, int g, const float* x, long long ldx, int M, HIn xh = HIn{}) {
    const int n = gcount(g);
    if (n == 0) return;
    const int first = first_adapted(g), in = in_dim(first);
    RowsSeg sg;
    sg.nt = n;
    sg.r = r;
    for (int i = 0; i < n; i++) {
      sg.kbeg[i] = 0;
      sg.kend[i] = in;
      sg.boff[i] = (long long)i * r * in;
    }
    lora_rows("lora_down", M, in, 1.0f, x, ldx, P + offAg[l * 4 + g], in, sg, act[l].u + ucol(first), NT * r, xh,
              xh.hi ? fac16(l, g, true) : B16{});
  }
  // Epilogue term y += s·u_t·B_t of the base forward GEMM: L(j, n) = Bcat[j·bw + bcol(t) + n]
  GemmEpi up_epi(int l, int t) {
    GemmEpi e{};
    if (!has(t)) return e;
    e.U = act[l].u + ucol(t);
    e.ldu = NT * r;
    e.L = P + offB[l * NT + t];
    e.slj = bw(group_of(t));
    e.sln = 1;
    e.rank = r;
    e.scale = lscale;
    return e;
  }
  // A group's projections as one stacked GEMM: possible when its targets are all adapted or none is (the
  // stacked output lines up with Bcat / the stacked At only then), the per-target precision overrides agree,
  // and (dX) the stacked rank fits the fused epilogue.
  bool group_uniform(int g) const {
    const int n = gcount(g), all = group_last(g) - group_first(g) + 1;
    if (n != 0 && n != all) return false;
    for (int t = group_first(g) + 1; t <= group_last(g); t++)
      if (tpf[t] != tpf[group_first(g)] || tpd[t] != tpd[group_first(g)]) return false;
    return true;
  }
  // Forward epilogue of a stacked group: each column segment adds its own target's s·u_t·B_t
  // (u_t at column ucol(first) + slot·r, B_t the matching Bcat columns).
  GemmEpi stacked_up_epi(int l, int g) {
    GemmEpi e{};
    if (gcount(g) == 0) return e;
    const int t0 = group_first(g);
    e.U = act[l].u + ucol(t0);
    e.ldu = NT * r;
    e.L = P + offBg[l * 4 + g];
    e.slj = bw(g);
    e.sln = 1;
    e.rank = r;
    e.scale = lscale;
    e.ustep = r;
    e.ub0 = out_dim(t0);
    e.ub1 = g == 0 ? out_dim(TQ) + out_dim(TK) : 1 << 30;
    return e;
  }
  // dX epilogue of a stacked group: dx_in += [du_1 … du_G]·[A_1ᵀ; …; A_Gᵀ], one rank-G·r term (At block).
  GemmEpi stacked_down_epi(int l, int g) {
    GemmEpi e{};
    if (gcount(g) == 0) return e;
    e.U = du_of(l) + ucol(group_first(g));
    e.ldu = NT * r;
    e.L = P + offAg[l * 4 + g];
    e.slj = in_dim(group_first(g));
    e.sln = 1;
    e.rank = gcount(g) * r;
    e.scale = 1.0f;
    return e;
  }
  // (Re)build the stacked copies of every layer (host side, before a step; never inside a capture).
  void build_stacks() {
    if (!stacks_dirty) return;
    // captured steps hold the old weight pointers (a re-uploaded tensor has new ones too): capture again
    for (auto& kv : graphs) (void)hipGraphExecDestroy(kv.second);
    graphs.clear();
    for (int l = 0; l < L; l++) {
      LayerW& w = lw[l];
      free_qweight(w.qkv);
      free_qweight(w.gu);
      free_qweight(w.xgu);
      stack(w.qkv, {&w.w[TQ], &w.w[TK], &w.w[TV]});
      if (!E) stack(w.gu, {&w.w[TG], &w.w[TU]});
      if (E) stack_experts(w.xgu, w.xg, w.xu);
      if (c.attn_bias && w.bias[0] && w.bias[1] && w.bias[2]) {
        if (!w.bias_qkv) w.bias_qkv = alloc<float>((size_t)W3);
        HOS_HIP_CHECK(hipMemcpyAsync(w.bias_qkv, w.bias[0], (size_t)qd * 4, hipMemcpyDeviceToDevice, st));
        HOS_HIP_CHECK(hipMemcpyAsync(w.bias_qkv + qd, w.bias[1], (size_t)kvd * 4, hipMemcpyDeviceToDevice, st));
        HOS_HIP_CHECK(hipMemcpyAsync(w.bias_qkv + qd + kvd, w.bias[2], (size_t)kvd * 4, hipMemcpyDeviceToDevice, st));
      }
    }
    HOS_HIP_CHECK(hipStreamSynchronize(st));
    stacks_dirty = false;
  }
  // Per-expert row interleave of two expert stacks of one encoding and width ([E·F][d] each): expert e's rows of a,
  // then its rows of b (the q and s arrays are row-major, so each expert's block of rows is one contiguous run of
  // each array); left empty unless both are present and alike.
  void stack_experts(QWeight& out, const QWeight& a, const QWeight& b) {
    if (!a.q || !b.q || a.type != b.type || a.cols != b.cols || a.rows != b.rows || a.rows % E != 0) return;
    out.type = a.type;
    out.rows = 2 * a.rows;
    out.cols = a.cols;
    qweight_sizes(out.type, out.rows, out.cols, &out.q_bytes, &out.s_bytes);
    HOS_HIP_CHECK(hipMalloc(&out.q, out.q_bytes));
    HOS_HIP_CHECK(hipMalloc((void**)&out.s, out.s_bytes > 0 ? out.s_bytes : 256));
    const size_t qe = a.q_bytes / E, se = a.s_bytes / E;  // one expert's bytes of each array
    for (int e = 0; e < E; e++)
      for (int h = 0; h < 2; h++) {
        const QWeight& src = h ? b : a;
        HOS_HIP_CHECK(hipMemcpyAsync((uint8_t*)out.q + (2 * e + h) * qe, (const uint8_t*)src.q + e * qe, qe,
                                     hipMemcpyDeviceToDevice, st));
        if (se > 0)
          HOS_HIP_CHECK(hipMemcpyAsync((uint8_t*)out.s + (2 * e + h) * se, (const uint8_t*)src.s + e * se, se,
                                       hipMemcpyDeviceToDevice, st));
      }
  }
  // Row-wise concatenation of repacked weights (their q and s arrays are row-major, so the stack is the
  // concatenation of each array); left empty unless every part is present with one encoding and width.
  void stack(QWeight& out, std::initializer_list<const QWeight*> parts) {
    const QWeight* p0 = *parts.begin();
    long long rows = 0;
    for (const QWeight* p : parts) {
      if (!p->q || p->type != p0->type || p->cols != p0->cols) return;
      rows += p->rows;
    }
    out.type = p0->type;
    out.rows = rows;
    out.cols = p0->cols;
    qweight_sizes(out.type, out.rows, out.cols, &out.q_bytes, &out.s_bytes);
    HOS_HIP_CHECK(hipMalloc(&out.q, out.q_bytes));
    HOS_HIP_CHECK(hipMalloc((void**)&out.s, out.s_bytes > 0 ? out.s_bytes : 256));
    size_t qo = 0, so = 0;
    for (const QWeight* p : parts) {
      HOS_HIP_CHECK(hipMemcpyAsync((uint8_t*)out.q + qo, p->q, p->q_bytes, hipMemcpyDeviceToDevice, st));
      HOS_HIP_CHECK(hipMemcpyAsync((uint8_t*)out.s + so, p->s, p->s_bytes, hipMemcpyDeviceToDevice, st));
      qo += p->q_bytes;
      so += p->s_bytes;
    }
  }

  // From dy, the gradient of the group's fused projection output (row stride ldy, target t at column
  // ycol(t)): du_t = s·dy_t·B_tᵀ for every adapted t (one launch). dB_t = s·u_tᵀ·dy_t is queued and launched with
  // the group's dA by lora_grad_a: dy, u, x and du are all unchanged in between.
  // dyh set: the du product reads the output gradient from that fp16 operand; the queued dB reads dy (f32) unless
  // it is null
  void lora_grad_b(int l, int g, const float* dy, long long ldy, long long kspan, int M, HIn dyh = HIn{}) {
    const int n = gcount(g);
    if (n == 0) return;
    ColsSeg cs;
    RowsSeg rs;
    rs.nt = n;
    rs.r = r;
    for (int t = group_first(g); t <= group_last(g); t++) {
      if (!has(t)) continue;
      const int i = cs.nseg++;
      cs.gbeg[i] = ycol(t);
      cs.len[i] = out_dim(t);
      cs.soff[i] = ucol(t);
      cs.ocol[i] = bcol(t);
      rs.kbeg[i] = ycol(t);
      rs.kend[i] = ycol(t) + out_dim(t);
      rs.boff[i] = bcol(t);
    }
    const int w = bw(g);
    lora_rows("lora_du", M, kspan, lscale, dy, ldy, P + offBg[l * 4 + g], w, rs, du_of(l) + ucol(first_adapted(g)),
              NT * r, dyh, dyh.hi ? fac16(l, g, false) : B16{});
    pend_db = ColsJob{r, lscale, act[l].u, NT * r, dy, ldy, cs, G + offBg[l * 4 + g], w, 1, dy ? HIn{} : dyh};
    pend_group = g;
  }
  // Epilogue term dx_in += du_t·A_tᵀ of the base dX GEMM: L(j, col) = At[(slot·r + j)·in + col]
  GemmEpi down_epi(int l, int t) {
    GemmEpi e{};
    if (!has(t)) return e;
    e.U = du_of(l) + ucol(t);
    e.ldu = NT * r;
    e.L = P + offA[l * NT + t];
    e.slj = in_dim(t);
    e.sln = 1;
    e.rank = r;
    e.scale = 1.0f;
    return e;
  }
  // [dA_1 … dA_G]ᵀ = ([du_1 … du_G])ᵀ·x, written straight into the stacked At layout, in one launch with the
  // group's queued dB
  // xh set: the input is read from that fp16 operand (x is not read)
  void lora_grad_a(int l, int g, const float* x, long long ldx, int M, HIn xh = HIn{}) {
    const int n = gcount(g);
    if (n == 0) return;
    HOS_REQUIRE(pend_group == g, HOS_E_INVALID, "peft: dA without the group's dB queued");
    pend_group = -1;
    const int first = first_adapted(g), in = in_dim(first);
    ColsSeg cs;
    cs.nseg = 1;
    cs.len[0] = in;
    const ColsJob da{n * r, 1.0f, du_of(l) + ucol(first), NT * r, x, ldx, cs, G + offAg[l * 4 + g], in, 1, xh};
    if (gbatch) {  // both products wait for the end of the backward (their inputs are kept per layer)
      gjobs.push_back(pend_db);
      gjobs.push_back(da);
      return;
    }
    double fl = 2.0 * M * n * r * in, by = 4.0 * (M * (double)in + (double)M * n * r + (double)n * r * in);
    for (int t = 0; t < pend_db.sg.nseg; t++) {
      fl += 2.0 * M * r * pend_db.sg.len[t];
      by += 4.0 * ((double)M * pend_db.sg.len[t] + (double)M * r + (double)r * pend_db.sg.len[t]);
    }
    Scope s(this, "lora_dab", fl, by);
    // (the cols launch takes a job on the fp16 operand first)
    if (xh.hi)
      launch_lora_cols2(M, da, &pend_db, ws, ws_bytes, st, &cbatch);
    else
      launch_lora_cols2(M, pend_db, &da, ws, ws_bytes, st, &cbatch);
  }
  void flush_dab() {
    Scope s(this, "lora_dab", 0, 0);
    launch_lora_cols_flush(cbatch, st);
  }
  // The whole backward's queued dA / dB products (gbatch).
  void run_gjobs(int M) {
    if (gjobs.empty()) return;
    double fl = 0.0, by = 0.0;
    for (const ColsJob& j : gjobs)
      for (int t = 0; t < j.sg.nseg; t++) {
        fl += 2.0 * M * j.ns * j.sg.len[t];
        by += 4.0 * ((double)M * j.sg.len[t] + (double)M * j.ns + (double)j.ns * j.sg.len[t]);
      }
    Scope s(this, "lora_dab", fl, by);
    launch_lora_cols_table(M, gjobs.data(), (int)gjobs.size(), gtab, st);
    gjobs.clear();
  }
  void check_ready() {
    check_tensors();
    build_stacks();
  }
  void check_tensors() {
    HOS_REQUIRE(tok.q != nullptr, HOS_E_MISSING_TENSOR, "missing tensor 'token_embd.weight'");
    HOS_REQUIRE(out_norm != nullptr, HOS_E_MISSING_TENSOR, "missing tensor 'output_norm.weight'");
    for (int l = 0; l < L; l++) {
      const char* names[NT] = {"attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down"};
      for (int t = 0; t < (E ? TG : NT); t++)
        HOS_REQUIRE(lw[l].w[t].q != nullptr, HOS_E_MISSING_TENSOR,
                    "missing tensor 'blk." + std::to_string(l) + "." + names[t] + ".weight'");
      if (E)
        HOS_REQUIRE(lw[l].router && lw[l].xg.q && lw[l].xu.q && lw[l].xd.q, HOS_E_MISSING_TENSOR,
                    "missing mixture-of-experts tensors of blk." + std::to_string(l));
      if (c.qk_norm)
        HOS_REQUIRE(lw[l].q_norm && lw[l].k_norm, HOS_E_MISSING_TENSOR,
                    "missing QK-norm weights of blk." + std::to_string(l));
      HOS_REQUIRE(lw[l].attn_norm && lw[l].ffn_norm, HOS_E_MISSING_TENSOR,
                  "missing norm weights of blk." + std::to_string(l));
      if (c.attn_bias)
        HOS_REQUIRE(lw[l].bias[0] && lw[l].bias[1] && lw[l].bias[2], HOS_E_MISSING_TENSOR,
                    "missing attention biases of blk." + std::to_string(l));
    }
  }

  // ---------------- mixture of experts (OLMoE) ----------------
  void grouped(bool dxdir, const QWeight& w, H16 a, long long lda, const int* tiles, float* out, long long ldo,
               int accumulate, int M, int np) {
    const double er = (double)w.rows / E;  // W rows of one expert
    Scope s(this, dxdir ? "qgemm_dx" : "qgemm_fwd", 2.0 * M * K * er * w.cols,
            2.0 * M * K * (dxdir ? er : w.cols) + wbytes(w) + 4.0 * M * K * (dxdir ? w.cols : er));
    GemmEpi e{};
    e.out = out;
    e.ldo = ldo;
    e.accumulate = accumulate;
    launch_qgemm_grouped(dxdir, w, GroupSched{tiles, max_tiles, E}, a, lda, e, np, st);
  }
  // x_next = x2 + Σ_top-K p_e·SwiGLU_e(xn2) (src/forward.rs:542-572); xn2 (f32) and its fp16 operand in hs
  // come from the FFN RMSNorm.
  void moe_forward(int l, int M, float* xnext) {
    LayerAct& a = act[l];
    LayerW& w = lw[l];
    const long long P = (long long)M * K;
    {
      Scope s(this, "moe_route", 2.0 * M * d * E, 4.0 * ((double)M * d + (double)E * d + 4.0 * M * E) + 4.0 * P * d);
      launch_gemm_f32(M, E, d, 1.0f, a.xn2, d, 1, w.router, 1, d, 0.0f, mlogits, E, ws, ws_bytes, st);
      launch_moe_route(mlogits, M, E, K, a.pfull, a.sel_e, a.sel_p, a.slot, a.counts, st);
      launch_moe_plan(a.counts, E, a.offsets, a.tiles, max_tiles, st);
      launch_moe_gather(hs, d, a.sel_e, a.slot, a.offsets, M, K, d, a.pos, hx, d, st);
    }
    if (w.xgu.q) {  // gate|up of every expert in one launch
      grouped(false, w.xgu, hx, d, a.tiles, a.gug, 2LL * F, 0, M, pf);
    } else {
      grouped(false, w.xg, hx, d, a.tiles, a.gug, 2LL * F, 0, M, pf);
      grouped(false, w.xu, hx, d, a.tiles, a.gug + F, 2LL * F, 0, M, pf);
    }
    {
      Scope s(this, "swiglu", 0, 8.0 * P * F + 2.0 * P * F);
      launch_swiglu_fwd(a.gug, (int)P, F, nullptr, hx, st);
    }
    grouped(false, w.xd, hx, F, a.tiles, a.yg, d, 0, M, pf);
    {
      Scope s(this, "moe_combine", 0, 4.0 * (2.0 * M * d + P * d));
      launch_moe_combine(a.yg, a.pos, a.sel_p, a.x2, M, K, d, xnext, st);
    }
  }
  // dx: gradient at x_next on entry; leaves dxn = gradient at xn2 (experts + router)
  void moe_backward(int l, int M) {
    LayerAct& a = act[l];
    LayerW& w = lw[l];
    const long long P = (long long)M * K;
    if (moe_combine_bwd_h16_ok(d)) {
      Scope s(this, "moe_combine", 0, 4.0 * (M * d + P * d) + 4.0 * P * d);
      launch_moe_combine_bwd_h16(dx, a.yg, a.pos, a.sel_p, M, K, d, hx, mdp, st);
    } else {
      {
        Scope s(this, "moe_combine", 0, 4.0 * (M * d + 2.0 * P * d));
        launch_moe_combine_bwd(dx, a.yg, a.pos, a.sel_p, M, K, d, mdY, mdp, st);
      }
      Scope s(this, "convert", 0, 6.0 * P * d);
      launch_to_h16(mdY, d, P, d, hx, st);
    }
    grouped(true, w.xd, hx, d, a.tiles, mdH, F, 0, M, pd);
    {
      Scope s(this, "swiglu", 0, 4.0 * P * F * 3 + 4.0 * P * F);
      launch_swiglu_bwd(a.gug, mdH, (int)P, F, nullptr, hx, st);
    }
    if (w.xgu.q) {  // d(gate|up) against the interleaved stack: one contraction over 2F
      grouped(true, w.xgu, hx, 2LL * F, a.tiles, mdX, d, 0, M, pd);
    } else {
      grouped(true, w.xg, hx, 2LL * F, a.tiles, mdX, d, 0, M, pd);
      grouped(true, w.xu, h16_offset(hx, F), 2LL * F, a.tiles, mdX, d, 1, M, pd);
    }
    {
      Scope s(this, "moe_route", 2.0 * M * d * E, 4.0 * (P * d + 2.0 * M * d + (double)E * d + 3.0 * M * E));
      launch_moe_router_bwd(a.pfull, mdp, a.sel_e, M, E, K, mdl, st);
      launch_moe_gather_sum(mdX, a.pos, M, K, d, dxn, st);
      launch_gemm_f32(M, d, E, 1.0f, mdl, E, 1, w.router, d, 1, 1.0f, dxn, d, ws, ws_bytes, st);
    }
  }

  // ---------------- forward ----------------
  void forward(int B, int T, bool need_logits_only) {
    const int M = B * T;
    {
      Scope s(this, "embed", 0, 4.0 * M * d + (double)M * d);
      launch_embed(tok, ids, act[0].x, M, d, st);
    }
    split_factors();
    if (rga) {
      Scope s(this, "rga", 0, 4.0 * (16.0 * Kg + Kg));
      launch_rga_bias(P + offGen, P + offWg, Kg, rgb, st);
    }
    for (int l = 0; l < L; l++) {
      LayerAct& a = act[l];
      LayerW& w = lw[l];
      float* xnext = (l + 1 < L) ? act[l + 1].x : xfinal;
      const bool lqkv = has(TQ) || has(TK) || has(TV);
      {
        Scope s(this, "rmsnorm", 0, 4.0 * M * d * (lqkv ? 2 : 1) + 2.0 * M * d);
        launch_rmsnorm_fwd(a.x, w.attn_norm, c.rms_eps, M, d, lqkv ? a.xn1 : nullptr, hs, a.inv1, st, xsrc);
        xsrc = SplitSrc{};
      }
      lora_down(l, 0, a.xn1, d, M, hs_in());
      if (w.qkv.q && group_uniform(0) && (!c.attn_bias || w.bias_qkv)) {
        qfwd(w.qkv, hs, d, M, a.qkv, W3, c.attn_bias ? w.bias_qkv : nullptr, nullptr, 0, stacked_up_epi(l, 0),
             tpf[TQ]);
      } else {
        qfwd(w.w[TQ], hs, d, M, a.qkv, W3, w.bias[0], nullptr, 0, up_epi(l, TQ), tpf[TQ]);
        qfwd(w.w[TK], hs, d, M, a.qkv + qd, W3, w.bias[1], nullptr, 0, up_epi(l, TK), tpf[TK]);
        qfwd(w.w[TV], hs, d, M, a.qkv + qd + kvd, W3, w.bias[2], nullptr, 0, up_epi(l, TV), tpf[TV]);
      }
      if (c.qk_norm) {
        Scope s(this, "rmsnorm", 0, 4.0 * M * (qd + kvd) * 3);
        launch_qknorm_fwd(a.qkv, W3, 0, qd, w.q_norm, c.rms_eps, M, a.qk_pre, a.qk_inv, st);
        launch_qknorm_fwd(a.qkv, W3, qd, kvd, w.k_norm, c.rms_eps, M, a.qk_pre + (size_t)M * qd, a.qk_inv + M, st);
      }
      {
        // RoPE on q and k is applied as they are split into the attention's planes (a.qkv stays unrotated: the
        // backward reads only the planes)
        Scope s(this, "attn_fwd", 2.0 * B * c.n_heads * (double)T * (T + 1) / 2 * c.head_dim * 2,
                4.0 * M * (W3 + qd) + 4.0 * B * c.n_heads * T);
        launch_attn_fwd(a.qkv, W3, qd, qd + kvd, B, T, c.n_heads, c.n_kv_heads, c.head_dim, a.o, qd, a.lse,
                        attn_planes[l], st, rope_tab, c.rope_neox);
      }
      to16(a.o, qd, M, qd);
      lora_down(l, 1, a.o, qd, M, hs_in());
      qfwd(w.w[TO], hs, qd, M, a.x2, d, nullptr, a.x, 0, up_epi(l, TO), tpf[TO]);
      const bool lgu = has(TG) || has(TU) || E;
      {
        Scope s(this, "rmsnorm", 0, 4.0 * M * d * (lgu ? 2 : 1) + 2.0 * M * d);
        launch_rmsnorm_fwd(a.x2, w.ffn_norm, c.rms_eps, M, d, lgu ? a.xn2 : nullptr, hs, a.inv2, st);
      }
      if (E) {
        moe_forward(l, M, xnext);
        continue;
      }
      lora_down(l, 2, a.xn2, d, M, hs_in());
      if (w.gu.q && group_uniform(2)) {
        qfwd(w.gu, hs, d, M, a.gu, 2LL * F, nullptr, nullptr, 0, stacked_up_epi(l, 2), tpf[TG]);
      } else {
        qfwd(w.w[TG], hs, d, M, a.gu, 2LL * F, nullptr, nullptr, 0, up_epi(l, TG), tpf[TG]);
        qfwd(w.w[TU], hs, d, M, a.gu + F, 2LL * F, nullptr, nullptr, 0, up_epi(l, TU), tpf[TU]);
      }
      const H16 hdn = a.hd.data ? a.hd : hs;  // the down projection's operand
      {
        Scope s(this, "swiglu", 0, 8.0 * M * F + 2.0 * M * F + (a.h ? 4.0 * M * F : 0));
        launch_swiglu_fwd(a.gu, M, F, a.h, hdn, st);
      }
      lora_down(l, 3, a.h, F, M, hdn.lo ? HIn{hdn.data, hdn.lo, hdn.rinv} : HIn{});
      if (rga)
        qfwd(w.w[TD], hdn, F, M, a.xr, d, nullptr, a.x2, 0, up_epi(l, TD), tpf[TD]);
      else  // x_{l+1} is formed (and stored) by the next RMSNorm from the partials when the launch splits
        xsrc = deferred(false, w.w[TD], hdn, F, M, xnext, d, a.x2, up_epi(l, TD), tpf[TD]);
      if (rga) rga_forward(l, M, xnext);
    }
    {
      Scope s(this, "rmsnorm", 0, 4.0 * M * d + 2.0 * M * d);
      launch_rmsnorm_fwd(xfinal, out_norm, c.rms_eps, M, d, nullptr, hs, invf, st, xsrc);
      xsrc = SplitSrc{};
    }
    GemmEpi he{};
    if (!need_logits_only) {  // the cross-entropy's softmax statistics come out of the head GEMM's epilogue
      he.rstat = lstat;
      he.rstat_ld = (V + 63) / 64;
    }
    qfwd(out_set ? out : tok, hs, d, M, logits, V, nullptr, nullptr, 0, he, phf);
  }

  // ---------------- loss + backward ----------------
  void loss_backward(int B, int T) {
    const int M = B * T;
    {
      Scope s(this, "ce", 0, 4.0 * M * V + 2.0 * M * V);
      float gscale = (1.0f / (float)B) / (float)T;  // scale(1/B) then CE's g/n (src/tensor.rs:2736-2741)
      launch_ce(logits, M, V, tgts, gscale, row_loss, dl, st, nullptr, lstat);
      launch_loss_reduce(row_loss, B, T, loss, st);
    }
    if (rga && rlambda > 0.0f) {
      Scope s(this, "rga", 0, 4.0 * L * M);
      launch_rga_loss(rgsum, Mmax, L, B, T, Kg, rlambda, rgm, loss, st);
    }
    const QWeight& head = out_set ? out : tok;
    const SplitSrc hsrc = deferred(true, head, dl, V, M, dxn, d, nullptr, GemmEpi{}, phd);
    // The RMSNorm backwards also write the fp16 operand of their dx for the GEMMs that follow; not where the
    // RGA backward changes dx in between or a mixture-of-experts FFN takes no such operand.
    const bool fuse16 = !rga && !E;
    // gbatch: dx walks the per-layer residual gradients (each RMSNorm backward writes a new one); restored below
    float* const dx_base = dx;
    if (gbatch) dx = dxs_l[L - 1];
    {
      Scope s(this, "rmsnorm", 0, 4.0 * M * d * 3 + 4.0 * M * d + (fuse16 ? 6.0 * M * d : 0));
      launch_fill(dx, (long long)M * d, 0.0f, st);
      launch_rmsnorm_bwd(dxn, xfinal, invf, out_norm, M, d, dx, st, fuse16 ? hs : H16{nullptr, nullptr, nullptr},
                         hsrc);
    }
    for (int l = L - 1; l >= 0; l--) {
      LayerAct& a = act[l];
      LayerW& w = lw[l];
      SplitSrc gsrc{};  // the stacked gate|up dX's partials, reduced by the FFN RMSNorm backward
      // gbatch: this layer's own output-gradient buffers (kept for the dA / dB products after the backward)
      float* const dq = gbatch ? dqkv_l[l] : dqkv;
      if (rga) rga_backward(l, B, T);  // dx: gradient at x_{l+1} -> at the FFN output
      // ---- FFN branch: x_{l+1} = x2 + h·W_down (+ LoRA), or the mixture of experts ----
      if (E) {
        moe_backward(l, M);
      } else {
      if (!fuse16) to16(dx, d, M, d);
      lora_grad_b(l, 3, dx, d, d, M, hs_in());
      qdx(w.w[TD], hs, d, M, dh, F, 0, down_epi(l, TD), tpd[TD]);
      lora_grad_a(l, 3, a.h, F, M, a.hd.data ? HIn{a.hd.data, a.hd.lo, a.hd.rinv} : HIn{});
      // The gate|up LoRA gradients read d(gate|up) from the fp16 operand the SwiGLU backward writes for the dX
      // GEMM when it carries the residual plane (the dB pass in 16-byte runs of each plane); an f32 copy only for
      // single-plane precision modes.
      const bool gu_lora = has(TG) || has(TU), gu_f32 = gu_lora && !hs.lo;
      // d(gate|up) as the fp16 operand: the shared scratch, or (gbatch) this layer's own copy
      const H16 hg = (gbatch && gu_lora) ? dgu16_l[l] : hs;
      {
        Scope s(this, "swiglu", 0, 4.0 * M * F * 3 + 4.0 * M * F + (gu_f32 ? 8.0 * M * F : 0));
        launch_swiglu_bwd(a.gu, dh, M, F, gu_f32 ? dgu : nullptr, hg, st);
      }
      if (gu_lora) lora_grad_b(l, 2, gu_f32 ? dgu : nullptr, 2LL * F, 2LL * F, M, HIn{hg.data, hg.lo, hg.rinv});
      if (w.gu.q && group_uniform(2) && gcount(2) * r <= 32) {
        gsrc = deferred(true, w.gu, hg, 2LL * F, M, dxn, d, nullptr, stacked_down_epi(l, 2), tpd[TG]);
      } else {
        H16 hu = h16_offset(hg, F);
        qdx(w.w[TG], hg, 2LL * F, M, dxn, d, 0, down_epi(l, TG), tpd[TG]);
        qdx(w.w[TU], hu, 2LL * F, M, dxn, d, 1, down_epi(l, TU), tpd[TU]);
      }
      lora_grad_a(l, 2, a.xn2, d, M);
      }
      {
        Scope s(this, "rmsnorm", 0, 4.0 * M * d * 4 + 6.0 * M * d);
        // gbatch: gradient at x2 into this layer's own buffer (the one at x_{l+1} stays for the down dB)
        float* const dx_in = dx;
        if (gbatch) dx = dx2s_l[l];
        launch_rmsnorm_bwd(dxn, a.x2, a.inv2, w.ffn_norm, M, d, dx, st, hs, gsrc, dx_in);
      }
      // ---- attention branch: x2 = x + attn(x)·W_o (+ LoRA) ----
      lora_grad_b(l, 1, dx, d, d, M, hs_in());
      qdx(w.w[TO], hs, d, M, dout, qd, 0, down_epi(l, TO), tpd[TO]);
      lora_grad_a(l, 1, a.o, qd, M);
      const bool rows_pass = !c.qk_norm && W3 <= kAttnRowsMax;
      {
        Scope s(this, "attn_bwd", 2.0 * B * c.n_heads * (double)T * (T + 1) / 2 * c.head_dim * 5,
                4.0 * M * (W3 * 2 + qd * 2) + 8.0 * B * c.n_heads * T);
        // without QK-norm the GQA group sum of dK/dV is left to the row pass below
        launch_attn_bwd(a.qkv, W3, qd, qd + kvd, a.o, dout, qd, a.lse, dvec, B, T, c.n_heads, c.n_kv_heads,
                        c.head_dim, dq, W3, attn_part, attn_planes[l], st, true, rows_pass);
      }
      {
        Scope s(this, "rope", 0, 8.0 * M * (qd + kvd));
        // the k heads follow the q heads in the row (qd = n_heads·head_dim): one launch rotates both; without
        // QK-norm in between the same row pass also sums dK/dV over each GQA group and writes the fp16 operand of
        // the q|k|v dX GEMM
        if (c.qk_norm)
          launch_rope(dq, W3, 0, c.n_heads + c.n_kv_heads, c.head_dim, T, rope_tab, c.rope_neox, true, M, st);
        else if (!rows_pass)
          launch_rope_h16(dq, W3, c.n_heads + c.n_kv_heads, c.head_dim, T, rope_tab, c.rope_neox, true, M, W3, hs,
                          st);
        else
          launch_attn_bwd_rows(dq, W3, c.head_dim, c.n_heads, c.n_kv_heads, qd + kvd, attn_part, T, rope_tab,
                               c.rope_neox, M, W3, hs, st);
      }
      if (c.qk_norm) {
        Scope s(this, "rmsnorm", 0, 4.0 * M * (qd + kvd) * 4);
        launch_qknorm_bwd(dq, W3, 0, qd, w.q_norm, a.qk_pre, a.qk_inv, M, st);
        launch_qknorm_bwd(dq, W3, qd, kvd, w.k_norm, a.qk_pre + (size_t)M * qd, a.qk_inv + M, M, st);
      }
      if (c.qk_norm) to16(dq, W3, M, W3);
      lora_grad_b(l, 0, dq, W3, W3, M, hs_in());
      if (w.qkv.q && group_uniform(0) && gcount(0) * r <= 128) {
        // one dX GEMM over the stacked q|k|v contraction, the three LoRA terms as one rank-3r update
        qdx(w.qkv, hs, W3, M, dxn, d, 0, stacked_down_epi(l, 0), tpd[TQ]);
      } else {
        H16 hk = h16_offset(hs, qd), hv = h16_offset(hs, qd + kvd);
        qdx(w.w[TQ], hs, W3, M, dxn, d, 0, down_epi(l, TQ), tpd[TQ]);
        qdx(w.w[TK], hk, W3, M, dxn, d, 1, down_epi(l, TK), tpd[TK]);
        qdx(w.w[TV], hv, W3, M, dxn, d, 1, down_epi(l, TV), tpd[TV]);
      }
      lora_grad_a(l, 0, a.xn1, d, M);
      if (!gbatch) flush_dab();  // the layer's dA/dB reductions
      {
        const bool emit = fuse16 && l > 0;
        Scope s(this, "rmsnorm", 0, 4.0 * M * d * 4 + (emit ? 6.0 * M * d : 0));
        float* const dx_in = dx;
        if (gbatch) dx = l > 0 ? dxs_l[l - 1] : dx_base;
        launch_rmsnorm_bwd(dxn, a.x, a.inv1, w.attn_norm, M, d, dx, st, emit ? hs : H16{nullptr, nullptr, nullptr},
                           SplitSrc{}, dx_in);
      }
    }
    dx = dx_base;
    if (gbatch) run_gjobs(M);  // every layer's LoRA dA / dB
    if (rga) {
      Scope s(this, "rga", 0, 4.0 * (L * Kg + 32.0 * Kg));
      launch_rga_genome_grad(P + offGen, P + offWg, rdgb, L, Kg, G + offWg, G + offGen, st);
    }
  }

  // ---------------- RGA adapter (src/peft.rs:565-584) ----------------
  // x_next = xr + (H ⊙ gate)·Up with [gate logits | bottleneck] = xr·RTᵀ
  void rga_forward(int l, int M, float* xnext) {
    LayerAct& a = act[l];
    RowsSeg rs;
    rs.nt = 1;
    rs.r = Rp;
    rs.kend[0] = d;
    lora_rows("rga", M, d, 1.0f, a.xr, d, P + offRT[l], d, rs, rz, Rp);
    {
      Scope s(this, "rga", 0, 4.0 * M * (3.0 * Rp + Kbp + 1));
      launch_rga_act_fwd(rz, Rp, M, Kg, bn, rgb, a.ra, a.hg, Kbp, rgsum + (long long)l * Mmax, st);
    }
    {
      Scope s(this, "rga", 2.0 * M * d * Kbp, 4.0 * ((double)M * d * 3 + (double)M * Kbp + (double)Kbp * d));
      HOS_HIP_CHECK(hipMemcpyAsync(xnext, a.xr, (size_t)M * d * 4, hipMemcpyDeviceToDevice, st));
      launch_gemm_f32(M, d, Kbp, 1.0f, a.hg, Kbp, 1, P + offUp[l], d, 1, 1.0f, xnext, d, ws, ws_bytes, st);
    }
  }
  // dx: gradient at x_next on entry, at xr on exit (identity + the adapter's input gradient); fills the
  // layer's RT and Up gradients and its gate-bias gradient.
  void rga_backward(int l, int B, int T) {
    const int M = B * T;
    LayerAct& a = act[l];
    ColsSeg cs;
    cs.nseg = 1;
    cs.len[0] = d;
    // dUp = (H ⊙ gate)ᵀ·dx, launched below with dRT (dx is unchanged until the dZ·RT update)
    const ColsJob dup{Kbp, 1.0f, a.hg, Kbp, dx, d, cs, G + offUp[l], d, 1};
    RowsSeg rs;
    rs.nt = 1;
    rs.r = Kbp;
    rs.kend[0] = d;
    lora_rows("rga", M, d, 1.0f, dx, d, P + offUp[l], d, rs, rdg, Kbp);  // dG = dx·Upᵀ
    {
      // the sparsity term: (1/B)·(λ/L)·mean over a sequence's T·K gates
      const float pc = rlambda > 0.0f ? rlambda / ((float)B * (float)L * (float)T * (float)Kg) : 0.0f;
      Scope s(this, "rga", 0, 4.0 * M * (3.0 * Rp + Kbp) + 4.0 * M * Kg);
      launch_rga_act_bwd(a.ra, Rp, rdg, Kbp, M, Kg, bn, pc, rz, st);
      launch_rga_colsum(rz, Rp, M, Kg, rdgb + (long long)l * Kg, st);
    }
    {
      const ColsJob drt{Rp, 1.0f, rz, Rp, a.xr, d, cs, G + offRT[l], d, 1};  // dRT = dZᵀ·xr
      Scope s(this, "rga", 2.0 * M * d * (Kbp + Rp), 4.0 * ((double)M * d * 2 + (double)M * (Kbp + Rp) + (double)(Kbp + Rp) * d));
      launch_lora_cols2(M, dup, &drt, ws, ws_bytes, st);
    }
    {
      Scope s(this, "rga", 2.0 * M * d * Rp, 4.0 * ((double)M * d * 2 + (double)M * Rp + (double)Rp * d));
      launch_gemm_f32(M, d, Rp, 1.0f, rz, Rp, 1, P + offRT[l], d, 1, 1.0f, dx, d, ws, ws_bytes, st);  // dx += dZ·RT
    }
  }

  void set_hyper(float lr, float wd) {
    hyp_host.lr = lr;
    hyp_host.wd = wd;
    HOS_HIP_CHECK(hipMemcpyAsync(hyp, &hyp_host, 2 * sizeof(float), hipMemcpyHostToDevice, st));
  }
  // AdamW over the arena with lr/wd/t from device memory (set_hyper first); bias corrections by f32 powi
  // of the device step count, exactly as the host's powi would give.
  void adamw_enqueue() {
    adam_t += 1;
    Scope s(this, "adamw", 0, 4.0 * nparams * 7);
    launch_adam_tick(hyp, st);
    // every LoRA factor is 2-D, so decay applies to all (src/main.rs:2571)
    launch_adamw_dev(P, G, M1, V1, nparams, 0.9f, 0.95f, 1e-8f, hyp, true, st);
  }
  void adamw(float lr, float wd) {
    set_hyper(lr, wd);
    adamw_enqueue();
  }
  // One optimizer step on device-resident ids/targets: zero-grad is implicit (every gradient buffer is
  // overwritten), forward, backward, AdamW, loss copy. Replayed from a captured graph after its first use.
  void step_body(const int32_t* ids_dev, const int32_t* targets_dev, int B, int T, float* loss_dev) {
    HOS_HIP_CHECK(hipMemcpyAsync(ids, ids_dev, (size_t)B * T * 4, hipMemcpyDeviceToDevice, st));
    HOS_HIP_CHECK(hipMemcpyAsync(tgts, targets_dev, (size_t)B * T * 4, hipMemcpyDeviceToDevice, st));
    forward(B, T, false);
    loss_backward(B, T);
    adamw_enqueue();
    if (loss_dev) HOS_HIP_CHECK(hipMemcpyAsync(loss_dev, loss, 4, hipMemcpyDeviceToDevice, st));
  }
  void step(const int32_t* ids_dev, const int32_t* targets_dev, int B, int T, float lr, float wd, float* loss_dev) {
    set_hyper(lr, wd);
    if (!use_graph || prof) {
      step_body(ids_dev, targets_dev, B, T, loss_dev);
      return;
    }
    const std::vector<uintptr_t> key = {(uintptr_t)B, (uintptr_t)T, (uintptr_t)ids_dev, (uintptr_t)targets_dev,
                                        (uintptr_t)loss_dev};
    auto it = graphs.find(key);
    if (it == graphs.end()) {
      hipGraph_t g = nullptr;
      HOS_HIP_CHECK(hipStreamBeginCapture(st, hipStreamCaptureModeRelaxed));
      try {
        step_body(ids_dev, targets_dev, B, T, loss_dev);
      } catch (...) {
        (void)hipStreamEndCapture(st, &g);
        if (g) (void)hipGraphDestroy(g);
        throw;
      }
      HOS_HIP_CHECK(hipStreamEndCapture(st, &g));
      adam_t -= 1;  // the capture enqueued nothing; the launch below runs the step
      hipGraphExec_t ex = nullptr;
      hipError_t e = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
      (void)hipGraphDestroy(g);
      HOS_HIP_CHECK(e);
      it = graphs.emplace(key, ex).first;
    }
    adam_t += 1;
    HOS_HIP_CHECK(hipGraphLaunch(it->second, st));
  }

  void collect_prof() {
    if (recs.empty()) return;
    HOS_HIP_CHECK(hipStreamSynchronize(st));
    for (auto& rc : recs) {
      float ms = 0;
      (void)hipEventElapsedTime(&ms, rc.e0, rc.e1);
      ProfAcc& a = acc[rc.cls];
      a.launches++;
      a.ms += ms;
      a.flops += rc.flops;
      a.bytes += rc.bytes;
      (void)hipEventDestroy(rc.e0);
      (void)hipEventDestroy(rc.e1);
    }
    recs.clear();
  }

  void init(hos_ctx* cx, const hos_peft_cfg* cfg) {
    ctx = cx;
    st = hos_internal_stream(cx);
    c = *cfg;
    HOS_REQUIRE(c.n_layers > 0 && c.dim > 0 && c.n_heads > 0 && c.n_kv_heads > 0 && c.ffn_dim > 0 && c.vocab > 0,
                HOS_E_INVALID, "peft: bad model dimensions");
    HOS_REQUIRE(c.n_heads % c.n_kv_heads == 0, HOS_E_INVALID, "peft: n_heads must be a multiple of n_kv_heads");
    HOS_REQUIRE(c.head_dim == 64 || c.head_dim == 128, HOS_E_UNSUPPORTED_ARCH, "peft: head_dim must be 64 or 128");
    E = c.n_experts;
    K = c.n_experts_used;
    HOS_REQUIRE(E == 0 || (E <= 64 && K >= 1 && K <= E), HOS_E_INVALID,
                "peft: mixture of experts needs 1 <= n_experts_used <= n_experts <= 64");
    HOS_REQUIRE(E == 0 || !(c.lora_targets & (HOS_T_GATE | HOS_T_UP | HOS_T_DOWN)), HOS_E_INVALID,
                "peft: a mixture-of-experts FFN takes no LoRA on gate/up/down");
    HOS_REQUIRE(c.lora_rank > 0 && c.max_batch > 0 && c.max_seq > 0, HOS_E_INVALID, "peft: bad rank/batch/seq");
    rga = c.rga_genes > 0;
    if (rga) {
      HOS_REQUIRE(c.lora_targets == 0, HOS_E_INVALID, "peft: RGA adapters replace LoRA (lora_targets must be 0)");
      HOS_REQUIRE(E == 0, HOS_E_UNSUPPORTED_ARCH, "peft: RGA on a mixture-of-experts model is not supported");
      HOS_REQUIRE(c.rga_genes <= RGA_MAX_GENES && c.rga_bottleneck > 0, HOS_E_INVALID, "peft: bad RGA genes/bottleneck");
      Kg = c.rga_genes;
      bn = c.rga_bottleneck;
      Rp = (Kg + Kg * bn + 3) & ~3;
      Kbp = (Kg * bn + 3) & ~3;
      HOS_REQUIRE(Rp <= 96, HOS_E_INVALID, "peft: RGA genes·(1 + bottleneck) must be <= 96");
      rlambda = c.rga_lambda;
    }
    HOS_REQUIRE(c.dim % 32 == 0 && c.ffn_dim % 32 == 0, HOS_E_INVALID, "peft: dim and ffn_dim must be multiples of 32");
    L = c.n_layers;
    d = c.dim;
    qd = c.n_heads * c.head_dim;
    kvd = c.n_kv_heads * c.head_dim;
    W3 = qd + 2 * kvd;
    F = c.ffn_dim;
    V = c.vocab;
    r = c.lora_rank;
    lscale = c.lora_alpha / (float)r;  // src/peft.rs:195
    Mmax = c.max_batch * c.max_seq;
    passes = c.gemm_passes == 0 ? 3 : c.gemm_passes;
    HOS_REQUIRE(passes >= 1 && passes <= 5, HOS_E_INVALID, "peft: gemm_passes must be 0 (default) or 1 to 5");
    // Default precision policy (measured against the f32 path, worst LoRA-gradient rel L2 at the
    // SmolLM2-135M / Qwen2.5-0.5B configs): the per-layer GEMMs need both operands to ~22 bits — the forward
    // as mode 5 (activation split, weight as its exact integer codes; mode 3 where the layout has none), the dX
    // as mode 3; the head's forward is fine in one pass (+2e-5) and its dX needs only the weight split (mode 4).
    // An explicit gemm_passes applies to every GEMM.
    if (c.gemm_passes == 0) {
      pf = 5;
      pd = 3;
      phf = 1;
      phd = 4;
    } else {
      pf = pd = phf = phd = passes;
    }
    const size_t M = (size_t)Mmax;
    lw.resize(L);
    // LoRA arena
    offA.assign((size_t)L * NT, -1);
    offB.assign((size_t)L * NT, -1);
    offAg.assign((size_t)L * 4, -1);
    offBg.assign((size_t)L * 4, -1);
    HOS_REQUIRE(r <= 32, HOS_E_INVALID, "peft: LoRA rank must be <= 32");
    long long off = 0;
    auto pad = [](long long v) { return (v + 63) & ~63LL; };  // 256-byte aligned blocks
    for (int l = 0; l < L; l++)
      for (int g = 0; g < 4; g++) {
        const int n = gcount(g);
        if (n == 0) continue;
        const int in = in_dim(group_first(g));
        offAg[l * 4 + g] = off;
        off = pad(off + (long long)n * r * in);
        offBg[l * 4 + g] = off;
        off = pad(off + (long long)r * bw(g));
        for (int t = group_first(g); t <= group_last(g); t++)
          if (has(t)) {
            offA[l * NT + t] = offAg[l * 4 + g] + (long long)slot(t) * r * in;
            offB[l * NT + t] = offBg[l * 4 + g] + bcol(t);
          }
      }
    if (rga) {  // RGA arena, in PeftModel::params order: wg, per layer the bank, the genome
      offWg = off;
      off = pad(off + (long long)RGA_GLEN * Kg);
      offRT.assign(L, -1);
      offUp.assign(L, -1);
      for (int l = 0; l < L; l++) {
        offRT[l] = off;
        off = pad(off + (long long)Rp * d);
        offUp[l] = off;
        off = pad(off + (long long)Kbp * d);
      }
      offGen = off;
      off = pad(off + RGA_GLEN);
    }
    nparams = off;
    {
      std::vector<SplitRow> tab;
      scA.assign((size_t)L * 4, 0);
      scB.assign((size_t)L * 4, 0);
      nfac = 0;
      for (int l = 0; l < L; l++)
        for (int g = 0; g < 4; g++) {
          if (offAg[l * 4 + g] < 0) continue;
          const int n = gcount(g), in = in_dim(group_first(g)), w = bw(g);
          scA[l * 4 + g] = (int)tab.size();
          for (int i = 0; i < n * r; i++) tab.push_back(SplitRow{offAg[l * 4 + g] + (long long)i * in, in});
          scB[l * 4 + g] = (int)tab.size();
          for (int j = 0; j < r; j++) tab.push_back(SplitRow{offBg[l * 4 + g] + (long long)j * w, w});
          nfac += (long long)n * r * in + (long long)r * w;
        }
      n_split = (int)tab.size();
      if (n_split > 0) {
        split_tab = alloc<SplitRow>(tab.size());
        HOS_HIP_CHECK(hipMemcpy(split_tab, tab.data(), tab.size() * sizeof(SplitRow), hipMemcpyHostToDevice));
        P16h = alloc<_Float16>(nparams);
        P16l = alloc<_Float16>(nparams);
        psc = alloc<float>(tab.size());
      }
    }
    P = alloc<float>(nparams);
    G = alloc<float>(nparams);
    M1 = alloc<float>(nparams);
    V1 = alloc<float>(nparams);
    launch_fill(P, nparams, 0.0f, st);
    launch_fill(G, nparams, 0.0f, st);
    launch_fill(M1, nparams, 0.0f, st);
    launch_fill(V1, nparams, 0.0f, st);
    // activations
    act.resize(L);
    for (int l = 0; l < L; l++) {
      LayerAct& a = act[l];
      a.x = alloc<float>(M * d);
      a.xn1 = (has(TQ) || has(TK) || has(TV)) ? alloc<float>(M * d) : nullptr;
      a.inv1 = alloc<float>(M);
      a.qkv = alloc<float>(M * W3);
      a.o = alloc<float>(M * qd);
      a.lse = alloc<float>(M * c.n_heads);
      a.x2 = alloc<float>(M * d);
      a.xn2 = (has(TG) || has(TU) || E) ? alloc<float>(M * d) : nullptr;
      a.inv2 = alloc<float>(M);
      a.gu = E ? nullptr : alloc<float>(M * 2 * F);
      if (has(TD) && !E && (alo_mode(pf) || alo_mode(pd) || alo_mode(phf))) {
        a.h = nullptr;
        a.hd.data = alloc<half_t>(M * F);
        a.hd.lo = alloc<half_t>(M * F);
        a.hd.rinv = alloc<float>(M);
      } else {
        a.h = has(TD) ? alloc<float>(M * F) : nullptr;
      }
      a.u = alloc<float>(M * NT * r);
      if (rga) {
        a.xr = alloc<float>(M * d);
        a.ra = alloc<float>(M * Rp);
        a.hg = alloc<float>(M * Kbp);
      }
      if (c.qk_norm) {
        a.qk_pre = alloc<float>(M * (qd + kvd));
        a.qk_inv = alloc<float>(2 * M);
      }
      if (E) {
        const size_t P = M * K;
        max_tiles = (int)((P + GROUP_BM - 1) / GROUP_BM) + E;
        a.pfull = alloc<float>(M * E);
        a.sel_p = alloc<float>(P);
        a.sel_e = alloc<int>(P);
        a.slot = alloc<int>(P);
        a.pos = alloc<int>(P);
        a.counts = alloc<int>(E);
        a.offsets = alloc<int>(E + 1);
        a.tiles = alloc<int>(3 * (size_t)max_tiles);
        a.gug = alloc<float>(P * 2 * F);
        a.yg = alloc<float>(P * d);
      }
    }
    if (E) {
      const size_t P = M * K, xc = std::max<size_t>((size_t)d, 2 * (size_t)F);
      hx.data = alloc<half_t>(P * xc);
      hx.rinv = alloc<float>(P);
      hx.lo = (alo_mode(pf) || alo_mode(pd)) ? alloc<half_t>(P * xc) : nullptr;
      mlogits = alloc<float>(M * E);
      mdY = alloc<float>(P * d);
      mdH = alloc<float>(P * F);
      mdX = alloc<float>(P * d);
      mdp = alloc<float>(P);
      mdl = alloc<float>(M * E);
    }
    if (rga) {
      rz = alloc<float>(M * Rp);
      rdg = alloc<float>(M * Kbp);
      rgb = alloc<float>(Kg);
      rdgb = alloc<float>((size_t)L * Kg);
      rgsum = alloc<float>((size_t)L * M);
      rgm = alloc<float>((size_t)L * M);  // B <= B·T <= the row capacity
    }
    xfinal = alloc<float>(M * d);
    invf = alloc<float>(M);
    size_t hcols = std::max<size_t>({(size_t)d, (size_t)W3, (size_t)qd, 2 * (size_t)F});
    hs.data = alloc<half_t>(M * hcols);
    hs.rinv = alloc<float>(M);
    const bool alo = alo_mode(pf) || alo_mode(pd) || alo_mode(phf);
    hs.lo = alo ? alloc<half_t>(M * hcols) : nullptr;
    logits = alloc<float>(M * V);
    lstat = alloc<float2>(M * (size_t)((V + 63) / 64));
    dl.data = alloc<half_t>(M * V);
    dl.rinv = alloc<float>(M);
    dl.lo = alo_mode(phd) ? alloc<half_t>(M * V) : nullptr;
    row_loss = alloc<float>(M);
    loss = alloc<float>(1);
    dx = alloc<float>(M * d);
    dxn = alloc<float>(M * d);
    dqkv = alloc<float>(M * W3);
    dout = alloc<float>(M * qd);
    dh = E ? nullptr : alloc<float>(M * F);
    dgu = (has(TG) || has(TU)) ? alloc<float>(M * 2 * F) : nullptr;
    du = alloc<float>(M * NT * r);
    // whole-backward batching of the LoRA dA / dB products: dense LoRA models with the two-plane fp16 operand
    gbatch = !rga && !E && c.lora_targets != 0 && hs.lo != nullptr;
    if (const char* e = getenv("HOS_LORA_GBATCH")) gbatch = gbatch && atoi(e) != 0;
    if (gbatch) {
      gtab.cap = 8 * L;  // a dA and a dB per adapted group of each layer
      void* hp = nullptr;
      HOS_HIP_CHECK(hipHostMalloc(&hp, lora_cols_table_bytes(gtab.cap), hipHostMallocDefault));
      gtab.host = (ColsJobDev*)hp;
      gtab.dev = (ColsJobDev*)alloc<unsigned char>(lora_cols_table_bytes(gtab.cap));
      du_l.resize(L);
      dqkv_l.resize(L);
      dxs_l.resize(L);
      dx2s_l.resize(L);
      dgu16_l.resize(L);
      for (int l = 0; l < L; l++) {
        du_l[l] = alloc<float>(M * NT * r);
        dqkv_l[l] = alloc<float>(M * W3);
        dxs_l[l] = alloc<float>(M * d);
        dx2s_l[l] = alloc<float>(M * d);
        if (has(TG) || has(TU)) {
          dgu16_l[l].data = alloc<half_t>(M * 2 * F);
          dgu16_l[l].lo = alloc<half_t>(M * 2 * F);
          dgu16_l[l].rinv = alloc<float>(M);
        }
      }
    }
    dvec = alloc<float>(M * c.n_heads);
    if (c.n_heads != c.n_kv_heads) attn_part = alloc<float>(M * c.n_heads * 2 * c.head_dim);
    attn_planes.resize(L);
    for (int l = 0; l < L; l++)
      attn_planes[l] = alloc<float>(attn_scratch_bytes(c.max_batch, c.max_seq, c.n_heads, c.n_kv_heads, c.head_dim) / 4);
    ws_bytes = std::max<size_t>(64ull << 20, std::min<size_t>(M * std::max<size_t>(d, F) * 4 * 8, 1ull << 30));
    ws = alloc<float>(ws_bytes / 4);
    ws2 = alloc<float>(ws_bytes / 4);
    cbatch = ColsBatch{};
    cbatch.cap = (64ull << 20) / 4;
    cbatch.base = alloc<float>(cbatch.cap);
    hyp = alloc<AdamHyper>(1);
    launch_fill((float*)hyp, sizeof(AdamHyper) / 4, 0.0f, st);  // lr = wd = 0, t = 0 (all-zero bits)
    ids = alloc<int32_t>(M);
    tgts = alloc<int32_t>(M);
    // RoPE (sin, cos) table with the reference's f32 powf/sinf/cosf (src/tensor.rs:2769-2778)
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
    if (gtab.host) (void)hipHostFree(gtab.host);
    gtab.host = nullptr;
    for (auto& kv : graphs) (void)hipGraphExecDestroy(kv.second);
    graphs.clear();
    for (auto& rc : recs) {
      (void)hipEventDestroy(rc.e0);
      (void)hipEventDestroy(rc.e1);
    }
    recs.clear();
    for (auto& l : lw) {
      for (auto& w : l.w) free_qweight(w);
      free_qweight(l.xg);
      free_qweight(l.xu);
      free_qweight(l.xgu);
      free_qweight(l.xd);
      free_qweight(l.qkv);
      free_qweight(l.gu);
    }
    free_qweight(tok);
    free_qweight(out);
    for (void* p : allocs) (void)hipFree(p);
    allocs.clear();
  }

  void set_f32(float** dst, const uint8_t* bytes, size_t nbytes, uint32_t type, size_t n, const std::string& name) {
    HOS_REQUIRE(type == GGUF_F32, HOS_E_UNSUPPORTED_QUANT, "tensor '" + name + "' must be F32");
    HOS_REQUIRE(nbytes == n * 4, HOS_E_FORMAT, "tensor '" + name + "' has " + std::to_string(nbytes) + " bytes");
    if (!*dst) *dst = alloc<float>(n);
    HOS_HIP_CHECK(hipMemcpyAsync(*dst, bytes, nbytes, hipMemcpyHostToDevice, st));
    HOS_HIP_CHECK(hipStreamSynchronize(st));
  }
  void set_q(QWeight& w, const uint8_t* bytes, size_t nbytes, uint32_t type, size_t rows, size_t cols, size_t want_r,
             size_t want_c, const std::string& name) {
    HOS_REQUIRE(rows == want_r && cols == want_c, HOS_E_FORMAT,
                "tensor '" + name + "' has shape [" + std::to_string(rows) + "," + std::to_string(cols) +
                    "], expected [" + std::to_string(want_r) + "," + std::to_string(want_c) + "]");
    free_qweight(w);
    upload_qweight(st, bytes, nbytes, type, rows, cols, w);
  }

  void set_tensor(const std::string& name, const uint8_t* bytes, size_t nbytes, uint32_t type, size_t rows,
                  size_t cols) {
    HOS_REQUIRE(bytes != nullptr, HOS_E_INVALID, "null bytes");
    stacks_dirty = true;
    if (name == "token_embd.weight") return set_q(tok, bytes, nbytes, type, rows, cols, V, d, name);
    if (name == "output.weight") {
      set_q(out, bytes, nbytes, type, rows, cols, V, d, name);
      out_set = true;
      return;
    }
    if (name == "output_norm.weight") return set_f32(&out_norm, bytes, nbytes, type, (size_t)d, name);
    HOS_REQUIRE(name.rfind("blk.", 0) == 0, HOS_E_INVALID, "unknown tensor '" + name + "'");
    size_t dot = name.find('.', 4);
    HOS_REQUIRE(dot != std::string::npos, HOS_E_INVALID, "unknown tensor '" + name + "'");
    int li = std::atoi(name.substr(4, dot - 4).c_str());
    HOS_REQUIRE(li >= 0 && li < L, HOS_E_INVALID, "layer index out of range in '" + name + "'");
    std::string leaf = name.substr(dot + 1);
    LayerW& w = lw[li];
    if (leaf == "attn_norm.weight") return set_f32(&w.attn_norm, bytes, nbytes, type, (size_t)d, name);
    if (leaf == "ffn_norm.weight") return set_f32(&w.ffn_norm, bytes, nbytes, type, (size_t)d, name);
    if (leaf == "attn_q.bias") return set_f32(&w.bias[0], bytes, nbytes, type, (size_t)qd, name);
    if (leaf == "attn_k.bias") return set_f32(&w.bias[1], bytes, nbytes, type, (size_t)kvd, name);
    if (leaf == "attn_v.bias") return set_f32(&w.bias[2], bytes, nbytes, type, (size_t)kvd, name);
    if (leaf == "attn_q_norm.weight") return set_f32(&w.q_norm, bytes, nbytes, type, (size_t)qd, name);
    if (leaf == "attn_k_norm.weight") return set_f32(&w.k_norm, bytes, nbytes, type, (size_t)kvd, name);
    if (E) {
      if (leaf == "ffn_gate_inp.weight") return set_f32(&w.router, bytes, nbytes, type, (size_t)E * d, name);
      if (leaf == "ffn_gate_exps.weight") return set_q(w.xg, bytes, nbytes, type, rows, cols, (size_t)E * F, d, name);
      if (leaf == "ffn_up_exps.weight") return set_q(w.xu, bytes, nbytes, type, rows, cols, (size_t)E * F, d, name);
      if (leaf == "ffn_down_exps.weight") return set_q(w.xd, bytes, nbytes, type, rows, cols, (size_t)E * d, F, name);
    }
    const char* names[NT] = {"attn_q.weight", "attn_k.weight", "attn_v.weight", "attn_output.weight",
                             "ffn_gate.weight", "ffn_up.weight", "ffn_down.weight"};
    for (int t = 0; t < NT; t++)
      if (leaf == names[t]) {
        int in, o;
        dims(t, &in, &o);
        return set_q(w.w[t], bytes, nbytes, type, rows, cols, (size_t)o, (size_t)in, name);
      }
    throw Error(HOS_E_INVALID, "unknown tensor '" + name + "'");
  }

  void check_bt(int B, int T) {
    HOS_REQUIRE(B > 0 && T > 0 && T <= c.max_seq && B * T <= Mmax, HOS_E_INVALID,
                "batch " + std::to_string(B) + " x seq " + std::to_string(T) + " exceeds max_batch/max_seq");
  }
};

namespace {
template <class F>
int pguard(hos_peft* p, F&& f) {
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
int lora_index(hos_peft* p, int layer, int target) {
  HOS_REQUIRE(layer >= 0 && layer < p->L && target >= 0 && target < NT, HOS_E_INVALID, "bad layer/target");
  HOS_REQUIRE(p->has(target), HOS_E_INVALID, "target " + std::to_string(target) + " is not adapted");
  return layer * NT + target;
}
void check_ids(hos_peft* p, const int32_t* ids, int n) {
  for (int i = 0; i < n; i++)
    HOS_REQUIRE(ids[i] >= 0 && ids[i] < p->V, HOS_E_INVALID, "token id " + std::to_string(ids[i]) + " out of range");
}
}  // namespace

namespace hos {


// One (layer, target) factor pair of an arena buffer in the reference layout (A [in, r], B [r, out]
// row-major); the device keeps A_tᵀ [r][in] inside its group's At block and B_t as columns of Bcat.
void peft_factor_io(hos_peft* p, PeftBuf which, int layer, int target, float* A, float* B, bool upload) {
  float* base = which == PEFT_PARAM ? p->P : which == PEFT_GRAD ? p->G : which == PEFT_ADAM_M ? p->M1 : p->V1;
  const int i = lora_index(p, layer, target);
  int in, o;
  p->dims(target, &in, &o);
  const int r = p->r;
  const size_t bpitch = (size_t)p->bw(p->group_of(target)) * 4;
  std::vector<float> at;
  if (A) at.resize((size_t)r * in);
  if (upload) {
    if (A) {
      for (int k = 0; k < in; k++)
        for (int j = 0; j < r; j++) at[(size_t)j * in + k] = A[(size_t)k * r + j];
      HOS_HIP_CHECK(hipMemcpyAsync(base + p->offA[i], at.data(), at.size() * 4, hipMemcpyHostToDevice, p->st));
    }
    if (B)
      HOS_HIP_CHECK(hipMemcpy2DAsync(base + p->offB[i], bpitch, B, (size_t)o * 4, (size_t)o * 4, (size_t)r,
                                     hipMemcpyHostToDevice, p->st));
    HOS_HIP_CHECK(hipStreamSynchronize(p->st));
    return;
  }
  if (A) HOS_HIP_CHECK(hipMemcpyAsync(at.data(), base + p->offA[i], at.size() * 4, hipMemcpyDeviceToHost, p->st));
  if (B)
    HOS_HIP_CHECK(hipMemcpy2DAsync(B, (size_t)o * 4, base + p->offB[i], bpitch, (size_t)o * 4, (size_t)r,
                                   hipMemcpyDeviceToHost, p->st));
  HOS_HIP_CHECK(hipStreamSynchronize(p->st));
  if (A)
    for (int k = 0; k < in; k++)
      for (int j = 0; j < r; j++) A[(size_t)k * r + j] = at[(size_t)j * in + k];
}

// An RGA parameter by adapter tensor name (src/peft.rs:741-760), reference layout, from / to an arena buffer.
// genome.0 and wg are stored as they are; rga.{l}.wr [d, K] and rga.{l}.down.{k} [d, b] are rows of the
// stacked transpose RT (rows 0..K-1 and K + k·b .. +b-1); rga.{l}.up.{k} [b, d] is a block of Up's rows.
void peft_rga_io(hos_peft* p, PeftBuf which, const std::string& name, float* data, size_t n, bool upload) {
  HOS_REQUIRE(p->rga, HOS_E_INVALID, "not an RGA model");
  float* base = which == PEFT_PARAM ? p->P : which == PEFT_GRAD ? p->G : which == PEFT_ADAM_M ? p->M1 : p->V1;
  const int d = p->d, K = p->Kg, b = p->bn;
  long long off = -1;
  size_t rows = 0, cols = 0;
  bool trans = false;  // stored transposed: element (i, j) of the [rows, cols] tensor at off + j·d + i
  if (name == "genome.0") {
    off = p->offGen;
    rows = 1;
    cols = RGA_GLEN;
  } else if (name == "wg") {
    off = p->offWg;
    rows = RGA_GLEN;
    cols = K;
  } else if (name.rfind("rga.", 0) == 0) {
    const size_t d1 = name.find('.', 4);
    HOS_REQUIRE(d1 != std::string::npos, HOS_E_INVALID, "unknown adapter tensor '" + name + "'");
    const int l = std::atoi(name.substr(4, d1 - 4).c_str());
    HOS_REQUIRE(l >= 0 && l < p->L, HOS_E_INVALID, "layer out of range in '" + name + "'");
    const std::string leaf = name.substr(d1 + 1);
    if (leaf == "wr") {
      off = p->offRT[l];
      rows = d;
      cols = K;
      trans = true;
    } else if (leaf.rfind("down.", 0) == 0 || leaf.rfind("up.", 0) == 0) {
      const bool dn = leaf[0] == 'd';
      const int k = std::atoi(leaf.substr(dn ? 5 : 3).c_str());
      HOS_REQUIRE(k >= 0 && k < K, HOS_E_INVALID, "gene out of range in '" + name + "'");
      if (dn) {
        off = p->offRT[l] + (long long)(K + k * b) * d;
        rows = d;
        cols = b;
        trans = true;
      } else {
        off = p->offUp[l] + (long long)k * b * d;
        rows = b;
        cols = d;
      }
    }
  }
  HOS_REQUIRE(off >= 0, HOS_E_INVALID, "unknown adapter tensor '" + name + "'");
  HOS_REQUIRE(n == rows * cols, HOS_E_INVALID,
              "adapter tensor '" + name + "' has " + std::to_string(rows * cols) + " elements, got " + std::to_string(n));
  std::vector<float> dev(n);
  if (upload) {
    if (trans)
      for (size_t i = 0; i < rows; i++)
        for (size_t j = 0; j < cols; j++) dev[j * rows + i] = data[i * cols + j];
    else
      std::memcpy(dev.data(), data, n * 4);
    HOS_HIP_CHECK(hipMemcpyAsync(base + off, dev.data(), n * 4, hipMemcpyHostToDevice, p->st));
    HOS_HIP_CHECK(hipStreamSynchronize(p->st));
    return;
  }
  HOS_HIP_CHECK(hipMemcpyAsync(dev.data(), base + off, n * 4, hipMemcpyDeviceToHost, p->st));
  HOS_HIP_CHECK(hipStreamSynchronize(p->st));
  if (trans)
    for (size_t i = 0; i < rows; i++)
      for (size_t j = 0; j < cols; j++) data[i * cols + j] = dev[j * rows + i];
  else
    std::memcpy(data, dev.data(), n * 4);
}

PeftShape peft_shape(const hos_peft* p) {
  PeftShape s{};
  s.L = p->L;
  s.r = p->r;
  s.targets = p->c.lora_targets;
  for (int t = 0; t < NT; t++) p->dims(t, &s.in[t], &s.out[t]);
  s.step = p->adam_t;
  s.lr = p->hyp_host.lr;
  s.wd = p->hyp_host.wd;
  s.vocab = p->V;
  s.dim = p->d;
  s.rga = p->rga;
  return s;
}

std::vector<std::pair<std::string, std::vector<uint32_t>>> peft_rga_tensors(const hos_peft* p, bool param_order) {
  std::vector<std::pair<std::string, std::vector<uint32_t>>> v;
  const uint32_t d = p->d, K = p->Kg, b = p->bn;
  auto rga = [&](int l, const std::string& leaf, uint32_t r, uint32_t c) {
    v.push_back({"rga." + std::to_string(l) + "." + leaf, {r, c}});
  };
  if (!param_order) {
    v.push_back({"genome.0", {1, (uint32_t)RGA_GLEN}});
    v.push_back({"wg", {(uint32_t)RGA_GLEN, K}});
  } else {
    v.push_back({"wg", {(uint32_t)RGA_GLEN, K}});
  }
  for (int l = 0; l < p->L; l++) {
    rga(l, "wr", d, K);
    if (param_order) {
      for (uint32_t k = 0; k < K; k++) rga(l, "down." + std::to_string(k), d, b);
      for (uint32_t k = 0; k < K; k++) rga(l, "up." + std::to_string(k), b, d);
    } else {
      for (uint32_t k = 0; k < K; k++) {
        rga(l, "down." + std::to_string(k), d, b);
        rga(l, "up." + std::to_string(k), b, d);
      }
    }
  }
  if (param_order) v.push_back({"genome.0", {1, (uint32_t)RGA_GLEN}});
  return v;
}

void peft_set_adam_state(hos_peft* p, uint64_t step, float lr, float wd) {
  HOS_REQUIRE(step <= 0x7fffffffull, HOS_E_FORMAT, "optimizer step count out of range");
  p->adam_t = step;
  p->hyp_host.t = (int)step;
  p->hyp_host.lr = lr;
  p->hyp_host.wd = wd;
  HOS_HIP_CHECK(hipMemcpyAsync(p->hyp, &p->hyp_host, sizeof(AdamHyper), hipMemcpyHostToDevice, p->st));
  HOS_HIP_CHECK(hipStreamSynchronize(p->st));
}

// The token embedding dequantized to f32 [vocab, dim] on the host (Model::load's tok_embd).
void peft_token_embedding(hos_peft* p, std::vector<float>& out) {
  HOS_REQUIRE(p->tok.q != nullptr, HOS_E_MISSING_TENSOR, "missing tensor 'token_embd.weight'");
  const size_t n = (size_t)p->V * p->d;
  float* dev = nullptr;
  HOS_HIP_CHECK(hipMalloc(&dev, n * 4));
  out.resize(n);
  launch_dequant(p->tok, dev, p->st);
  hipError_t e = hipMemcpyAsync(out.data(), dev, n * 4, hipMemcpyDeviceToHost, p->st);
  if (e == hipSuccess) e = hipStreamSynchronize(p->st);
  (void)hipFree(dev);
  HOS_HIP_CHECK(e);
}

int peft_call(hos_peft* p, const std::function<void()>& f) { return pguard(p, f); }

}  // namespace hos

extern "C" {

int hos_peft_create(hos_ctx* ctx, const hos_peft_cfg* cfg, hos_peft** out) {
  if (!ctx || !cfg || !out) return HOS_E_INVALID;
  *out = nullptr;
  auto* p = new hos_peft();
  p->ctx = ctx;
  int rc = pguard(p, [&] { p->init(ctx, cfg); });
  if (rc) {
    // keep the error readable through the context
    std::fprintf(stderr, "hos_peft_create: %s\n", p->err.c_str());
    p->release();
    delete p;
    return rc;
  }
  *out = p;
  return HOS_OK;
}

void hos_peft_destroy(hos_peft* p) {
  if (!p) return;
  (void)hipSetDevice(hos_internal_device(p->ctx));
  p->release();
  delete p;
}

const char* hos_peft_last_error(const hos_peft* p) { return p ? p->err.c_str() : "null model"; }

int hos_peft_set_tensor(hos_peft* p, const char* name, const uint8_t* bytes, size_t nbytes, uint32_t type, size_t rows,
                        size_t cols) {
  return pguard(p, [&] {
    HOS_REQUIRE(name != nullptr, HOS_E_INVALID, "null name");
    p->set_tensor(name, bytes, nbytes, type, rows, cols);
  });
}

int hos_peft_set_lora(hos_peft* p, int layer, int target, const float* A, const float* B) {
  return pguard(p, [&] {
    HOS_REQUIRE(A && B, HOS_E_INVALID, "null factor");
    hos::peft_factor_io(p, hos::PEFT_PARAM, layer, target, const_cast<float*>(A), const_cast<float*>(B), true);
  });
}
int hos_peft_get_lora(hos_peft* p, int layer, int target, float* A, float* B) {
  return pguard(p, [&] { hos::peft_factor_io(p, hos::PEFT_PARAM, layer, target, A, B, false); });
}
int hos_peft_get_lora_grad(hos_peft* p, int layer, int target, float* dA, float* dB) {
  return pguard(p, [&] { hos::peft_factor_io(p, hos::PEFT_GRAD, layer, target, dA, dB, false); });
}

int hos_peft_set_adapter(hos_peft* p, const char* name, const float* data, size_t n) {
  return pguard(p, [&] {
    HOS_REQUIRE(name && data, HOS_E_INVALID, "null pointer");
    hos::peft_rga_io(p, hos::PEFT_PARAM, name, const_cast<float*>(data), n, true);
  });
}
int hos_peft_get_adapter(hos_peft* p, const char* name, float* value, float* grad, size_t n) {
  return pguard(p, [&] {
    HOS_REQUIRE(name != nullptr, HOS_E_INVALID, "null name");
    if (value) hos::peft_rga_io(p, hos::PEFT_PARAM, name, value, n, false);
    if (grad) hos::peft_rga_io(p, hos::PEFT_GRAD, name, grad, n, false);
  });
}

int hos_peft_loss_grad(hos_peft* p, const int32_t* ids, const int32_t* targets, int B, int T, float* loss) {
  return pguard(p, [&] {
    HOS_REQUIRE(ids && targets && loss, HOS_E_INVALID, "null pointer");
    p->check_ready();
    p->check_bt(B, T);
    check_ids(p, ids, B * T);
    check_ids(p, targets, B * T);
    HOS_HIP_CHECK(hipMemcpyAsync(p->ids, ids, (size_t)B * T * 4, hipMemcpyHostToDevice, p->st));
    HOS_HIP_CHECK(hipMemcpyAsync(p->tgts, targets, (size_t)B * T * 4, hipMemcpyHostToDevice, p->st));
    p->forward(B, T, false);
    p->loss_backward(B, T);
    HOS_HIP_CHECK(hipMemcpyAsync(loss, p->loss, 4, hipMemcpyDeviceToHost, p->st));
    HOS_HIP_CHECK(hipStreamSynchronize(p->st));
  });
}

int hos_peft_adamw(hos_peft* p, float lr, float wd) {
  return pguard(p, [&] {
    p->adamw(lr, wd);
    HOS_HIP_CHECK(hipStreamSynchronize(p->st));
  });
}

int hos_peft_step_dev(hos_peft* p, const int32_t* ids_dev, const int32_t* targets_dev, int B, int T, float lr, float wd,
                      float* loss_dev) {
  return pguard(p, [&] {
    HOS_REQUIRE(ids_dev && targets_dev, HOS_E_INVALID, "null pointer");
    p->check_ready();
    p->check_bt(B, T);
    p->step(ids_dev, targets_dev, B, T, lr, wd, loss_dev);
  });
}

int hos_peft_use_graph(hos_peft* p, int enable) {
  return pguard(p, [&] { p->use_graph = enable != 0; });
}

int hos_peft_logits(hos_peft* p, const int32_t* ids, int T, float* out) {
  return pguard(p, [&] {
    HOS_REQUIRE(ids && out, HOS_E_INVALID, "null pointer");
    p->check_ready();
    p->check_bt(1, T);
    check_ids(p, ids, T);
    HOS_HIP_CHECK(hipMemcpyAsync(p->ids, ids, (size_t)T * 4, hipMemcpyHostToDevice, p->st));
    p->forward(1, T, true);
    HOS_HIP_CHECK(hipMemcpyAsync(out, p->logits, (size_t)T * p->V * 4, hipMemcpyDeviceToHost, p->st));
    HOS_HIP_CHECK(hipStreamSynchronize(p->st));
  });
}

int hos_peft_profile(hos_peft* p, int enable) {
  return pguard(p, [&] {
    p->collect_prof();
    p->prof = enable != 0;
    if (enable) p->acc.clear();
  });
}

int hos_peft_profile_only(hos_peft* p, const char* cls) {
  return pguard(p, [&] { p->prof_only = cls ? cls : ""; });
}

int hos_peft_kernel_stats(hos_peft* p, const char* cls, long long* launches, double* total_ms, double* flops,
                          double* bytes) {
  return pguard(p, [&] {
    HOS_REQUIRE(cls != nullptr, HOS_E_INVALID, "null class");
    p->collect_prof();
    auto it = p->acc.find(cls);
    ProfAcc a = it == p->acc.end() ? ProfAcc{} : it->second;
    if (launches) *launches = a.launches;
    if (total_ms) *total_ms = a.ms;
    if (flops) *flops = a.flops;
    if (bytes) *bytes = a.bytes;
  });
}

}  // extern "C"
