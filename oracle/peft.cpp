// ORACLE — test infrastructure only. CPU restatement of HOS's LoRA PEFT model and
// training step:
//   t_const (frozen base, transposed f32 [in,out])   src/peft.rs:24-33
//   PeftModel::build_multi (LoRA branch)              src/peft.rs:134-231
//   PeftModel::loss_g / forward                       src/peft.rs:447-604
//   cmd_peft step loop (zero_grad, accumulate, AdamW) src/main.rs:2583-2601
//   train_minibatch                                   src/train.rs:33-52
//   RGA adapters (PeftModel "rga": genome-regulated gene bank) src/peft.rs:61-96, 200-215, 491-499, 565-584,
//     params order :283-311, loss_g's gate sparsity term :447-459 (one genome; no clones, no grown FFN)
// Extensions the benchmark configs need, each reducing exactly to the reference when
// switched to the reference's setting:
//   * LoRA targets beyond q/v (k, o, gate, up, down), applied as `y += (x·A·B)·(α/r)`
//     right after the base projection, in the order q, k, v (then biases), o, gate, up, down;
//     targets = q|v reproduces src/peft.rs:508-512 exactly.
//   * LoRA A/B supplied by the caller (the reference draws A with Tensor::randn,
//     src/tensor.rs:241-256, and B = 0; randn_uniform restates that draw).
#include <algorithm>
#include <map>
#include <string>

#include "autograd.hpp"
#include "oracle.h"

namespace orc {

struct Lora {
  Tensor A, B;  // A [in, r], B [r, out]
};

// Experts of one MoE projection, kept in their GGUF bytes and dequantized per forward (QExperts,
// src/model.rs:659-671): expert e is the e-th [rows, cols] block.
struct Experts {
  std::vector<uint8_t> bytes;
  uint32_t type = 0;
  size_t rows = 0, cols = 0, expert_bytes = 0;
  explicit operator bool() const { return !bytes.empty(); }
  // expert e as a frozen [cols, rows] constant (t_const of its [rows, cols] matrix)
  Tensor expert(size_t e) const;
};

struct BaseLayer {
  Tensor attn_norm, wq, wk, wv, wo, bq, bk, bv, ffn_norm, w_gate, w_up, w_down;
  Tensor q_norm, k_norm;  // OLMoE QK-norm weights (absent for other models)
  Tensor router;          // MoE router as [dim, n_experts] (ffn_gate_inp.weight [n_experts, dim])
  Experts gate_x, up_x, down_x;
  Lora lora[7];  // q k v o gate up down
};

// RgaLayer (src/peft.rs:61-66): gate weights and the gene bank of one layer.
struct RgaLayer {
  Tensor wr;                     // [dim, K]
  std::vector<Tensor> down, up;  // K x [dim, b], K x [b, dim]
};

struct Model {
  orc_cfg c;
  Tensor tok_embd, out_norm, out;
  std::vector<BaseLayer> layers;
  // RGA (src/peft.rs:77-83): genome [1, GLEN], wg [GLEN, K], per-layer banks
  Tensor genome, wg;
  std::vector<RgaLayer> rga;
  bool is_rga() const { return c.rga_genes > 0; }
  std::unique_ptr<AdamW> opt;
  // Full-parameter finetune (FtModel, src/finetune.rs:62-108): every weight a trainable f32 parameter,
  // the head an untied copy when the file ties it; no LoRA.
  bool full = false;
  float lora_scale() const { return c.lora_alpha / (float)c.lora_rank; }

  std::vector<Tensor> params() const {
    if (full) {  // FtModel::params order, src/finetune.rs:181-200
      std::vector<Tensor> p{tok_embd, out_norm, out};
      for (auto& l : layers) {
        for (const Tensor& t : {l.attn_norm, l.wq, l.wk, l.wv, l.wo, l.ffn_norm, l.w_gate, l.w_up, l.w_down}) p.push_back(t);
        for (const Tensor& b : {l.bq, l.bk, l.bv})
          if (b) p.push_back(b);
      }
      return p;
    }
    // RGA: params_bank (wg, then per layer wr, down..., up...) then the genome (src/peft.rs:283-311)
    if (is_rga()) {
      std::vector<Tensor> p{wg};
      for (auto& l : rga) {
        p.push_back(l.wr);
        for (auto& t : l.down) p.push_back(t);
        for (auto& t : l.up) p.push_back(t);
      }
      p.push_back(genome);
      return p;
    }
    // LoRA factors per layer, in target order (src/peft.rs:295-302 lists aq,bq,av,bv).
    std::vector<Tensor> p;
    for (auto& l : layers)
      for (int t = 0; t < 7; t++)
        if (l.lora[t].A) {
          p.push_back(l.lora[t].A);
          p.push_back(l.lora[t].B);
        }
    return p;
  }
};

static const int kTargetBits[7] = {ORC_T_Q, ORC_T_K, ORC_T_V, ORC_T_O, ORC_T_GATE, ORC_T_UP, ORC_T_DOWN};

void target_dims(const orc_cfg& c, int t, size_t* in, size_t* out) {
  size_t d = c.dim, qd = (size_t)c.n_heads * c.head_dim, kvd = (size_t)c.n_kv_heads * c.head_dim, f = c.ffn_dim;
  switch (t) {
    case 0: *in = d; *out = qd; break;
    case 1: *in = d; *out = kvd; break;
    case 2: *in = d; *out = kvd; break;
    case 3: *in = qd; *out = d; break;
    case 4: *in = d; *out = f; break;
    case 5: *in = d; *out = f; break;
    default: *in = f; *out = d; break;
  }
}

Model* model_create(const orc_cfg* cfg) {
  auto* m = new Model();
  m->c = *cfg;
  m->layers.resize(cfg->n_layers);
  size_t r = cfg->lora_rank;
  for (auto& l : m->layers)
    for (int t = 0; t < 7; t++)
      if (cfg->lora_targets & kTargetBits[t]) {
        size_t in, out;
        target_dims(*cfg, t, &in, &out);
        l.lora[t].A = param(std::vector<float>(in * r, 0.0f), {in, r});
        l.lora[t].B = param(std::vector<float>(r * out, 0.0f), {r, out});
      }
  if (cfg->rga_genes > 0) {  // shapes of src/peft.rs:200-215 (GLEN = 8); values come from the caller
    const size_t k = cfg->rga_genes, b = cfg->rga_bottleneck, d = cfg->dim, glen = 8;
    m->genome = param(std::vector<float>(glen, 0.0f), {1, glen});
    m->wg = param(std::vector<float>(glen * k, 0.0f), {glen, k});
    m->rga.resize(cfg->n_layers);
    for (auto& l : m->rga) {
      l.wr = param(std::vector<float>(d * k, 0.0f), {d, k});
      for (size_t kk = 0; kk < k; kk++) {
        l.down.push_back(param(std::vector<float>(d * b, 0.0f), {d, b}));
        l.up.push_back(param(std::vector<float>(b * d, 0.0f), {b, d}));
      }
    }
  }
  return m;
}

// t_const, src/peft.rs:24-33: W [out,in] row-major (GGUF) -> constant [in,out]; transposed_param
// (src/finetune.rs:26-35) is the same transpose as a trainable parameter.
static Tensor t_const(const std::vector<float>& d, size_t out, size_t inn, bool trainable = false) {
  std::vector<float> t(out * inn);
  for (size_t o = 0; o < out; o++)
    for (size_t i = 0; i < inn; i++) t[i * out + o] = d[o * inn + i];
  return tnew(std::move(t), {inn, out}, trainable);
}

Tensor Experts::expert(size_t e) const {
  std::vector<float> f(rows * cols);
  dequant_into(bytes.data() + e * expert_bytes, type, rows * cols, f.data());
  return t_const(f, rows, cols);
}

// Tensor names follow GGUF (src/model.rs:760-880). Bytes are dequantized with the
// restated dequant_into, as Weight::to_f32 does (src/model.rs:251-273).
int model_set_tensor(Model* m, const std::string& name, const uint8_t* bytes, uint32_t type, size_t rows, size_t cols) {
  {
    // MoE expert stacks stay quantized (src/model.rs:815-833): rows = n_experts · per-expert rows.
    const char* stacks[3] = {"ffn_gate_exps.weight", "ffn_up_exps.weight", "ffn_down_exps.weight"};
    for (int k = 0; k < 3; k++) {
      const std::string sfx = std::string(".") + stacks[k];
      if (name.size() > sfx.size() && name.compare(name.size() - sfx.size(), sfx.size(), sfx) == 0) {
        const orc_cfg& c = m->c;
        size_t dot = name.find('.', 4);
        int li = std::stoi(name.substr(4, dot - 4));
        if (li < 0 || li >= c.n_layers || c.n_experts <= 0 || rows % (size_t)c.n_experts) return ORC_E_INVALID;
        BaseLayer& l = m->layers[li];
        Experts& x = k == 0 ? l.gate_x : (k == 1 ? l.up_x : l.down_x);
        x.type = type;
        x.rows = rows / c.n_experts;
        x.cols = cols;
        x.expert_bytes = bytes_for(type, x.rows * cols);
        if (!x.expert_bytes) return ORC_E_UNSUPPORTED_QUANT;
        x.bytes.assign(bytes, bytes + x.expert_bytes * c.n_experts);
        return 0;
      }
    }
  }
  std::vector<float> f(rows * cols);
  int rc = dequant_into(bytes, type, rows * cols, f.data());
  if (rc) return rc;
  const orc_cfg& c = m->c;
  const bool tr = m->full;
  auto vec1 = [&](std::vector<float> v) { return tnew(std::move(v), {rows * cols}, tr); };
  if (name == "token_embd.weight") {
    m->tok_embd = tnew(f, {rows, cols}, tr);
    if (!m->out) m->out = t_const(f, rows, cols, tr);  // tied head until output.weight arrives
    return 0;
  }
  if (name == "output.weight") { m->out = t_const(f, rows, cols, tr); return 0; }
  if (name == "output_norm.weight") { m->out_norm = vec1(f); return 0; }
  if (name.rfind("blk.", 0) != 0) return ORC_E_INVALID;
  size_t dot = name.find('.', 4);
  int li = std::stoi(name.substr(4, dot - 4));
  if (li < 0 || li >= c.n_layers) return ORC_E_INVALID;
  std::string leaf = name.substr(dot + 1);
  BaseLayer& l = m->layers[li];
  if (leaf == "attn_norm.weight") l.attn_norm = vec1(f);
  else if (leaf == "ffn_norm.weight") l.ffn_norm = vec1(f);
  else if (leaf == "attn_q.weight") l.wq = t_const(f, rows, cols, tr);
  else if (leaf == "attn_k.weight") l.wk = t_const(f, rows, cols, tr);
  else if (leaf == "attn_v.weight") l.wv = t_const(f, rows, cols, tr);
  else if (leaf == "attn_output.weight") l.wo = t_const(f, rows, cols, tr);
  else if (leaf == "ffn_gate.weight") l.w_gate = t_const(f, rows, cols, tr);
  else if (leaf == "ffn_up.weight") l.w_up = t_const(f, rows, cols, tr);
  else if (leaf == "ffn_down.weight") l.w_down = t_const(f, rows, cols, tr);
  else if (leaf == "attn_q.bias") l.bq = vec1(f);
  else if (leaf == "attn_k.bias") l.bk = vec1(f);
  else if (leaf == "attn_v.bias") l.bv = vec1(f);
  else if (leaf == "attn_q_norm.weight") l.q_norm = constant(f, {rows * cols});
  else if (leaf == "attn_k_norm.weight") l.k_norm = constant(f, {rows * cols});
  else if (leaf == "ffn_gate_inp.weight") l.router = t_const(f, rows, cols);
  else return ORC_E_INVALID;
  return 0;
}

static Tensor lora_apply(const Model* m, const Lora& lo, const Tensor& y, const Tensor& x) {
  if (!lo.A) return y;
  return add(y, scale(matmul(matmul(x, lo.A), lo.B), m->lora_scale()));
}

// Mixture-of-experts FFN, src/forward.rs:542-572 over a batch of rows: router logits, softmax over all
// experts, the top n_experts_used by probability (a stable descending sort, ties in expert order), and
// Σ p·expert_e(xn) over the selected experts with the raw probabilities; each expert is a SwiGLU FFN
// (silu(x·gate_e)·(x·up_e))·down_e on its dequantized weights, run on the rows routed to it. The
// routing is piecewise constant: gradients flow through the probabilities and the experts only.
static Tensor moe_ffn(const Model* m, const BaseLayer& bl, const Tensor& xn) {
  const orc_cfg& c = m->c;
  const size_t T = xn->shape[0], d = xn->shape[1], E = c.n_experts, K = c.n_experts_used;
  Tensor p = softmax_rows(matmul(xn, bl.router));
  std::vector<std::vector<size_t>> rows(E);
  std::vector<std::vector<std::pair<size_t, size_t>>> sel(T);
  for (size_t t = 0; t < T; t++) {
    std::vector<size_t> idx(E);
    for (size_t e = 0; e < E; e++) idx[e] = e;
    const float* pr = &p->data[t * E];
    std::stable_sort(idx.begin(), idx.end(), [pr](size_t a, size_t b) { return pr[a] > pr[b]; });
    for (size_t s = 0; s < K; s++) {
      const size_t e = idx[s];
      sel[t].push_back({e, rows[e].size()});
      rows[e].push_back(t);
    }
  }
  std::vector<Tensor> ys(E);
  for (size_t e = 0; e < E; e++) {
    if (rows[e].empty()) continue;
    Tensor xe = gather_rows(xn, rows[e]);
    Tensor h = mul(silu(matmul(xe, bl.gate_x.expert(e))), matmul(xe, bl.up_x.expert(e)));
    ys[e] = matmul(h, bl.down_x.expert(e));
  }
  return moe_mix(ys, p, sel, d);
}

// PeftModel::forward, src/peft.rs:474-604 -> logits; gate_means receives the per-layer RGA gate means.
Tensor model_forward(const Model* m, const std::vector<size_t>& ids, std::vector<Tensor>* gate_means) {
  const orc_cfg& c = m->c;
  size_t t = ids.size(), hd = c.head_dim, nh = c.n_heads, nkv = c.n_kv_heads;
  size_t qd = nh * hd, group = nh / nkv;
  float sc = 1.0f / std::sqrt((float)hd);
  std::vector<size_t> pos(t);
  for (size_t i = 0; i < t; i++) pos[i] = i;
  std::vector<float> mk(nh * t * t, 0.0f);
  for (size_t h = 0; h < nh; h++)
    for (size_t i = 0; i < t; i++)
      for (size_t j = i + 1; j < t; j++) mk[(h * t + i) * t + j] = -1e9f;
  Tensor mask = constant(std::move(mk), {nh * t, t});

  // the genome's per-gene gate bias [K] (src/peft.rs:491-499)
  Tensor g_bias;
  if (m->is_rga()) g_bias = reshape(matmul(m->genome, m->wg), {(size_t)c.rga_genes});

  Tensor x = embedding(m->tok_embd, ids);
  for (size_t li = 0; li < m->layers.size(); li++) {
    const BaseLayer& bl = m->layers[li];
    Tensor xn = rmsnorm_eps(x, bl.attn_norm, c.rms_eps);
    Tensor q = matmul(xn, bl.wq);
    Tensor k = matmul(xn, bl.wk);
    Tensor v = matmul(xn, bl.wv);
    q = lora_apply(m, bl.lora[0], q, xn);
    k = lora_apply(m, bl.lora[1], k, xn);
    v = lora_apply(m, bl.lora[2], v, xn);
    if (bl.bq) q = add(q, bl.bq);
    if (bl.bk) k = add(k, bl.bk);
    if (bl.bv) v = add(v, bl.bv);
    // OLMoE QK-norm: RMSNorm over the full q / k projections before RoPE (src/forward.rs:487-493), as the
    // autograd rmsnorm_eps
    if (c.qk_norm) {
      q = rmsnorm_eps(q, bl.q_norm, c.rms_eps);
      k = rmsnorm_eps(k, bl.k_norm, c.rms_eps);
    }
    q = rope(q, nh, hd, c.rope_base, c.rope_neox != 0, pos);
    k = rope(k, nkv, hd, c.rope_base, c.rope_neox != 0, pos);
    Tensor qh = reshape(transpose12_4d(reshape(q, {1, t, nh, hd})), {nh, t, hd});
    Tensor kh = reshape(transpose12_4d(reshape(k, {1, t, nkv, hd})), {nkv, t, hd});
    Tensor vh = reshape(transpose12_4d(reshape(v, {1, t, nkv, hd})), {nkv, t, hd});
    kh = repeat_interleave_dim0(kh, group);
    vh = repeat_interleave_dim0(vh, group);
    Tensor scores = scale(bmm(qh, transpose_last2(kh)), sc);
    Tensor att = reshape(softmax_rows(add(reshape(scores, {nh * t, t}), mask)), {nh, t, t});
    Tensor ctx = reshape(transpose12_4d(reshape(bmm(att, vh), {1, nh, t, hd})), {t, qd});
    Tensor o = lora_apply(m, bl.lora[3], matmul(ctx, bl.wo), ctx);
    x = add(x, o);
    Tensor xn2 = rmsnorm_eps(x, bl.ffn_norm, c.rms_eps);
    if (c.n_experts > 0) {
      x = add(x, moe_ffn(m, bl, xn2));
      continue;
    }
    Tensor gt = lora_apply(m, bl.lora[4], matmul(xn2, bl.w_gate), xn2);
    Tensor up = lora_apply(m, bl.lora[5], matmul(xn2, bl.w_up), xn2);
    Tensor hmid = mul(silu(gt), up);
    Tensor dn = lora_apply(m, bl.lora[6], matmul(hmid, bl.w_down), hmid);
    x = add(x, dn);
    // RGA: genome-regulated sparse gene expression on the residual (src/peft.rs:565-584)
    if (m->is_rga()) {
      const RgaLayer& rl = m->rga[li];
      Tensor gate = sigmoid(add(matmul(x, rl.wr), g_bias));  // [t, K]
      Tensor upd;
      for (int kk = 0; kk < c.rga_genes; kk++) {
        Tensor gene = matmul(relu(matmul(x, rl.down[kk])), rl.up[kk]);  // [t, dim]
        Tensor gated = mul_broadcast(gene, col(gate, (size_t)kk));
        upd = upd ? add(upd, gated) : gated;
      }
      x = add(x, upd);
      if (gate_means) gate_means->push_back(mean(gate));
    }
  }
  return matmul(rmsnorm_eps(x, m->out_norm, c.rms_eps), m->out);
}

// One optimizer-step's gradient: zero_grad, then for each of the B sequences
// loss(seq)·(1/B) backward, summing the scaled losses (src/main.rs:2583-2596).
float model_loss_grad(Model* m, const int32_t* ids, const int32_t* tgts, int B, int T) {
  for (auto& p : m->params()) zero_grad(p);
  float mean_loss = 0.0f;
  for (int b = 0; b < B; b++) {
    std::vector<size_t> id(T), tg(T);
    for (int i = 0; i < T; i++) {
      id[i] = (size_t)ids[b * T + i];
      tg[i] = (size_t)tgts[b * T + i];
    }
    // loss_g (src/peft.rs:447-459): cross-entropy + (RGA, lambda > 0) (λ/L)·Σ_l mean(gate_l)
    std::vector<Tensor> gm;
    Tensor lossb = cross_entropy(model_forward(m, id, &gm), tg);
    const float lambda = m->is_rga() ? m->c.rga_lambda : 0.0f;
    if (lambda > 0.0f && !gm.empty()) {
      Tensor sgm = gm[0];
      for (size_t i = 1; i < gm.size(); i++) sgm = add(sgm, gm[i]);
      lossb = add(lossb, scale(sgm, lambda / (float)gm.size()));
    }
    Tensor loss = scale(lossb, 1.0f / (float)B);
    backward(loss);
    mean_loss += loss->data[0];
  }
  return mean_loss;
}

// AdamW::step over the LoRA params; decay = (ndim == 2), src/main.rs:2571 (all LoRA
// factors are 2-D). The optimizer is created on first use with (lr, wd), as cmd_peft
// builds it once before the loop (src/main.rs:2581).
void model_adamw(Model* m, float lr, float wd) {
  auto ps = m->params();
  if (!m->opt) m->opt.reset(new AdamW(ps, lr, wd));
  m->opt->lr = lr;
  m->opt->wd = wd;
  std::vector<bool> decay(ps.size());
  for (size_t i = 0; i < ps.size(); i++) decay[i] = ps[i]->shape.size() == 2;
  m->opt->step(ps, decay);
}

}  // namespace orc

// ---- LoRA factor access for the extern "C" surface ----
extern "C" {
// Full-parameter finetune model (FtModel): set tensors, loss_grad and adamw as for the LoRA model.
void* orc_ft_create(const orc_cfg* cfg) {
  orc_cfg c = *cfg;
  c.lora_targets = 0;
  auto* m = orc::model_create(&c);
  m->full = true;
  return m;
}
// Value (and gradient) of one parameter by its GGUF tensor name, in the GGUF layout ([out, in] row-major
// for matrices; the model keeps them transposed as FtModel does).
int orc_ft_get(void* mh, const char* cname, float* value, float* grad) {
  auto* m = (orc::Model*)mh;
  std::string name(cname);
  orc::Tensor t;
  bool transposed = true;
  if (name == "token_embd.weight") { t = m->tok_embd; transposed = false; }
  else if (name == "output.weight") t = m->out;
  else if (name == "output_norm.weight") { t = m->out_norm; transposed = false; }
  else if (name.rfind("blk.", 0) == 0) {
    size_t dot = name.find('.', 4);
    int li = std::stoi(name.substr(4, dot - 4));
    if (li < 0 || li >= m->c.n_layers) return ORC_E_INVALID;
    auto& l = m->layers[li];
    std::string leaf = name.substr(dot + 1);
    if (leaf == "attn_norm.weight") { t = l.attn_norm; transposed = false; }
    else if (leaf == "ffn_norm.weight") { t = l.ffn_norm; transposed = false; }
    else if (leaf == "attn_q.bias") { t = l.bq; transposed = false; }
    else if (leaf == "attn_k.bias") { t = l.bk; transposed = false; }
    else if (leaf == "attn_v.bias") { t = l.bv; transposed = false; }
    else if (leaf == "attn_q.weight") t = l.wq;
    else if (leaf == "attn_k.weight") t = l.wk;
    else if (leaf == "attn_v.weight") t = l.wv;
    else if (leaf == "attn_output.weight") t = l.wo;
    else if (leaf == "ffn_gate.weight") t = l.w_gate;
    else if (leaf == "ffn_up.weight") t = l.w_up;
    else if (leaf == "ffn_down.weight") t = l.w_down;
  }
  if (!t) return ORC_E_INVALID;
  auto put = [&](const std::vector<float>& src, float* dst) {
    if (!dst) return;
    if (!transposed) {
      std::memcpy(dst, src.data(), src.size() * 4);
      return;
    }
    const size_t inn = t->shape[0], out = t->shape[1];
    for (size_t o = 0; o < out; o++)
      for (size_t i = 0; i < inn; i++) dst[o * inn + i] = src[i * out + o];
  };
  put(t->data, value);
  put(t->grad, grad);
  return 0;
}
void orc_model_destroy(void* mh) { delete (orc::Model*)mh; }
// An RGA parameter by its adapter tensor name (PeftModel::adapter_tensors, src/peft.rs:741-760): genome.0, wg,
// rga.{l}.wr, rga.{l}.down.{k}, rga.{l}.up.{k}, in the reference layout. set != 0 writes value from the caller;
// otherwise value and grad (each may be NULL) are read. n must equal the tensor's element count.
int orc_model_rga_tensor(void* mh, const char* cname, float* value, float* grad, size_t n, int set) {
  auto* m = (orc::Model*)mh;
  if (!m->is_rga()) return ORC_E_INVALID;
  std::string name(cname);
  orc::Tensor t;
  if (name == "genome.0") t = m->genome;
  else if (name == "wg") t = m->wg;
  else if (name.rfind("rga.", 0) == 0) {
    size_t d1 = name.find('.', 4);
    if (d1 == std::string::npos) return ORC_E_INVALID;
    int li = std::stoi(name.substr(4, d1 - 4));
    if (li < 0 || li >= m->c.n_layers) return ORC_E_INVALID;
    std::string leaf = name.substr(d1 + 1);
    auto& l = m->rga[li];
    if (leaf == "wr") t = l.wr;
    else if (leaf.rfind("down.", 0) == 0 || leaf.rfind("up.", 0) == 0) {
      const bool dn = leaf[0] == 'd';
      int k = std::stoi(leaf.substr(dn ? 5 : 3));
      if (k < 0 || k >= m->c.rga_genes) return ORC_E_INVALID;
      t = dn ? l.down[k] : l.up[k];
    }
  }
  if (!t || t->data.size() != n) return ORC_E_INVALID;
  if (set) {
    std::memcpy(t->data.data(), value, n * 4);
    return 0;
  }
  if (value) std::memcpy(value, t->data.data(), n * 4);
  if (grad) std::memcpy(grad, t->grad.data(), n * 4);
  return 0;
}
int orc_model_set_lora(void* mh, int layer, int target, const float* A, const float* B) {
  auto* m = (orc::Model*)mh;
  if (layer < 0 || layer >= m->c.n_layers || target < 0 || target > 6) return ORC_E_INVALID;
  auto& lo = m->layers[layer].lora[target];
  if (!lo.A) return ORC_E_INVALID;
  std::memcpy(lo.A->data.data(), A, lo.A->data.size() * 4);
  std::memcpy(lo.B->data.data(), B, lo.B->data.size() * 4);
  return 0;
}
int orc_model_get_lora(void* mh, int layer, int target, float* A, float* B) {
  auto* m = (orc::Model*)mh;
  if (layer < 0 || layer >= m->c.n_layers || target < 0 || target > 6) return ORC_E_INVALID;
  auto& lo = m->layers[layer].lora[target];
  if (!lo.A) return ORC_E_INVALID;
  if (A) std::memcpy(A, lo.A->data.data(), lo.A->data.size() * 4);
  if (B) std::memcpy(B, lo.B->data.data(), lo.B->data.size() * 4);
  return 0;
}
int orc_model_get_lora_grad(void* mh, int layer, int target, float* dA, float* dB) {
  auto* m = (orc::Model*)mh;
  if (layer < 0 || layer >= m->c.n_layers || target < 0 || target > 6) return ORC_E_INVALID;
  auto& lo = m->layers[layer].lora[target];
  if (!lo.A) return ORC_E_INVALID;
  if (dA) std::memcpy(dA, lo.A->grad.data(), lo.A->grad.size() * 4);
  if (dB) std::memcpy(dB, lo.B->grad.data(), lo.B->grad.size() * 4);
  return 0;
}
}
