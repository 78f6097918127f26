// ORACLE — test infrastructure only. extern "C" surface of the CPU restatement, loaded
// with ctypes by tests/ and bench.py's cpu_baseline leg. Never linked by the product.
#include <string>

#include "autograd.hpp"
#include "oracle.h"

namespace orc {
struct Model;
Model* model_create(const orc_cfg* cfg);
int model_set_tensor(Model* m, const std::string& name, const uint8_t* bytes, uint32_t type, size_t rows, size_t cols);
Tensor model_forward(const Model* m, const std::vector<size_t>& ids, std::vector<Tensor>* gate_means);
float model_loss_grad(Model* m, const int32_t* ids, const int32_t* tgts, int B, int T);
void model_adamw(Model* m, float lr, float wd);
void target_dims(const orc_cfg& c, int t, size_t* in, size_t* out);
}  // namespace orc

using namespace orc;

namespace {
std::vector<float> vec(const float* p, size_t n) { return std::vector<float>(p, p + n); }
void put(const std::vector<float>& v, float* dst) {
  if (dst) std::memcpy(dst, v.data(), v.size() * 4);
}
// Seed the output node's gradient with `gout` and run the reverse pass from it, the way
// backward() does from a scalar (src/tensor.rs:2844-2881) but with a given upstream grad.
void backward_from(const Tensor& out, const float* gout) {
  std::vector<Tensor> topo;
  std::unordered_set<const Node*> vis;
  std::function<void(const Tensor&)> dfs = [&](const Tensor& t) {
    if (vis.count(t.get())) return;
    vis.insert(t.get());
    for (auto& p : t->parents) dfs(p);
    topo.push_back(t);
  };
  dfs(out);
  std::memcpy(out->grad.data(), gout, out->grad.size() * 4);
  for (auto it = topo.rbegin(); it != topo.rend(); ++it)
    if ((*it)->backward) {
      std::vector<float> g = (*it)->grad;
      (*it)->backward(g, (*it)->parents);
    }
}
}  // namespace

struct orc_model;  // opaque handle = orc::Model

#include <omp.h>

extern "C" {

float orc_f16_to_f32(uint16_t h) { return f16_to_f32(h); }
uint16_t orc_f32_to_f16(float f) { return f32_to_f16(f); }
// OpenMP threads for the following calls (n <= 0 leaves the setting); returns the count now in effect.
int orc_set_threads(int n) {
  if (n > 0) omp_set_num_threads(n);
  return omp_get_max_threads();
}
size_t orc_bytes_for(uint32_t type, size_t n) { return bytes_for(type, n); }
int orc_dequant(const uint8_t* bytes, uint32_t type, size_t n, float* out) { return dequant_into(bytes, type, n, out); }
int orc_quantize(const float* x, size_t n, uint32_t type, uint8_t* out) { return quantize(x, n, type, out); }
void orc_pack_scales_mins(const uint8_t* s, const uint8_t* m, uint8_t* q) { pack_scales_mins(s, m, q); }
void orc_qkx_scale_min(const float* x, int len, int nmax, float* s, float* m) { qkx_scale_min(x, len, nmax, s, m); }

// ---- single-op forward + backward with a given upstream gradient ----

int orc_op_matmul(const float* a, size_t m, size_t k, const float* b, size_t n, const float* gout, float* out,
                  float* da, float* db) {
  Tensor A = param(vec(a, m * k), {m, k}), B = param(vec(b, k * n), {k, n});
  Tensor Y = matmul(A, B);
  put(Y->data, out);
  if (gout) {
    backward_from(Y, gout);
    put(A->grad, da);
    put(B->grad, db);
  }
  return 0;
}

int orc_op_rmsnorm(const float* x, const float* w, size_t r, size_t d, float eps, const float* gout, float* out,
                   float* gx, float* gw) {
  Tensor X = param(vec(x, r * d), {r, d}), W = param(vec(w, d), {d});
  Tensor Y = rmsnorm_eps(X, W, eps);
  put(Y->data, out);
  if (gout) {
    backward_from(Y, gout);
    put(X->grad, gx);
    put(W->grad, gw);
  }
  return 0;
}

int orc_op_rope(const float* x, size_t rows, size_t nh, size_t hd, float base, int neox, const int32_t* pos,
                const float* gout, float* out, float* dx) {
  Tensor X = param(vec(x, rows * nh * hd), {rows, nh * hd});
  std::vector<size_t> p(rows);
  for (size_t i = 0; i < rows; i++) p[i] = (size_t)pos[i];
  Tensor Y = rope(X, nh, hd, base, neox != 0, p);
  put(Y->data, out);
  if (gout) {
    backward_from(Y, gout);
    put(X->grad, dx);
  }
  return 0;
}

// SwiGLU as the model builds it: silu(gate).mul(up) (src/peft.rs:584-588).
int orc_op_swiglu(const float* g, const float* u, size_t n, const float* gout, float* out, float* dg, float* du) {
  Tensor G = param(vec(g, n), {n}), U = param(vec(u, n), {n});
  Tensor Y = mul(silu(G), U);
  put(Y->data, out);
  if (gout) {
    backward_from(Y, gout);
    put(G->grad, dg);
    put(U->grad, du);
  }
  return 0;
}

int orc_op_softmax_rows(const float* x, size_t r, size_t c, const float* gout, float* out, float* dx) {
  Tensor X = param(vec(x, r * c), {r, c});
  Tensor Y = softmax_rows(X);
  put(Y->data, out);
  if (gout) {
    backward_from(Y, gout);
    put(X->grad, dx);
  }
  return 0;
}

// cross_entropy(...).scale(gscale): loss and dlogits for an upstream scalar gscale.
int orc_op_cross_entropy(const float* logits, size_t n, size_t vocab, const int32_t* targets, float gscale,
                         float* loss, float* dlogits) {
  Tensor L = param(vec(logits, n * vocab), {n, vocab});
  std::vector<size_t> tg(n);
  for (size_t i = 0; i < n; i++) tg[i] = (size_t)targets[i];
  Tensor Y = cross_entropy(L, tg);
  *loss = Y->data[0];
  if (dlogits) {
    backward_from(Y, &gscale);
    put(L->grad, dlogits);
  }
  return 0;
}

// Causal GQA attention exactly as PeftModel::forward composes it (src/peft.rs:479-489,
// 530-553): q [T, nh·hd], k/v [T, nkv·hd] (already roped) -> ctx [T, nh·hd].
int orc_op_attention(const float* q, const float* k, const float* v, size_t t, size_t nh, size_t nkv, size_t hd,
                     const float* gout, float* out, float* dq, float* dk, float* dv) {
  Tensor Q = param(vec(q, t * nh * hd), {t, nh * hd});
  Tensor K = param(vec(k, t * nkv * hd), {t, nkv * hd});
  Tensor V = param(vec(v, t * nkv * hd), {t, nkv * hd});
  size_t group = nh / nkv;
  float sc = 1.0f / std::sqrt((float)hd);
  std::vector<float> mk(nh * t * t, 0.0f);
  for (size_t h = 0; h < nh; h++)
    for (size_t i = 0; i < t; i++)
      for (size_t j = i + 1; j < t; j++) mk[(h * t + i) * t + j] = -1e9f;
  Tensor mask = constant(std::move(mk), {nh * t, t});
  Tensor qh = reshape(transpose12_4d(reshape(Q, {1, t, nh, hd})), {nh, t, hd});
  Tensor kh = repeat_interleave_dim0(reshape(transpose12_4d(reshape(K, {1, t, nkv, hd})), {nkv, t, hd}), group);
  Tensor vh = repeat_interleave_dim0(reshape(transpose12_4d(reshape(V, {1, t, nkv, hd})), {nkv, t, hd}), group);
  Tensor scores = scale(bmm(qh, transpose_last2(kh)), sc);
  Tensor att = reshape(softmax_rows(add(reshape(scores, {nh * t, t}), mask)), {nh, t, t});
  Tensor Y = reshape(transpose12_4d(reshape(bmm(att, vh), {1, nh, t, hd})), {t, nh * hd});
  put(Y->data, out);
  if (gout) {
    backward_from(Y, gout);
    put(Q->grad, dq);
    put(K->grad, dk);
    put(V->grad, dv);
  }
  return 0;
}

// One AdamW step on one parameter tensor with externally held state (src/tensor.rs:2952-2975).
int orc_adamw(float* p, const float* g, float* m, float* v, size_t n, uint64_t t, float lr, float wd, int decay) {
  Tensor P = param(vec(p, n), {n});
  P->grad = vec(g, n);
  AdamW opt({P}, lr, wd);
  opt.t = t - 1;
  opt.m[0] = vec(m, n);
  opt.v[0] = vec(v, n);
  opt.step({P}, {decay != 0});
  put(P->data, p);
  put(opt.m[0], m);
  put(opt.v[0], v);
  return 0;
}

// Tensor::randn (src/tensor.rs:241-256) for reference-faithful LoRA A init.
void orc_randn_uniform(size_t rows, size_t cols, uint64_t* seed, float* out) {
  Tensor t = randn_uniform({rows, cols}, seed);
  put(t->data, out);
}

// ---- tests/autograd.rs closures, evaluated for gradient checking ----
// shapes: ndims[i] dims each, packed into `dims`. Returns 0 and fills loss + grads.
int orc_case(const char* name, int n_in, const float** data, const int64_t* dims, const int* ndims, float* loss,
             float** grads) {
  std::vector<Tensor> t;
  size_t off = 0;
  for (int i = 0; i < n_in; i++) {
    std::vector<size_t> sh;
    for (int j = 0; j < ndims[i]; j++) sh.push_back((size_t)dims[off + j]);
    off += ndims[i];
    t.push_back(param(vec(data[i], numel(sh)), sh));
  }
  std::string n(name);
  Tensor y;
  if (n == "matmul") y = mean(matmul(t[0], t[1]));
  else if (n == "add_bias") y = mean(add(t[0], t[1]));
  else if (n == "mul") y = mean(mul(t[0], t[1]));
  else if (n == "sub") y = mean(sub(t[0], t[1]));
  else if (n == "relu") y = mean(relu(t[0]));
  else if (n == "silu") y = mean(silu(t[0]));
  else if (n == "square") y = mean(square(t[0]));
  else if (n == "scale") y = mean(scale(t[0], 2.5f));
  else if (n == "rmsnorm") y = mean(rmsnorm_eps(t[0], t[1], 1e-5f));
  else if (n == "softmax_rows") y = mean(square(softmax_rows(t[0])));
  else if (n == "cross_entropy") y = cross_entropy(t[0], {2, 0});
  else if (n == "embedding") y = mean(embedding(t[0], {2, 0, 2}));
  else if (n == "bmm") y = mean(bmm(t[0], t[1]));
  else if (n == "transpose_last2") y = mean(transpose_last2(t[0]));
  else if (n == "transpose12_4d") y = mean(transpose12_4d(t[0]));
  else if (n == "transpose") y = mean(square(transpose(t[0])));
  else if (n == "reshape") y = mean(square(reshape(t[0], {4, 1})));
  else if (n == "mlp") y = cross_entropy(matmul(relu(matmul(t[0], t[1])), t[2]), {1, 0});
  else if (n == "rope_interleaved") y = mean(square(rope(t[0], 2, 4, 10000.0f, false, {0, 1})));
  else if (n == "rope_neox") y = mean(square(rope(t[0], 2, 4, 10000.0f, true, {0, 1})));
  else if (n == "repeat_interleave") y = mean(square(repeat_interleave_dim0(t[0], 2)));
  else if (n == "sigmoid") y = mean(square(sigmoid(t[0])));
  else return ORC_E_INVALID;
  *loss = y->data[0];
  if (grads) {
    backward(y);
    for (int i = 0; i < n_in; i++) put(t[i]->grad, grads[i]);
  }
  return 0;
}

// ---- whole-model API ----

orc_model* orc_model_create(const orc_cfg* cfg) { return (orc_model*)model_create(cfg); }

int orc_model_set_tensor(orc_model* m, const char* name, const uint8_t* bytes, uint32_t type, size_t rows,
                         size_t cols) {
  return model_set_tensor((Model*)m, name, bytes, type, rows, cols);
}
float orc_model_loss_grad(orc_model* m, const int32_t* ids, const int32_t* tgts, int B, int T) {
  return model_loss_grad((Model*)m, ids, tgts, B, T);
}
void orc_model_adamw(orc_model* m, float lr, float wd) { model_adamw((Model*)m, lr, wd); }
int orc_model_logits(orc_model* m, const int32_t* ids, int T, float* out) {
  std::vector<size_t> id(T);
  for (int i = 0; i < T; i++) id[i] = (size_t)ids[i];
  Tensor y = model_forward((Model*)m, id, nullptr);
  put(y->data, out);
  return 0;
}

}  // extern "C"
