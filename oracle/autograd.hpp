// ORACLE — test infrastructure only. CPU restatement of HOS's tensor autograd core,
// src/tensor.rs. Same loop nests, same summation order, no FMA contraction
// (-ffp-contract=off), glibc expf/logf/powf/sinf/cosf/sqrtf as Rust's f32 methods
// call on Linux. OpenMP splits only loops whose iterations write disjoint outputs, each
// output keeping its serial summation order, so results are identical to one thread.
#pragma once
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <functional>
#include <memory>
#include <unordered_set>
#include <vector>

namespace orc {

struct Node;
using Tensor = std::shared_ptr<Node>;
using BackFn = std::function<void(const std::vector<float>&, const std::vector<Tensor>&)>;

// src/tensor.rs:180-195 (Inner): data, shape, grad, requires_grad, parents, backward.
struct Node {
  std::vector<float> data;
  std::vector<size_t> shape;
  std::vector<float> grad;
  bool requires_grad = false;
  std::vector<Tensor> parents;
  BackFn backward;

  void add_grad(const std::vector<float>& g) {  // src/tensor.rs:281-286
    for (size_t i = 0; i < g.size(); i++) grad[i] += g[i];
  }
};

inline size_t numel(const std::vector<size_t>& s) {
  size_t n = 1;
  for (size_t v : s) n *= v;
  return n;
}

// src/tensor.rs:217-230 (Tensor::new / param / constant)
inline Tensor tnew(std::vector<float> data, std::vector<size_t> shape, bool req) {
  auto t = std::make_shared<Node>();
  t->grad.assign(data.size(), 0.0f);
  t->data = std::move(data);
  t->shape = std::move(shape);
  t->requires_grad = req;
  return t;
}
inline Tensor param(std::vector<float> d, std::vector<size_t> s) { return tnew(std::move(d), std::move(s), true); }
inline Tensor constant(std::vector<float> d, std::vector<size_t> s) { return tnew(std::move(d), std::move(s), false); }

// src/tensor.rs:287-303 (Tensor::build): parents/backward only when any parent requires grad.
inline Tensor build(std::vector<float> data, std::vector<size_t> shape, std::vector<Tensor> parents, BackFn bw) {
  bool req = false;
  for (auto& p : parents) req = req || p->requires_grad;
  auto out = tnew(std::move(data), std::move(shape), req);
  if (req) {
    out->parents = std::move(parents);
    out->backward = std::move(bw);
  }
  return out;
}

// src/tensor.rs:241-256 (Tensor::randn): xorshift64, UNIFORM in ±sqrt(1/fan).
inline Tensor randn_uniform(std::vector<size_t> shape, uint64_t* seed) {
  size_t n = numel(shape);
  float fan = shape.empty() ? 1.0f : (float)shape.back();
  float scale = std::sqrt(1.0f / fan);
  std::vector<float> d(n);
  for (size_t i = 0; i < n; i++) {
    uint64_t x = *seed;
    x ^= x << 13;
    x ^= x >> 7;
    x ^= x << 17;
    *seed = x;
    d[i] = ((float)(x >> 40) / (float)(1ull << 24) * 2.0f - 1.0f) * scale;
  }
  return param(std::move(d), std::move(shape));
}

// ---- ops ----

// C[i][c] += Σ_s A[i][s]·B[s][c] with, for every element, the terms added one at a time in ascending s (one f32
// rounding per product and per add, no fused multiply-add): exactly the arithmetic of the reference's scalar loops
// (src/tensor.rs:307-391), whatever order the elements themselves are visited in. The loops are tiled (row and
// column blocks, chunks of s that carry each element's running sum through C) and the inner 4-row × 16-column
// block keeps its running sums in SSE registers; none of this changes an element's sequence of roundings.
typedef float orc_v4 __attribute__((vector_size(16)));
#ifndef ORC_R
#define ORC_R 4  // rows of the register block
#endif
#ifndef ORC_Q
#define ORC_Q 2  // 4-float vectors of the register block (8 running sums + 2 B vectors + 1 broadcast in 16 xmm)
#endif
inline void ordered_gemm(const float* A, size_t lda, const float* B, size_t ldb, float* C, size_t ldc, size_t M,
                         size_t S, size_t N) {
  const size_t MB = 32, NB = 128, SB = 256;
  const long long nib = (long long)((M + MB - 1) / MB), njb = (long long)((N + NB - 1) / NB);
#pragma omp parallel for schedule(dynamic)
  for (long long t = 0; t < nib * njb; t++) {
    const size_t i0 = (size_t)(t / njb) * MB, c0 = (size_t)(t % njb) * NB;
    const size_t i1 = std::min(M, i0 + MB), c1 = std::min(N, c0 + NB);
    for (size_t s0 = 0; s0 < S; s0 += SB) {
      const size_t s1 = std::min(S, s0 + SB);
      size_t i = i0;
      for (; i + ORC_R <= i1; i += ORC_R) {
        size_t c = c0;
        for (; c + 4 * ORC_Q <= c1; c += 4 * ORC_Q) {
          orc_v4 acc[ORC_R][ORC_Q];
          for (int r = 0; r < ORC_R; r++)
            for (int q = 0; q < ORC_Q; q++) std::memcpy(&acc[r][q], &C[(i + r) * ldc + c + 4 * q], 16);
          for (size_t sv = s0; sv < s1; sv++) {
            orc_v4 bv[ORC_Q];
            for (int q = 0; q < ORC_Q; q++) std::memcpy(&bv[q], &B[sv * ldb + c + 4 * q], 16);
            for (int r = 0; r < ORC_R; r++) {
              const float a = A[(i + r) * lda + sv];
              const orc_v4 av = {a, a, a, a};
              for (int q = 0; q < ORC_Q; q++) acc[r][q] = acc[r][q] + av * bv[q];
            }
          }
          for (int r = 0; r < ORC_R; r++)
            for (int q = 0; q < ORC_Q; q++) std::memcpy(&C[(i + r) * ldc + c + 4 * q], &acc[r][q], 16);
        }
        for (; c < c1; c++)
          for (int r = 0; r < ORC_R; r++) {
            float acc = C[(i + r) * ldc + c];
            for (size_t sv = s0; sv < s1; sv++) acc += A[(i + r) * lda + sv] * B[sv * ldb + c];
            C[(i + r) * ldc + c] = acc;
          }
      }
      for (; i < i1; i++)
        for (size_t c = c0; c < c1; c++) {
          float acc = C[i * ldc + c];
          for (size_t sv = s0; sv < s1; sv++) acc += A[i * lda + sv] * B[sv * ldb + c];
          C[i * ldc + c] = acc;
        }
    }
  }
}

// dst[c][r] = src[r][c] for src [R, Cn] (blocked for cache locality).
inline std::vector<float> transpose_copy(const float* src, size_t R, size_t Cn) {
  std::vector<float> dst(R * Cn);
  const size_t TB = 64;
#pragma omp parallel for schedule(static)
  for (long long r0 = 0; r0 < (long long)R; r0 += TB)
    for (size_t c0 = 0; c0 < Cn; c0 += TB)
      for (size_t r = (size_t)r0; r < std::min(R, (size_t)r0 + TB); r++)
        for (size_t c = c0; c < std::min(Cn, c0 + TB); c++) dst[c * R + r] = src[r * Cn + c];
  return dst;
}

// src/tensor.rs:307-391: fwd i-p-j; dA = g·Bᵀ (i-j-p); dB = Aᵀ·g (i-p-j); frozen B skips dB.
inline Tensor matmul(const Tensor& A, const Tensor& B) {
  size_t m = A->shape[0], k = A->shape[1], n = B->shape[1];
  std::vector<float> out(m * n, 0.0f);
  const float* a = A->data.data();
  const float* b = B->data.data();
  ordered_gemm(a, k, b, n, out.data(), n, m, k, n);  // out[i][j]: Σ over p ascending (the i-p-j loop)
  return build(std::move(out), {m, n}, {A, B}, [m, k, n](const std::vector<float>& g, const std::vector<Tensor>& par) {
    bool need_a = par[0]->requires_grad, need_b = par[1]->requires_grad;
    const float* a = par[0]->data.data();
    const float* b = par[1]->data.data();
    if (need_a) {
      std::vector<float> da(m * k, 0.0f);
      // da[i][p]: Σ over j ascending of g[i][j]·b[p][j] (the i-j-p loop), as a GEMM against Bᵀ
      const std::vector<float> bt = transpose_copy(b, k, n);
      ordered_gemm(g.data(), n, bt.data(), k, da.data(), k, m, n, k);
      par[0]->add_grad(da);
    }
    if (need_b) {
      std::vector<float> db(k * n, 0.0f);
      // db[p][j]: Σ over i ascending of a[i][p]·g[i][j] (the i-p-j loop), as a GEMM of Aᵀ
      const std::vector<float> at = transpose_copy(a, m, k);
      ordered_gemm(at.data(), m, g.data(), n, db.data(), n, k, m, n);
      par[1]->add_grad(db);
    }
  });
}

// src/tensor.rs:394-436: elementwise add, or row-broadcast of a 1-D bias.
inline Tensor add(const Tensor& A, const Tensor& B) {
  bool broadcast = B->shape.size() == 1 && A->shape.size() == 2 && B->shape[0] == A->shape[1];
  size_t m = broadcast ? A->shape[0] : A->data.size();
  size_t f = broadcast ? A->shape[1] : 1;
  std::vector<float> out = A->data;
  if (broadcast) {
    for (size_t i = 0; i < m; i++)
      for (size_t j = 0; j < f; j++) out[i * f + j] += B->data[j];
  } else {
    for (size_t i = 0; i < out.size(); i++) out[i] += B->data[i];
  }
  return build(std::move(out), A->shape, {A, B}, [broadcast, m, f](const std::vector<float>& g, const std::vector<Tensor>& par) {
    par[0]->add_grad(g);
    if (broadcast) {
      std::vector<float> db(f, 0.0f);
      for (size_t i = 0; i < m; i++)
        for (size_t j = 0; j < f; j++) db[j] += g[i * f + j];
      par[1]->add_grad(db);
    } else {
      par[1]->add_grad(g);
    }
  });
}

// src/tensor.rs:438-455
inline Tensor sub(const Tensor& A, const Tensor& B) {
  std::vector<float> out(A->data.size());
  for (size_t i = 0; i < out.size(); i++) out[i] = A->data[i] - B->data[i];
  return build(std::move(out), A->shape, {A, B}, [](const std::vector<float>& g, const std::vector<Tensor>& par) {
    par[0]->add_grad(g);
    std::vector<float> neg(g.size());
    for (size_t i = 0; i < g.size(); i++) neg[i] = -g[i];
    par[1]->add_grad(neg);
  });
}

// src/tensor.rs:458-480
inline Tensor mul(const Tensor& A, const Tensor& B) {
  std::vector<float> out(A->data.size());
  for (size_t i = 0; i < out.size(); i++) out[i] = A->data[i] * B->data[i];
  return build(std::move(out), A->shape, {A, B}, [](const std::vector<float>& g, const std::vector<Tensor>& par) {
    const auto& a = par[0]->data;
    const auto& b = par[1]->data;
    std::vector<float> ga(g.size()), gb(g.size());
    for (size_t i = 0; i < g.size(); i++) ga[i] = g[i] * b[i];
    for (size_t i = 0; i < g.size(); i++) gb[i] = g[i] * a[i];
    par[0]->add_grad(ga);
    par[1]->add_grad(gb);
  });
}

// src/tensor.rs:2082-2100: silu(x) = x / (1 + exp(-x)); d = s + x·s·(1−s).
inline Tensor silu(const Tensor& A) {
  std::vector<float> out(A->data.size());
  for (size_t i = 0; i < out.size(); i++) {
    float x = A->data[i];
    out[i] = x / (1.0f + std::exp(-x));
  }
  return build(std::move(out), A->shape, {A}, [](const std::vector<float>& g, const std::vector<Tensor>& par) {
    const auto& a = par[0]->data;
    std::vector<float> ga(g.size());
    for (size_t i = 0; i < g.size(); i++) {
      float x = a[i];
      float s = 1.0f / (1.0f + std::exp(-x));
      ga[i] = g[i] * (s + x * s * (1.0f - s));
    }
    par[0]->add_grad(ga);
  });
}

// src/tensor.rs:2064-2079 (relu)
inline Tensor relu(const Tensor& A) {
  std::vector<float> out(A->data.size());
  for (size_t i = 0; i < out.size(); i++) out[i] = A->data[i] > 0.0f ? A->data[i] : 0.0f;
  return build(std::move(out), A->shape, {A}, [](const std::vector<float>& g, const std::vector<Tensor>& par) {
    const auto& a = par[0]->data;
    std::vector<float> ga(g.size());
    for (size_t i = 0; i < g.size(); i++) ga[i] = a[i] > 0.0f ? g[i] : 0.0f;
    par[0]->add_grad(ga);
  });
}

// src/tensor.rs:2103-2117 (sigmoid)
inline Tensor sigmoid(const Tensor& A) {
  std::vector<float> out(A->data.size());
  for (size_t i = 0; i < out.size(); i++) out[i] = 1.0f / (1.0f + std::exp(-A->data[i]));
  std::vector<float> saved = out;
  return build(std::move(out), A->shape, {A}, [saved](const std::vector<float>& g, const std::vector<Tensor>& par) {
    std::vector<float> dx(g.size());
    for (size_t i = 0; i < g.size(); i++) dx[i] = g[i] * saved[i] * (1.0f - saved[i]);
    par[0]->add_grad(dx);
  });
}

// src/tensor.rs:2120-2129: sequential f32 sum / n.
inline Tensor mean(const Tensor& A) {
  size_t n = A->data.size();
  float s = 0.0f;
  for (size_t i = 0; i < n; i++) s += A->data[i];
  s = s / (float)n;
  return build({s}, {1}, {A}, [n](const std::vector<float>& g, const std::vector<Tensor>& par) {
    float sc = g[0] / (float)n;
    par[0]->add_grad(std::vector<float>(n, sc));
  });
}

inline Tensor square(const Tensor& A) { return mul(A, A); }  // src/tensor.rs:2131-2133

// src/tensor.rs:2387-2399: column j of a [n, c] matrix as [n, 1]; bwd scatters into that column.
inline Tensor col(const Tensor& A, size_t j) {
  const size_t n = A->shape[0], c = A->shape[1];
  std::vector<float> out(n);
  for (size_t i = 0; i < n; i++) out[i] = A->data[i * c + j];
  return build(std::move(out), {n, 1}, {A}, [n, c, j](const std::vector<float>& g, const std::vector<Tensor>& par) {
    std::vector<float> gi(n * c, 0.0f);
    for (size_t i = 0; i < n; i++) gi[i * c + j] = g[i];
    par[0]->add_grad(gi);
  });
}

// src/tensor.rs:2402-2436: a[n, c] * b[n, 1] row-broadcast; db[i] = Σ_j g[i, j]·a[i, j] in j order.
inline Tensor mul_broadcast(const Tensor& A, const Tensor& B) {
  const size_t n = A->shape[0], c = A->shape[1];
  std::vector<float> out(n * c);
  for (size_t i = 0; i < n; i++)
    for (size_t j = 0; j < c; j++) out[i * c + j] = A->data[i * c + j] * B->data[i];
  return build(std::move(out), {n, c}, {A, B}, [n, c](const std::vector<float>& g, const std::vector<Tensor>& par) {
    const auto& a = par[0]->data;
    const auto& b = par[1]->data;
    std::vector<float> da(n * c), db(n, 0.0f);
    for (size_t i = 0; i < n; i++)
      for (size_t j = 0; j < c; j++) {
        da[i * c + j] = g[i * c + j] * b[i];
        db[i] += g[i * c + j] * a[i * c + j];
      }
    par[0]->add_grad(da);
    par[1]->add_grad(db);
  });
}

// src/tensor.rs:2136-2145
inline Tensor scale(const Tensor& A, float c) {
  std::vector<float> out(A->data.size());
  for (size_t i = 0; i < out.size(); i++) out[i] = A->data[i] * c;
  return build(std::move(out), A->shape, {A}, [c](const std::vector<float>& g, const std::vector<Tensor>& par) {
    std::vector<float> gg(g.size());
    for (size_t i = 0; i < g.size(); i++) gg[i] = g[i] * c;
    par[0]->add_grad(gg);
  });
}

// src/tensor.rs:2148-2167 (2-D transpose)
inline Tensor transpose(const Tensor& A) {
  size_t m = A->shape[0], n = A->shape[1];
  std::vector<float> out(m * n);
  for (size_t i = 0; i < m; i++)
    for (size_t j = 0; j < n; j++) out[j * m + i] = A->data[i * n + j];
  return build(std::move(out), {n, m}, {A}, [m, n](const std::vector<float>& g, const std::vector<Tensor>& par) {
    std::vector<float> gi(m * n);
    for (size_t i = 0; i < m; i++)
      for (size_t j = 0; j < n; j++) gi[i * n + j] = g[j * m + i];
    par[0]->add_grad(gi);
  });
}

// src/tensor.rs:2170-2178 (reshape clones data; identity grad)
inline Tensor reshape(const Tensor& A, std::vector<size_t> shape) {
  return build(A->data, std::move(shape), {A}, [](const std::vector<float>& g, const std::vector<Tensor>& par) {
    par[0]->add_grad(g);
  });
}

// src/tensor.rs:2181-2204: [b,m,n] -> [b,n,m]
inline Tensor transpose_last2(const Tensor& A) {
  size_t bs = A->shape[0], m = A->shape[1], n = A->shape[2];
  std::vector<float> out(bs * m * n);
  for (size_t bi = 0; bi < bs; bi++)
    for (size_t i = 0; i < m; i++)
      for (size_t j = 0; j < n; j++) out[bi * n * m + j * m + i] = A->data[bi * m * n + i * n + j];
  return build(std::move(out), {bs, n, m}, {A}, [bs, m, n](const std::vector<float>& g, const std::vector<Tensor>& par) {
    std::vector<float> gi(bs * m * n);
    for (size_t bi = 0; bi < bs; bi++)
      for (size_t i = 0; i < m; i++)
        for (size_t j = 0; j < n; j++) gi[bi * m * n + i * n + j] = g[bi * n * m + j * m + i];
    par[0]->add_grad(gi);
  });
}

// src/tensor.rs:2207-2280 (CPU branch): batched i-p-j; bwd accumulates dA and dB in one
// i-p-j nest per batch.
inline Tensor bmm(const Tensor& A, const Tensor& B) {
  size_t bs = A->shape[0], m = A->shape[1], k = A->shape[2], n = B->shape[2];
  std::vector<float> out(bs * m * n, 0.0f);
  const float* a = A->data.data();
  const float* b = B->data.data();
#pragma omp parallel for schedule(static)
  for (long long bi = 0; bi < (long long)bs; bi++) {
    size_t ao = bi * m * k, bo = bi * k * n, oo = bi * m * n;
    for (size_t i = 0; i < m; i++)
      for (size_t p = 0; p < k; p++) {
        float av = a[ao + i * k + p];
        for (size_t j = 0; j < n; j++) out[oo + i * n + j] += av * b[bo + p * n + j];
      }
  }
  return build(std::move(out), {bs, m, n}, {A, B}, [bs, m, k, n](const std::vector<float>& g, const std::vector<Tensor>& par) {
    const float* a = par[0]->data.data();
    const float* b = par[1]->data.data();
    std::vector<float> da(bs * m * k, 0.0f), db(bs * k * n, 0.0f);
#pragma omp parallel for schedule(static)
    for (long long bi = 0; bi < (long long)bs; bi++) {
      size_t ao = bi * m * k, bo = bi * k * n, oo = bi * m * n;
      for (size_t i = 0; i < m; i++)
        for (size_t p = 0; p < k; p++)
          for (size_t j = 0; j < n; j++) {
            da[ao + i * k + p] += g[oo + i * n + j] * b[bo + p * n + j];
            db[bo + p * n + j] += a[ao + i * k + p] * g[oo + i * n + j];
          }
    }
    par[0]->add_grad(da);
    par[1]->add_grad(db);
  });
}

// src/tensor.rs:2283-2312: [a,b,c,e] -> [a,c,b,e]
inline Tensor transpose12_4d(const Tensor& A) {
  size_t d0 = A->shape[0], d1 = A->shape[1], d2 = A->shape[2], d3 = A->shape[3];
  std::vector<float> out(d0 * d1 * d2 * d3);
  for (size_t i = 0; i < d0; i++)
    for (size_t j = 0; j < d1; j++)
      for (size_t k = 0; k < d2; k++)
        for (size_t l = 0; l < d3; l++) out[((i * d2 + k) * d1 + j) * d3 + l] = A->data[((i * d1 + j) * d2 + k) * d3 + l];
  return build(std::move(out), {d0, d2, d1, d3}, {A}, [d0, d1, d2, d3](const std::vector<float>& g, const std::vector<Tensor>& par) {
    std::vector<float> gi(d0 * d1 * d2 * d3);
    for (size_t i = 0; i < d0; i++)
      for (size_t j = 0; j < d1; j++)
        for (size_t k = 0; k < d2; k++)
          for (size_t l = 0; l < d3; l++) gi[((i * d1 + j) * d2 + k) * d3 + l] = g[((i * d2 + k) * d1 + j) * d3 + l];
    par[0]->add_grad(gi);
  });
}

// src/tensor.rs:2438-2457
inline Tensor embedding(const Tensor& table, const std::vector<size_t>& ids) {
  size_t d = table->shape[1], vocab = table->shape[0];
  std::vector<float> out(ids.size() * d);
  for (size_t i = 0; i < ids.size(); i++) std::memcpy(&out[i * d], &table->data[ids[i] * d], d * 4);
  return build(std::move(out), {ids.size(), d}, {table}, [ids, vocab, d](const std::vector<float>& g, const std::vector<Tensor>& par) {
    std::vector<float> gw(vocab * d, 0.0f);
    for (size_t i = 0; i < ids.size(); i++)
      for (size_t j = 0; j < d; j++) gw[ids[i] * d + j] += g[i * d + j];
    par[0]->add_grad(gw);
  });
}

// src/tensor.rs:2460-2491
inline Tensor softmax_rows(const Tensor& A) {
  size_t r = A->shape[0], c = A->shape[1];
  std::vector<float> out(r * c);
#pragma omp parallel for schedule(static)
  for (long long i = 0; i < (long long)r; i++) {
    const float* row = &A->data[i * c];
    float mx = -INFINITY;
    for (size_t j = 0; j < c; j++) mx = std::fmax(mx, row[j]);
    float sum = 0.0f;
    for (size_t j = 0; j < c; j++) {
      float e = std::exp(row[j] - mx);
      out[i * c + j] = e;
      sum += e;
    }
    for (size_t j = 0; j < c; j++) out[i * c + j] /= sum;
  }
  std::vector<float> probs = out;
  return build(std::move(out), {r, c}, {A}, [probs, r, c](const std::vector<float>& g, const std::vector<Tensor>& par) {
    std::vector<float> gi(r * c);
#pragma omp parallel for schedule(static)
    for (long long i = 0; i < (long long)r; i++) {
      const float* s = &probs[i * c];
      const float* go = &g[i * c];
      float dot = 0.0f;
      for (size_t j = 0; j < c; j++) dot += go[j] * s[j];
      for (size_t j = 0; j < c; j++) gi[i * c + j] = s[j] * (go[j] - dot);
    }
    par[0]->add_grad(gi);
  });
}

// Rows of X in the order `rows` gives (a row may repeat); backward scatter-adds into the source rows.
// Used by the mixture-of-experts FFN to run each expert only on the tokens routed to it.
inline Tensor gather_rows(const Tensor& X, const std::vector<size_t>& rows) {
  size_t d = X->shape[1], n = rows.size();
  std::vector<float> out(n * d);
  for (size_t i = 0; i < n; i++) std::memcpy(&out[i * d], &X->data[rows[i] * d], d * sizeof(float));
  return build(std::move(out), {n, d}, {X}, [rows, d](const std::vector<float>& g, const std::vector<Tensor>& par) {
    std::vector<float> gx(par[0]->data.size(), 0.0f);
    for (size_t i = 0; i < rows.size(); i++)
      for (size_t j = 0; j < d; j++) gx[rows[i] * d + j] += g[i * d + j];
    par[0]->add_grad(gx);
  });
}

// Mixture-of-experts combine, src/forward.rs:542-572: for each token t, over its selected experts in
// selection order (descending probability), ffn[t] += p[t, e]·y_e[row of t]; the probabilities are the raw
// softmax values (no renormalisation, OLMoE's norm_topk_prob = false). ys[e] holds expert e's outputs for
// the tokens routed to it (null when none); sel[t][s] = (expert, row in ys[e]). Backward: dy_e[row] =
// p[t, e]·g[t]; dp[t, e] = y_e[row]·g[t] for the selected experts (0 for the others).
inline Tensor moe_mix(const std::vector<Tensor>& ys, const Tensor& P,
                      const std::vector<std::vector<std::pair<size_t, size_t>>>& sel, size_t d) {
  size_t T = sel.size(), E = P->shape[1];
  std::vector<float> out(T * d, 0.0f);
  for (size_t t = 0; t < T; t++)
    for (auto [e, row] : sel[t]) {
      const float w = P->data[t * E + e];
      const float* y = &ys[e]->data[row * d];
      for (size_t j = 0; j < d; j++) out[t * d + j] += w * y[j];
    }
  std::vector<Tensor> parents{P};
  std::vector<int> slot(E, -1);
  for (size_t e = 0; e < E; e++)
    if (ys[e]) {
      slot[e] = (int)parents.size();
      parents.push_back(ys[e]);
    }
  return build(std::move(out), {T, d}, parents,
               [sel, slot, T, E, d](const std::vector<float>& g, const std::vector<Tensor>& par) {
                 const Tensor& Pt = par[0];
                 std::vector<float> gp(T * E, 0.0f);
                 std::vector<std::vector<float>> gy(par.size());
                 for (size_t i = 1; i < par.size(); i++) gy[i].assign(par[i]->data.size(), 0.0f);
                 for (size_t t = 0; t < T; t++)
                   for (auto [e, row] : sel[t]) {
                     const int k = slot[e];
                     const float w = Pt->data[t * E + e];
                     const float* y = &par[k]->data[row * d];
                     float dp = 0.0f;
                     for (size_t j = 0; j < d; j++) {
                       gy[k][row * d + j] += w * g[t * d + j];
                       dp += y[j] * g[t * d + j];
                     }
                     gp[t * E + e] = dp;
                   }
                 Pt->add_grad(gp);
                 for (size_t i = 1; i < par.size(); i++)
                   if (par[i]->requires_grad) par[i]->add_grad(gy[i]);
               });
}

// src/tensor.rs:2500-2544: y = x·inv·w, inv = 1/sqrt(mean(x²)+eps).
inline Tensor rmsnorm_eps(const Tensor& X, const Tensor& W, float eps) {
  size_t r = X->shape[0], d = X->shape[1];
  std::vector<float> out(r * d), invs(r);
  const float* w = W->data.data();
#pragma omp parallel for schedule(static)
  for (long long i = 0; i < (long long)r; i++) {
    const float* row = &X->data[i * d];
    float ss = 0.0f;
    for (size_t j = 0; j < d; j++) ss += row[j] * row[j];
    ss = ss / (float)d;
    float inv = 1.0f / std::sqrt(ss + eps);
    invs[i] = inv;
    for (size_t j = 0; j < d; j++) out[i * d + j] = row[j] * inv * w[j];
  }
  return build(std::move(out), {r, d}, {X, W}, [invs, r, d](const std::vector<float>& g, const std::vector<Tensor>& par) {
    const float* w = par[1]->data.data();
    const float* xa = par[0]->data.data();
    std::vector<float> gx(r * d), gw(d, 0.0f);
#pragma omp parallel for schedule(static)
    for (long long i = 0; i < (long long)r; i++) {
      const float* x = xa + i * d;
      float inv = invs[i];
      const float* go = &g[i * d];
      float sgwx = 0.0f;
      for (size_t j = 0; j < d; j++) sgwx += go[j] * w[j] * x[j];
      for (size_t j = 0; j < d; j++) gx[i * d + j] = go[j] * w[j] * inv - inv * inv * inv * x[j] / (float)d * sgwx;
    }
    for (size_t i = 0; i < r; i++)
      for (size_t j = 0; j < d; j++) gw[j] += g[i * d + j] * xa[i * d + j] * invs[i];
    par[0]->add_grad(gx);
    par[1]->add_grad(gw);
  });
}

// src/tensor.rs:2709-2743: per-row softmax, loss = mean(−ln max(p_t, 1e−12)); bwd (p − 1hot)·g/n.
inline Tensor cross_entropy(const Tensor& L, const std::vector<size_t>& targets) {
  size_t n = L->shape[0], vocab = L->shape[1];
  std::vector<float> probs(n * vocab), terms(n);
#pragma omp parallel for schedule(static)
  for (long long i = 0; i < (long long)n; i++) {
    const float* row = &L->data[i * vocab];
    float mx = -INFINITY;
    for (size_t j = 0; j < vocab; j++) mx = std::fmax(mx, row[j]);
    float sum = 0.0f;
    for (size_t j = 0; j < vocab; j++) {
      float e = std::exp(row[j] - mx);
      probs[i * vocab + j] = e;
      sum += e;
    }
    for (size_t j = 0; j < vocab; j++) probs[i * vocab + j] /= sum;
    terms[i] = -std::log(std::fmax(probs[i * vocab + targets[i]], 1e-12f));
  }
  float loss = 0.0f;
  for (size_t i = 0; i < n; i++) loss += terms[i];  // serial, in row order
  loss /= (float)n;
  auto pr = std::make_shared<std::vector<float>>(std::move(probs));
  return build({loss}, {1}, {L}, [pr, targets, n, vocab](const std::vector<float>& g, const std::vector<Tensor>& par) {
    std::vector<float> gi = *pr;
    for (size_t i = 0; i < n; i++) gi[i * vocab + targets[i]] -= 1.0f;
    float sc = g[0] / (float)n;
#pragma omp parallel for schedule(static)
    for (long long i = 0; i < (long long)gi.size(); i++) gi[i] *= sc;
    par[0]->add_grad(gi);
  });
}

// src/tensor.rs:2750-2814: freq = 1/base^(2i/hd) (powf), (sin,cos)(pos·freq); bwd = Rᵀ.
inline Tensor rope(const Tensor& A, size_t n_heads, size_t head_dim, float base, bool neox, const std::vector<size_t>& pos) {
  size_t rows = A->shape[0], width = A->shape[1], half = head_dim / 2;
  auto sc = std::make_shared<std::vector<float>>(rows * half * 2);
  for (size_t r = 0; r < rows; r++)
    for (size_t i = 0; i < half; i++) {
      float freq = 1.0f / std::pow(base, 2.0f * (float)i / (float)head_dim);
      float ang = (float)pos[r] * freq;
      (*sc)[(r * half + i) * 2] = std::sin(ang);
      (*sc)[(r * half + i) * 2 + 1] = std::cos(ang);
    }
  std::vector<float> out = A->data;
  for (size_t r = 0; r < rows; r++)
    for (size_t h = 0; h < n_heads; h++) {
      size_t off = r * width + h * head_dim;
      for (size_t i = 0; i < half; i++) {
        float s = (*sc)[(r * half + i) * 2], c = (*sc)[(r * half + i) * 2 + 1];
        size_t ia = neox ? i : 2 * i, ib = neox ? i + half : 2 * i + 1;
        float xa = out[off + ia], xb = out[off + ib];
        out[off + ia] = xa * c - xb * s;
        out[off + ib] = xa * s + xb * c;
      }
    }
  return build(std::move(out), {rows, width}, {A}, [sc, rows, n_heads, head_dim, half, width, neox](const std::vector<float>& g, const std::vector<Tensor>& par) {
    std::vector<float> dx(g.size(), 0.0f);
    for (size_t r = 0; r < rows; r++)
      for (size_t h = 0; h < n_heads; h++) {
        size_t off = r * width + h * head_dim;
        for (size_t i = 0; i < half; i++) {
          float s = (*sc)[(r * half + i) * 2], c = (*sc)[(r * half + i) * 2 + 1];
          size_t ia = neox ? i : 2 * i, ib = neox ? i + half : 2 * i + 1;
          float ga = g[off + ia], gb = g[off + ib];
          dx[off + ia] = ga * c + gb * s;
          dx[off + ib] = -ga * s + gb * c;
        }
      }
    par[0]->add_grad(dx);
  });
}

// src/tensor.rs:2819-2841
inline Tensor repeat_interleave_dim0(const Tensor& A, size_t g) {
  size_t d0 = A->shape[0];
  size_t block = 1;
  for (size_t i = 1; i < A->shape.size(); i++) block *= A->shape[i];
  std::vector<float> out(d0 * g * block);
  for (size_t i = 0; i < d0 * g; i++) std::memcpy(&out[i * block], &A->data[(i / g) * block], block * 4);
  std::vector<size_t> ns = A->shape;
  ns[0] = d0 * g;
  return build(std::move(out), ns, {A}, [d0, g, block](const std::vector<float>& grad, const std::vector<Tensor>& par) {
    std::vector<float> din(d0 * block, 0.0f);
    for (size_t i = 0; i < d0 * g; i++) {
      size_t dst = (i / g) * block;
      for (size_t j = 0; j < block; j++) din[dst + j] += grad[i * block + j];
    }
    par[0]->add_grad(din);
  });
}

// src/tensor.rs:2844-2881: DFS topological order, seed 1, reverse VJPs.
inline void backward(const Tensor& root) {
  std::vector<Tensor> topo;
  std::unordered_set<const Node*> visited;
  std::function<void(const Tensor&)> dfs = [&](const Tensor& t) {
    if (visited.count(t.get())) return;
    visited.insert(t.get());
    for (auto& p : t->parents) dfs(p);
    topo.push_back(t);
  };
  dfs(root);
  for (auto& g : root->grad) g = 1.0f;
  for (auto it = topo.rbegin(); it != topo.rend(); ++it) {
    const Tensor& node = *it;
    if (node->backward) {
      std::vector<float> grad = node->grad;
      node->backward(grad, node->parents);
    }
  }
}

inline void zero_grad(const Tensor& t) { std::fill(t->grad.begin(), t->grad.end(), 0.0f); }  // :2883-2888

// compiler-rt __powisf2 (what Rust's f32::powi lowers to): square-and-multiply.
inline float powi_f32(float a, int b) {
  bool recip = b < 0;
  float r = 1.0f;
  while (true) {
    if (b & 1) r *= a;
    b /= 2;
    if (b == 0) break;
    a *= a;
  }
  return recip ? 1.0f / r : r;
}

// src/tensor.rs:2923-2976 (AdamW): β1 .9, β2 .95, eps 1e-8, decoupled decay.
struct AdamW {
  float lr, beta1 = 0.9f, beta2 = 0.95f, eps = 1e-8f, wd;
  uint64_t t = 0;
  std::vector<std::vector<float>> m, v;
  AdamW(const std::vector<Tensor>& params, float lr_, float wd_) : lr(lr_), wd(wd_) {
    for (auto& p : params) {
      m.emplace_back(p->data.size(), 0.0f);
      v.emplace_back(p->data.size(), 0.0f);
    }
  }
  void step(const std::vector<Tensor>& params, const std::vector<bool>& decay) {
    t += 1;
    float bc1 = 1.0f - powi_f32(beta1, (int)t);
    float bc2 = 1.0f - powi_f32(beta2, (int)t);
    for (size_t i = 0; i < params.size(); i++) {
      const auto& g = params[i]->grad;
      auto& data = params[i]->data;
      auto& mi = m[i];
      auto& vi = v[i];
      for (size_t j = 0; j < g.size(); j++) {
        mi[j] = beta1 * mi[j] + (1.0f - beta1) * g[j];
        vi[j] = beta2 * vi[j] + (1.0f - beta2) * g[j] * g[j];
        float mh = mi[j] / bc1;
        float vh = vi[j] / bc2;
        float u = lr * mh / (std::sqrt(vh) + eps);
        if (decay[i]) u += lr * wd * data[j];
        data[j] -= u;  // step_raw, src/tensor.rs:2896-2905
      }
    }
  }
};

}  // namespace orc
