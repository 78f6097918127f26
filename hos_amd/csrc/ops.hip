// Op-level C ABI: one entry point per fused kernel of the training path, on device pointers, enqueued on
// the context's stream (hos_hip_synchronize waits). These are the reference's autograd ops
// (src/tensor.rs) with their VJPs, so each can be checked against the CPU path on its own, as the
// reference's tests/autograd.rs checks the ops; the training step (peft.hip) schedules the same kernels.
#include <algorithm>
#include <cmath>
#include <mutex>
#include <string>
#include <vector>

#include "ctx.hpp"
#include "fused.hpp"
#include "lora.hpp"
#include "moe.hpp"

using namespace hos;

// Scratch of hos_hip_lora_noalloc (64 MiB, one copy per GPU); host code uses only the per-device address
// lora_scratch_ptr() looks up.
constexpr size_t kLoraScratch = 64ull << 20;
static __device__ __align__(256) char scratch[kLoraScratch];

namespace {

template <class F>
int op_guard(hos_ctx* c, F&& f) {
  if (!c) return HOS_E_INVALID;
  try {
    HOS_HIP_CHECK(hipSetDevice(hos_internal_device(c)));
    f(hos_internal_stream(c));
    internal_set_error(c, "");
    return HOS_OK;
  } catch (const Error& e) {
    internal_set_error(c, e.what());
    return e.code;
  } catch (const std::bad_alloc&) {
    internal_set_error(c, "host allocation failed");
    return HOS_E_OOM;
  } catch (const std::exception& e) {
    internal_set_error(c, e.what());
    return HOS_E_DEVICE;
  }
}

// fp16 operand scratch the fused kernels also write (rows × cols, no residual plane)
H16 op_h16(hos_ctx* c, size_t rows, size_t cols) {
  DevMem& d = internal_scratch(c, 0);
  DevMem& r = internal_scratch(c, 1);
  d.ensure(rows * cols * 2);
  r.ensure(rows * 4 + 4);
  return H16{(half_t*)d.p, (float*)r.p, nullptr};
}

__global__ void transpose_kernel(const float* __restrict__ src, int rows, int cols, float* __restrict__ dst) {
  __shared__ float t[32][33];
  const int c0 = blockIdx.x * 32, r0 = blockIdx.y * 32;
  for (int i = threadIdx.y; i < 32; i += 8) {
    const int r = r0 + i, c = c0 + threadIdx.x;
    if (r < rows && c < cols) t[i][threadIdx.x] = src[(long long)r * cols + c];
  }
  __syncthreads();
  for (int i = threadIdx.y; i < 32; i += 8) {
    const int c = c0 + i, r = r0 + threadIdx.x;
    if (r < rows && c < cols) dst[(long long)c * rows + r] = t[threadIdx.x][i];
  }
}
// dst [cols][rows] = src [rows][cols]ᵀ
void transpose(const float* src, int rows, int cols, float* dst, hipStream_t st) {
  dim3 g(ceil_div(cols, 32), ceil_div(rows, 32));
  transpose_kernel<<<g, dim3(32, 8), 0, st>>>(src, rows, cols, dst);
  HOS_HIP_CHECK(hipGetLastError());
}

void lora_check(const float* x, const float* dy, size_t in, size_t out, int r, const float* A, const float* B,
                const float* u, const float* dA, const float* dB) {
  HOS_REQUIRE(x && dy && A && B && u && dA && dB && r > 0 && r <= 96, HOS_E_INVALID, "lora: bad arguments");
  HOS_REQUIRE(in % 4 == 0 && out % 4 == 0, HOS_E_INVALID, "lora: in and out must be multiples of 4");
}

// The two cols jobs of the branch: dB = s·uᵀ·dy [r, out] and dA = (duᵀ·x)ᵀ [in, r] (strided stores).
void lora_cols_jobs(const float* dy, const float* x, size_t rows, size_t in, size_t out, int r, float scale,
                    const float* u, const float* du, float* dB, float* dA, ColsJob* jdb, ColsJob* jda) {
  (void)rows;
  ColsSeg cb;
  cb.nseg = 1;
  cb.len[0] = (int)out;
  ColsSeg ca;
  ca.nseg = 1;
  ca.len[0] = (int)in;
  *jdb = ColsJob{r, scale, u, r, dy, (long long)out, cb, dB, (long long)out, 1};
  *jda = ColsJob{r, 1.0f, du, r, x, (long long)in, ca, dA, 1, (long long)r};  // dA(c, j): written as [in, r]
}

// The LoRA branch on caller-provided scratch: at [r, in] (Aᵀ), du [rows, r], ws the split partials.
void lora_run(const float* x, const float* dy, size_t rows, size_t in, size_t out, int r, const float* A,
              const float* B, float scale, float* y, float* u, float* dA, float* dB, float* dx, float* at, float* du,
              float* ws, size_t wsb, hipStream_t st) {
  transpose(A, (int)in, r, at, st);
  RowsSeg down;
  down.nt = 1;
  down.r = r;
  down.kend[0] = (int)in;
  RowsSeg up;
  up.nt = 1;
  up.r = r;
  up.kend[0] = (int)out;
  // u = x·A and du = s·dy·Bᵀ (independent) in one launch
  launch_lora_rows2((long long)rows, RowsCall{(long long)in, 1.0f, x, (long long)in, at, (long long)in, down, u, r},
                    RowsCall{(long long)out, scale, dy, (long long)out, B, (long long)out, up, du, r}, ws, wsb, st);
  if (y)
    launch_gemm_f32((long long)rows, (long long)out, r, scale, u, r, 1, B, (long long)out, 1, 1.0f, y, (long long)out,
                    ws, wsb, st);
  // dB = s·uᵀ·dy and dA = (duᵀ·x)ᵀ in one launch
  ColsJob jdb, jda;
  lora_cols_jobs(dy, x, rows, in, out, r, scale, u, du, dB, dA, &jdb, &jda);
  launch_lora_cols2((long long)rows, jdb, &jda, ws, wsb, st);
  if (dx)
    launch_gemm_f32((long long)rows, (long long)in, r, 1.0f, du, r, 1, A, 1, r, 1.0f, dx, (long long)in, ws, wsb, st);
}

// Workspace the branch's split launches need (the f32 GEMMs of y and dx split only into what is left).
size_t lora_ws_need(size_t rows, size_t in, size_t out, int r) {
  ColsJob jdb, jda;
  lora_cols_jobs(nullptr, nullptr, rows, in, out, r, 1.0f, nullptr, nullptr, nullptr, nullptr, &jdb, &jda);
  return std::max(lora_rows_ws_bytes((long long)rows, (long long)in, r) +
                      lora_rows_ws_bytes((long long)rows, (long long)out, r),
                  lora_cols2_ws_bytes((long long)rows, jdb, &jda));
}

size_t align256(size_t b) { return (b + 255) / 256 * 256; }

// Scratch of hos_hip_lora_noalloc: a file-scope device array, one copy per GPU, held for the life of the
// process. Host code never passes the array's name to a kernel (on the host it is only a stand-in symbol):
// the device address is looked up once per device with hipGetSymbolAddress and kept per device. Every call
// on one GPU shares the array and leaves its contents behind; the kernels write every scratch element before
// reading it, so nothing needs clearing. Calls that overlap on one GPU (two streams or two contexts) race.
// The cached address is valid for the life of the loaded code object: hipDeviceReset (which frees the module's
// device globals) is not supported in a process that uses this entry point.
void* lora_scratch_ptr() {
  static std::mutex mu;
  static void* ptr[64] = {};
  int dev = 0;
  HOS_HIP_CHECK(hipGetDevice(&dev));
  HOS_REQUIRE(dev >= 0 && dev < 64, HOS_E_DEVICE, "lora_noalloc: device index out of range");
  std::lock_guard<std::mutex> lk(mu);
  if (!ptr[dev]) {
    void* p = nullptr;
    HOS_HIP_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    HOS_REQUIRE(p != nullptr, HOS_E_DEVICE, "lora_noalloc: no device address for the scratch array");
    ptr[dev] = p;
  }
  return ptr[dev];
}

}  // namespace

extern "C" {

// embedding (src/tensor.rs:2438-2457): out[r] = deq(table)[ids[r]] with the table uploaded under `key`.
int hos_hip_embedding(hos_ctx* c, uint64_t key, const int32_t* ids_dev, size_t rows, float* out_dev) {
  return op_guard(c, [&](hipStream_t st) {
    HOS_REQUIRE(ids_dev && out_dev, HOS_E_INVALID, "null pointer");
    const QWeight& w = internal_qweight(c, key);
    launch_embed(w, ids_dev, out_dev, (int)rows, (int)w.cols, st);
  });
}

// rmsnorm_eps forward (src/tensor.rs:2500-2520): y = x·inv·w, inv = 1/sqrt(mean(x²) + eps) per row.
int hos_hip_rmsnorm_fwd(hos_ctx* c, const float* x, const float* w, size_t rows, size_t d, float eps, float* y,
                        float* inv) {
  return op_guard(c, [&](hipStream_t st) {
    HOS_REQUIRE(x && w && y && inv, HOS_E_INVALID, "null pointer");
    launch_rmsnorm_fwd(const_cast<float*>(x), w, eps, (int)rows, (int)d, y, op_h16(c, rows, d), inv, st);  // x read only
  });
}

// rmsnorm_eps backward (src/tensor.rs:2521-2544), input gradient: gx = g·w·inv − inv³·x/d·Σ(g·w·x).
// (The weight gradient is not formed: the norm weights are frozen in PEFT.)
int hos_hip_rmsnorm_bwd(hos_ctx* c, const float* g, const float* x, const float* inv, const float* w, size_t rows,
                        size_t d, float* gx) {
  return op_guard(c, [&](hipStream_t st) {
    HOS_REQUIRE(g && x && inv && w && gx, HOS_E_INVALID, "null pointer");
    launch_fill(gx, (long long)(rows * d), 0.0f, st);
    launch_rmsnorm_bwd(const_cast<float*>(g), x, inv, w, (int)rows, (int)d, gx, st);  // g read only
  });
}

// rope (src/tensor.rs:2750-2814) in place on the heads of rows [rows, ld] starting at column col0;
// position = row % seq_len; inverse != 0 applies Rᵀ (the backward).
int hos_hip_rope(hos_ctx* c, float* x, size_t rows, size_t ld, size_t col0, int n_heads, int head_dim, int seq_len,
                 float base, int neox, int inverse) {
  return op_guard(c, [&](hipStream_t st) {
    HOS_REQUIRE(x && n_heads > 0 && head_dim > 0 && head_dim % 2 == 0 && seq_len > 0, HOS_E_INVALID,
                "rope: bad arguments");
    const int half = head_dim / 2;
    std::vector<float2> tab((size_t)seq_len * half);
    for (int p = 0; p < seq_len; p++)
      for (int i = 0; i < half; i++) {
        const float freq = 1.0f / powf(base, 2.0f * (float)i / (float)head_dim);
        const float ang = (float)p * freq;
        tab[(size_t)p * half + i] = make_float2(sinf(ang), cosf(ang));
      }
    DevMem& t = internal_scratch(c, 2);
    t.ensure(tab.size() * sizeof(float2));
    HOS_HIP_CHECK(hipMemcpyAsync(t.p, tab.data(), tab.size() * sizeof(float2), hipMemcpyHostToDevice, st));
    launch_rope(x, (long long)ld, (int)col0, n_heads, head_dim, seq_len, (const float2*)t.p, neox != 0, inverse != 0,
                (int)rows, st);
    HOS_HIP_CHECK(hipStreamSynchronize(st));  // the host table must outlive the copy
  });
}

// SwiGLU silu(gate)·up (src/tensor.rs:2082-2100, 458-480); gu rows = [gate (F) | up (F)], h [rows, F].
int hos_hip_swiglu_fwd(hos_ctx* c, const float* gu, size_t rows, size_t F, float* h) {
  return op_guard(c, [&](hipStream_t st) {
    HOS_REQUIRE(gu && h, HOS_E_INVALID, "null pointer");
    launch_swiglu_fwd(gu, (int)rows, (int)F, h, op_h16(c, rows, F), st);
  });
}
// Its backward: dgu rows = [d gate | d up].
int hos_hip_swiglu_bwd(hos_ctx* c, const float* gu, const float* dh, size_t rows, size_t F, float* dgu) {
  return op_guard(c, [&](hipStream_t st) {
    HOS_REQUIRE(gu && dh && dgu, HOS_E_INVALID, "null pointer");
    launch_swiglu_bwd(gu, dh, (int)rows, (int)F, dgu, op_h16(c, rows, 2 * F), st);
  });
}

// Causal GQA attention of PeftModel::forward (src/peft.rs:530-553; bmm/softmax src/tensor.rs:2207-2280,
// 2460-2491) over B sequences of T rows. qkv rows [B·T, ld]: q heads at column 0, k at kcol, v at vcol.
// o [B·T, ldo]; lse [B, n_heads, T] (saved for the backward).
int hos_hip_attention_fwd(hos_ctx* c, const float* qkv, size_t ld, size_t kcol, size_t vcol, int B, int T,
                          int n_heads, int n_kv_heads, int head_dim, float* o, size_t ldo, float* lse) {
  return op_guard(c, [&](hipStream_t st) {
    HOS_REQUIRE(qkv && o && lse && B > 0 && T > 0 && n_kv_heads > 0 && n_heads % n_kv_heads == 0, HOS_E_INVALID,
                "attention: bad arguments");
    DevMem& pl = internal_scratch(c, 7);  // bf16 planes of q, k, v
    pl.ensure(attn_scratch_bytes(B, T, n_heads, n_kv_heads, head_dim));
    launch_attn_fwd(qkv, (long long)ld, (int)kcol, (int)vcol, B, T, n_heads, n_kv_heads, head_dim, o, (long long)ldo,
                    lse, pl.p, st);
  });
}
// Its backward: dqkv (same layout as qkv, row stride ldd) receives dq, dk, dv.
int hos_hip_attention_bwd(hos_ctx* c, const float* qkv, size_t ld, size_t kcol, size_t vcol, const float* o,
                          const float* dout, size_t ldo, const float* lse, int B, int T, int n_heads, int n_kv_heads,
                          int head_dim, float* dqkv, size_t ldd) {
  return op_guard(c, [&](hipStream_t st) {
    HOS_REQUIRE(qkv && o && dout && lse && dqkv && B > 0 && T > 0 && n_kv_heads > 0 && n_heads % n_kv_heads == 0,
                HOS_E_INVALID, "attention: bad arguments");
    const size_t M = (size_t)B * T;
    DevMem& dv = internal_scratch(c, 3);
    dv.ensure(M * n_heads * 4);
    float* part = nullptr;
    if (n_heads != n_kv_heads) {
      DevMem& pm = internal_scratch(c, 4);
      pm.ensure(M * n_heads * 2 * head_dim * 4);
      part = (float*)pm.p;
    }
    DevMem& pl = internal_scratch(c, 7);  // bf16 planes of q, k, v
    pl.ensure(attn_scratch_bytes(B, T, n_heads, n_kv_heads, head_dim));
    launch_attn_bwd(qkv, (long long)ld, (int)kcol, (int)vcol, o, dout, (long long)ldo, lse, (float*)dv.p, B, T,
                    n_heads, n_kv_heads, head_dim, dqkv, (long long)ldd, part, pl.p, st);
  });
}

// cross_entropy (src/tensor.rs:2709-2743) per row: row_loss[r] = −ln max(p_target, 1e−12) and
// dlogits = (p − onehot)·gscale (the reference's g/n is gscale = 1/rows).
int hos_hip_cross_entropy(hos_ctx* c, const float* logits, size_t rows, size_t V, const int32_t* targets,
                          float gscale, float* row_loss, float* dlogits) {
  return op_guard(c, [&](hipStream_t st) {
    HOS_REQUIRE(logits && targets && row_loss && dlogits, HOS_E_INVALID, "null pointer");
    launch_ce(logits, (int)rows, (int)V, targets, gscale, row_loss, H16{nullptr, nullptr, nullptr}, st, dlogits);
  });
}

// The MoE router of src/forward.rs:542-552 on logits [rows, E]: softmax probabilities pfull [rows, E], the top K
// experts per row by probability (a stable descending sort: ties to the lower expert) with their raw
// probabilities, sel_e / sel_p [rows, K] in selection order; slot [rows, K] is each selection's rank among its
// expert's selections and counts [E] the per-expert totals (the grouping the expert GEMMs use).
int hos_hip_moe_route(hos_ctx* c, const float* logits, size_t rows, int E, int K, float* pfull, int32_t* sel_e,
                      float* sel_p, int32_t* slot, int32_t* counts) {
  return op_guard(c, [&](hipStream_t st) {
    HOS_REQUIRE(logits && pfull && sel_e && sel_p && slot && counts, HOS_E_INVALID, "null pointer");
    launch_moe_route(logits, (int)rows, E, K, pfull, sel_e, sel_p, slot, counts, st);
  });
}

// AdamW::step (src/tensor.rs:2952-2975) on n parameters; `step` is the 1-based step count t that the
// bias corrections 1 − β^t use (f32 powi, as the reference).
int hos_hip_adamw(hos_ctx* c, float* p, const float* g, float* m, float* v, size_t n, float lr, float beta1,
                  float beta2, float eps, float wd, int step, int decay) {
  return op_guard(c, [&](hipStream_t st) {
    HOS_REQUIRE(p && g && m && v && step >= 1, HOS_E_INVALID, "adamw: bad arguments");
    const float bc1 = 1.0f - powi_f32(beta1, step), bc2 = 1.0f - powi_f32(beta2, step);
    launch_adamw(p, g, m, v, (long long)n, lr, beta1, beta2, eps, wd, bc1, bc2, decay != 0, st);
  });
}

// One LoRA branch y += s·(x·A)·B (src/peft.rs:508-512) and its backward through the matmul VJPs
// (src/tensor.rs:340-391), reference layouts A [in, r], B [r, out]:
//   u = x·A [rows, r];  y += s·u·B (y optional);  dB = s·uᵀ·dy;  du = s·dy·Bᵀ;  dA = xᵀ·du;
//   dx += du·Aᵀ (dx optional). x [rows, in] and dy [rows, out] row-major, r ≤ 96.
int hos_hip_lora(hos_ctx* c, const float* x, const float* dy, size_t rows, size_t in, size_t out, int r,
                 const float* A, const float* B, float scale, float* y, float* u, float* dA, float* dB, float* dx) {
  return op_guard(c, [&](hipStream_t st) {
    lora_check(x, dy, in, out, r, A, B, u, dA, dB);
    DevMem& wsm = internal_ws(c);
    DevMem& at = internal_scratch(c, 5);  // Aᵀ [r, in]
    at.ensure((size_t)r * in * 4);
    DevMem& dub = internal_scratch(c, 6);  // du [rows, r]
    dub.ensure(rows * r * 4 + 4);
    lora_run(x, dy, rows, in, out, r, A, B, scale, y, u, dA, dB, dx, (float*)at.p, (float*)dub.p, (float*)wsm.p,
             wsm.n, st);
  });
}

// hos_hip_lora without any device allocation: Aᵀ, du and the split partials live in `scratch`.
int hos_hip_lora_noalloc(hos_ctx* c, const float* x, const float* dy, size_t rows, size_t in, size_t out, int r,
                         const float* A, const float* B, float scale, float* y, float* u, float* dA, float* dB,
                         float* dx) {
  return op_guard(c, [&](hipStream_t st) {
    lora_check(x, dy, in, out, r, A, B, u, dA, dB);
    const size_t at_b = align256((size_t)r * in * 4), du_b = align256(rows * r * 4 + 4);
    const size_t ws_b = lora_ws_need(rows, in, out, r);
    HOS_REQUIRE(at_b + du_b + ws_b <= kLoraScratch, HOS_E_INVALID,
                "lora_noalloc: rows " + std::to_string(rows) + ", in " + std::to_string(in) + ", out " +
                    std::to_string(out) + ", r " + std::to_string(r) + " need " + std::to_string(at_b + du_b + ws_b) +
                    " bytes of scratch; the maximum is " + std::to_string(kLoraScratch));
    char* base = (char*)lora_scratch_ptr();
    float* ws = (float*)(base + at_b + du_b);
    lora_run(x, dy, rows, in, out, r, A, B, scale, y, u, dA, dB, dx, (float*)base, (float*)(base + at_b), ws,
             kLoraScratch - at_b - du_b, st);
  });
}

}  // extern "C"
