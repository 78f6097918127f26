// C ABI: context, keyed f32 GEMMs, quantized weights, device memory (include/hos_hip.h).
#include <cstring>
#include <unordered_map>
#include <vector>

#include "ctx.hpp"

using namespace hos;

namespace hos {

DevMem::~DevMem() { reset(); }
void DevMem::reset() {
  if (p) (void)hipFree(p);
  p = nullptr;
  n = 0;
}
void DevMem::ensure(size_t bytes) {
  if (bytes <= n) return;
  reset();
  if (bytes == 0) return;
  hipError_t e = hipMalloc(&p, bytes);
  if (e != hipSuccess) {
    p = nullptr;
    throw Error(HOS_E_OOM, "hipMalloc(" + std::to_string(bytes) + ") failed: " + hipGetErrorString(e));
  }
  n = bytes;
}

void free_qweight(QWeight& w) {
  if (w.q) (void)hipFree(w.q);
  if (w.s) (void)hipFree(w.s);
  w.q = nullptr;
  w.s = nullptr;
}

void upload_qweight(hipStream_t st, const uint8_t* bytes, size_t nbytes, uint32_t type, size_t rows, size_t cols,
                    QWeight& w) {
  HOS_REQUIRE(bytes != nullptr, HOS_E_INVALID, "upload_quant: null bytes");
  size_t be = block_elems(type);
  HOS_REQUIRE(be != 0, HOS_E_UNSUPPORTED_QUANT,
              "unsupported quantization type " + std::to_string(type) +
                  " (supported: F32, F16, BF16, Q4_0, Q5_0, Q8_0, Q4_K, Q5_K, Q6_K)");
  HOS_REQUIRE(rows > 0 && cols > 0 && cols % be == 0, HOS_E_INVALID,
              "upload_quant: cols must be a positive multiple of the block size " + std::to_string(be));
  HOS_REQUIRE(cols % 32 == 0, HOS_E_INVALID, "upload_quant: cols must be a multiple of 32");
  HOS_REQUIRE(rows <= (1ull << 40) / cols, HOS_E_INVALID, "upload_quant: matrix too large");
  size_t need = gguf_bytes_for(type, rows * cols);
  HOS_REQUIRE(nbytes == need, HOS_E_FORMAT,
              "upload_quant: got " + std::to_string(nbytes) + " bytes, expected " + std::to_string(need));
  w.type = storage_type(type);
  w.rows = (long long)rows;
  w.cols = (long long)cols;
  qweight_sizes(w.type, w.rows, w.cols, &w.q_bytes, &w.s_bytes);
  DevMem raw;
  raw.ensure(nbytes);
  HOS_HIP_CHECK(hipMalloc(&w.q, w.q_bytes));
  HOS_HIP_CHECK(hipMalloc((void**)&w.s, w.s_bytes > 0 ? w.s_bytes : 256));  // never read for unscaled types
  HOS_HIP_CHECK(hipMemcpyAsync(raw.p, bytes, nbytes, hipMemcpyHostToDevice, st));
  repack_weight((const uint8_t*)raw.p, type, w, st);
  HOS_HIP_CHECK(hipStreamSynchronize(st));
}

}  // namespace hos

struct hos_ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  std::string err;
  std::unordered_map<uint64_t, QWeight> qw;
  std::unordered_map<uint64_t, DevMem> f32cache;
  DevMem ws, t0, t1, t2, t3, t4, t5;
  DevMem ops[8];  // scratch of the op-level entry points (ops.hip)
  int passes = 1;
  hipEvent_t tev[2] = {nullptr, nullptr};  // hos_hip_timer_begin / _end
  bool tarmed = false;                     // a timer_begin not yet closed by a timer_end
  static constexpr size_t kWs = 256ull << 20;
};

namespace {

template <class F>
int guard(hos_ctx* c, F&& f) {
  if (!c) return HOS_E_INVALID;
  try {
    HOS_HIP_CHECK(hipSetDevice(c->device));
    f();
    c->err.clear();
    return HOS_OK;
  } catch (const Error& e) {
    c->err = e.what();
    return e.code;
  } catch (const std::bad_alloc&) {
    c->err = "host allocation failed";
    return HOS_E_OOM;
  } catch (const std::exception& e) {
    c->err = e.what();
    return HOS_E_DEVICE;
  }
}

const QWeight& get_qw(hos_ctx* c, uint64_t key) {
  auto it = c->qw.find(key);
  HOS_REQUIRE(it != c->qw.end(), HOS_E_INVALID, "no quantized weight uploaded under key " + std::to_string(key));
  return it->second;
}

// Device copy of a host f32 operand: cached under `key` when key != 0 (buf_keyed).
const float* operand(hos_ctx* c, const float* host, size_t n, uint64_t key, DevMem& scratch) {
  HOS_REQUIRE(host != nullptr || n == 0, HOS_E_INVALID, "null operand");
  if (key) {
    auto it = c->f32cache.find(key);
    if (it != c->f32cache.end() && it->second.n >= n * 4) return (const float*)it->second.p;
    DevMem& m = c->f32cache[key];
    m.ensure(n * 4);
    HOS_HIP_CHECK(hipMemcpyAsync(m.p, host, n * 4, hipMemcpyHostToDevice, c->stream));
    return (const float*)m.p;
  }
  scratch.ensure(n * 4);
  HOS_HIP_CHECK(hipMemcpyAsync(scratch.p, host, n * 4, hipMemcpyHostToDevice, c->stream));
  return (const float*)scratch.p;
}

// fp16 operand scratch (+ residual plane when the context runs multi-pass GEMMs).
H16 operand_h16(hos_ctx* c, long long K, size_t t) {
  c->t2.ensure(t * K * 2);
  c->t3.ensure(t * 4 + 4);
  H16 a{(half_t*)c->t2.p, (float*)c->t3.p, nullptr};
  if (c->passes == 2 || c->passes == 3 || c->passes == 5) {
    c->t5.ensure(t * K * 2);
    a.lo = (half_t*)c->t5.p;
  }
  return a;
}

void qgemm_dev(hos_ctx* c, bool dx, uint64_t key, const float* in_dev, size_t t, float* out_dev,
               const GemmEpi* lora = nullptr) {
  const QWeight& w = get_qw(c, key);
  long long K = dx ? w.rows : w.cols;
  long long N = dx ? w.cols : w.rows;
  HOS_REQUIRE(in_dev && out_dev, HOS_E_INVALID, "qgemm: null pointer");
  H16 a = operand_h16(c, K, t);
  launch_to_h16(in_dev, K, (long long)t, K, a, c->stream);
  c->ws.ensure(hos_ctx::kWs);
  GemmEpi epi = lora ? *lora : GemmEpi{};
  epi.out = out_dev;
  epi.ldo = N;
  if (dx)
    launch_qgemm_dx(w, a, K, (long long)t, epi, (float*)c->ws.p, c->ws.n, c->passes, c->stream);
  else
    launch_qgemm_fwd(w, a, K, (long long)t, epi, (float*)c->ws.p, c->ws.n, c->passes, c->stream);
}

}  // namespace

extern "C" {

int hos_hip_create(int device, hos_ctx** out) {
  if (!out) return HOS_E_INVALID;
  *out = nullptr;
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n == 0) return HOS_E_DEVICE;
  if (device < 0 || device >= n) return HOS_E_INVALID;
  auto* c = new hos_ctx();
  c->device = device;
  if (hipSetDevice(device) != hipSuccess || hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess) {
    delete c;
    return HOS_E_DEVICE;
  }
  *out = c;
  return HOS_OK;
}

void hos_hip_destroy(hos_ctx* c) {
  if (!c) return;
  (void)hipSetDevice(c->device);
  (void)hipStreamSynchronize(c->stream);
  for (auto& kv : c->qw) free_qweight(kv.second);
  c->qw.clear();
  c->f32cache.clear();
  for (auto& e : c->tev)
    if (e) (void)hipEventDestroy(e);
  (void)hipStreamDestroy(c->stream);
  delete c;
}

const char* hos_hip_last_error(const hos_ctx* c) { return c ? c->err.c_str() : "null context"; }

int hos_hip_synchronize(hos_ctx* c) {
  return guard(c, [&] { HOS_HIP_CHECK(hipStreamSynchronize(c->stream)); });
}

int hos_hip_device_arch(hos_ctx* c, char* buf, size_t len) {
  return guard(c, [&] {
    HOS_REQUIRE(buf && len > 0, HOS_E_INVALID, "null buffer");
    hipDeviceProp_t p;
    HOS_HIP_CHECK(hipGetDeviceProperties(&p, c->device));
    std::snprintf(buf, len, "%s", p.gcnArchName);
  });
}

int hos_hip_matmul_f32_keyed(hos_ctx* c, const float* a, size_t m, size_t k, const float* b, size_t n, uint64_t b_key,
                             float* out) {
  return guard(c, [&] {
    HOS_REQUIRE(out, HOS_E_INVALID, "null out");
    const float* da = operand(c, a, m * k, 0, c->t0);
    const float* db = operand(c, b, k * n, b_key, c->t1);
    c->t4.ensure(m * n * 4);
    c->ws.ensure(hos_ctx::kWs);
    launch_gemm_f32(m, n, k, 1.0f, da, k, 1, db, n, 1, 0.0f, (float*)c->t4.p, n, (float*)c->ws.p, c->ws.n, c->stream);
    HOS_HIP_CHECK(hipMemcpyAsync(out, c->t4.p, m * n * 4, hipMemcpyDeviceToHost, c->stream));
    HOS_HIP_CHECK(hipStreamSynchronize(c->stream));
  });
}

int hos_hip_matmul_abt_keyed(hos_ctx* c, const float* a, size_t m, size_t n, const float* b, size_t k, uint64_t b_key,
                             float* out) {
  return guard(c, [&] {
    HOS_REQUIRE(out, HOS_E_INVALID, "null out");
    const float* da = operand(c, a, m * n, 0, c->t0);
    const float* db = operand(c, b, k * n, b_key, c->t1);
    c->t4.ensure(m * k * 4);
    c->ws.ensure(hos_ctx::kWs);
    // C[m,k] = Σ_j A[m,j]·B[k,j]: contraction j; B(j, kk) = B[kk·n + j]
    launch_gemm_f32(m, k, n, 1.0f, da, n, 1, db, 1, n, 0.0f, (float*)c->t4.p, k, (float*)c->ws.p, c->ws.n, c->stream);
    HOS_HIP_CHECK(hipMemcpyAsync(out, c->t4.p, m * k * 4, hipMemcpyDeviceToHost, c->stream));
    HOS_HIP_CHECK(hipStreamSynchronize(c->stream));
  });
}

int hos_hip_matmul_atb_keyed(hos_ctx* c, const float* a, size_t k, size_t m, const float* b, size_t n, uint64_t a_key,
                             float* out) {
  return guard(c, [&] {
    HOS_REQUIRE(out, HOS_E_INVALID, "null out");
    const float* da = operand(c, a, m * k, a_key, c->t0);
    const float* db = operand(c, b, m * n, 0, c->t1);
    c->t4.ensure(k * n * 4);
    c->ws.ensure(hos_ctx::kWs);
    // C[k,n] = Σ_i A[i,kk]·B[i,n]: A(row kk, contraction i) = A[i·k + kk]
    launch_gemm_f32(k, n, m, 1.0f, da, 1, k, db, n, 1, 0.0f, (float*)c->t4.p, n, (float*)c->ws.p, c->ws.n, c->stream);
    HOS_HIP_CHECK(hipMemcpyAsync(out, c->t4.p, k * n * 4, hipMemcpyDeviceToHost, c->stream));
    HOS_HIP_CHECK(hipStreamSynchronize(c->stream));
  });
}

int hos_hip_evict(hos_ctx* c, uint64_t key) {
  return guard(c, [&] {
    HOS_HIP_CHECK(hipStreamSynchronize(c->stream));
    c->f32cache.erase(key);
    auto it = c->qw.find(key);
    if (it != c->qw.end()) {
      free_qweight(it->second);
      c->qw.erase(it);
    }
  });
}

int hos_hip_clear_cache(hos_ctx* c) {
  return guard(c, [&] {
    HOS_HIP_CHECK(hipStreamSynchronize(c->stream));
    c->f32cache.clear();
  });
}

int hos_hip_upload_quant(hos_ctx* c, uint64_t key, const uint8_t* bytes, size_t nbytes, uint32_t type, size_t rows,
                         size_t cols) {
  return guard(c, [&] {
    HOS_REQUIRE(key != 0, HOS_E_INVALID, "upload_quant: key 0 is reserved");
    QWeight w;
    try {
      upload_qweight(c->stream, bytes, nbytes, type, rows, cols, w);
    } catch (...) {
      free_qweight(w);
      throw;
    }
    auto it = c->qw.find(key);
    if (it != c->qw.end()) free_qweight(it->second);
    c->qw[key] = w;
  });
}

int hos_hip_dequant(hos_ctx* c, uint64_t key, float* out) {
  return guard(c, [&] {
    HOS_REQUIRE(out, HOS_E_INVALID, "null out");
    const QWeight& w = get_qw(c, key);
    size_t n = (size_t)(w.rows * w.cols);
    c->t4.ensure(n * 4);
    launch_dequant(w, (float*)c->t4.p, c->stream);
    HOS_HIP_CHECK(hipMemcpyAsync(out, c->t4.p, n * 4, hipMemcpyDeviceToHost, c->stream));
    HOS_HIP_CHECK(hipStreamSynchronize(c->stream));
  });
}

static int qgemm_host(hos_ctx* c, bool dx, uint64_t key, const float* in, size_t t, float* out) {
  return guard(c, [&] {
    HOS_REQUIRE(in && out, HOS_E_INVALID, "null pointer");
    const QWeight& w = get_qw(c, key);
    size_t K = (size_t)(dx ? w.rows : w.cols), N = (size_t)(dx ? w.cols : w.rows);
    c->t0.ensure(t * K * 4);
    c->t1.ensure(t * N * 4);
    HOS_HIP_CHECK(hipMemcpyAsync(c->t0.p, in, t * K * 4, hipMemcpyHostToDevice, c->stream));
    qgemm_dev(c, dx, key, (const float*)c->t0.p, t, (float*)c->t1.p);
    HOS_HIP_CHECK(hipMemcpyAsync(out, c->t1.p, t * N * 4, hipMemcpyDeviceToHost, c->stream));
    HOS_HIP_CHECK(hipStreamSynchronize(c->stream));
  });
}

int hos_hip_qgemm_fwd(hos_ctx* c, uint64_t key, const float* x, size_t t, float* y) {
  return qgemm_host(c, false, key, x, t, y);
}
int hos_hip_qgemm_dx(hos_ctx* c, uint64_t key, const float* dy, size_t t, float* dx) {
  return qgemm_host(c, true, key, dy, t, dx);
}
int hos_hip_qgemm_fwd_dev(hos_ctx* c, uint64_t key, const float* x, size_t t, float* y) {
  return guard(c, [&] { qgemm_dev(c, false, key, x, t, y); });
}
int hos_hip_qgemm_dx_dev(hos_ctx* c, uint64_t key, const float* dy, size_t t, float* dx) {
  return guard(c, [&] { qgemm_dev(c, true, key, dy, t, dx); });
}

int hos_hip_qgemm_lora_dev(hos_ctx* c, int which, uint64_t key, const float* in_dev, size_t t, const float* u_dev,
                           size_t ldu, const float* l_dev, size_t slj, size_t sln, int rank, float scale,
                           float* out_dev) {
  return guard(c, [&] {
    HOS_REQUIRE(which == 0 || which == 1, HOS_E_INVALID, "qgemm_lora: which must be 0 (forward) or 1 (dX)");
    HOS_REQUIRE(rank >= 1 && u_dev && l_dev && ldu >= (size_t)rank, HOS_E_INVALID, "qgemm_lora: bad rank-r factors");
    GemmEpi e{};
    e.U = u_dev;
    e.ldu = (long long)ldu;
    e.L = l_dev;
    e.slj = (long long)slj;
    e.sln = (long long)sln;
    e.rank = rank;
    e.scale = scale;
    qgemm_dev(c, which == 1, key, in_dev, t, out_dev, &e);
  });
}

int hos_hip_time_qgemm(hos_ctx* c, int which, uint64_t key, const float* in_dev, size_t t, float* out_dev, int iters,
                       float* avg_ms) {
  return guard(c, [&] {
    HOS_REQUIRE(in_dev && out_dev && avg_ms && iters > 0, HOS_E_INVALID, "time_qgemm: bad arguments");
    const QWeight& w = get_qw(c, key);
    bool dx = which == 1;
    long long K = dx ? w.rows : w.cols, N = dx ? w.cols : w.rows;
    H16 a = operand_h16(c, K, t);
    launch_to_h16(in_dev, K, (long long)t, K, a, c->stream);
    c->ws.ensure(hos_ctx::kWs);
    GemmEpi epi{out_dev, N, nullptr, 0, nullptr};
    auto run = [&] {
      if (dx)
        launch_qgemm_dx(w, a, K, (long long)t, epi, (float*)c->ws.p, c->ws.n, c->passes, c->stream);
      else
        launch_qgemm_fwd(w, a, K, (long long)t, epi, (float*)c->ws.p, c->ws.n, c->passes, c->stream);
    };
    run();  // warm-up
    hipEvent_t e0, e1;
    HOS_HIP_CHECK(hipEventCreate(&e0));
    HOS_HIP_CHECK(hipEventCreate(&e1));
    HOS_HIP_CHECK(hipEventRecord(e0, c->stream));
    for (int i = 0; i < iters; i++) run();
    HOS_HIP_CHECK(hipEventRecord(e1, c->stream));
    HOS_HIP_CHECK(hipEventSynchronize(e1));
    float ms = 0.0f;
    HOS_HIP_CHECK(hipEventElapsedTime(&ms, e0, e1));
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    *avg_ms = ms / (float)iters;
  });
}

int hos_hip_timer_begin(hos_ctx* c) {
  return guard(c, [&] {
    for (auto& e : c->tev)
      if (!e) HOS_HIP_CHECK(hipEventCreate(&e));
    HOS_HIP_CHECK(hipEventRecord(c->tev[0], c->stream));
    c->tarmed = true;
  });
}

int hos_hip_timer_end(hos_ctx* c, float* ms) {
  return guard(c, [&] {
    HOS_REQUIRE(ms && c->tev[0] && c->tarmed, HOS_E_INVALID, "timer_end: no open timer_begin on this context");
    c->tarmed = false;
    HOS_HIP_CHECK(hipEventRecord(c->tev[1], c->stream));
    HOS_HIP_CHECK(hipEventSynchronize(c->tev[1]));
    HOS_HIP_CHECK(hipEventElapsedTime(ms, c->tev[0], c->tev[1]));
  });
}

int hos_hip_quantize(hos_ctx* c, const float* x, size_t n, uint32_t type, uint8_t* out) {
  return guard(c, [&] {
    HOS_REQUIRE(x && out, HOS_E_INVALID, "null pointer");
    size_t be = block_elems(type);
    HOS_REQUIRE(be != 0, HOS_E_UNSUPPORTED_QUANT, "quantize: unsupported type " + std::to_string(type));
    HOS_REQUIRE(n % be == 0, HOS_E_INVALID, "quantize: length must be a multiple of the block size");
    size_t nb = gguf_bytes_for(type, n);
    c->t0.ensure(n * 4);
    c->t1.ensure(nb);
    HOS_HIP_CHECK(hipMemcpyAsync(c->t0.p, x, n * 4, hipMemcpyHostToDevice, c->stream));
    launch_quantize((const float*)c->t0.p, n, type, (uint8_t*)c->t1.p, c->stream);
    HOS_HIP_CHECK(hipMemcpyAsync(out, c->t1.p, nb, hipMemcpyDeviceToHost, c->stream));
    HOS_HIP_CHECK(hipStreamSynchronize(c->stream));
  });
}

int hos_hip_quantize_dev(hos_ctx* c, const float* x_dev, size_t n, uint32_t type, uint8_t* out_dev) {
  return guard(c, [&] {
    HOS_REQUIRE(x_dev && out_dev, HOS_E_INVALID, "null pointer");
    size_t be = block_elems(type);
    HOS_REQUIRE(be != 0, HOS_E_UNSUPPORTED_QUANT, "quantize: unsupported type " + std::to_string(type));
    HOS_REQUIRE(n % be == 0, HOS_E_INVALID, "quantize: length must be a multiple of the block size");
    launch_quantize(x_dev, n, type, out_dev, c->stream);
    HOS_HIP_CHECK(hipStreamSynchronize(c->stream));
  });
}

int hos_hip_randn_dev(hos_ctx* c, float* out_dev, size_t n, uint64_t seed, float stddev) {
  return guard(c, [&] {
    HOS_REQUIRE(out_dev != nullptr, HOS_E_INVALID, "null pointer");
    launch_randn(out_dev, n, seed, stddev, c->stream);
    HOS_HIP_CHECK(hipStreamSynchronize(c->stream));
  });
}

size_t hos_hip_bytes_for(uint32_t type, size_t n) { return gguf_bytes_for(type, n); }

int hos_hip_set_gemm_passes(hos_ctx* c, int passes) {
  return guard(c, [&] {
    HOS_REQUIRE(passes >= 1 && passes <= 5, HOS_E_INVALID, "gemm precision mode must be 1 to 5");
    c->passes = passes;
  });
}

int hos_hip_dev_alloc(hos_ctx* c, size_t nbytes, void** dptr) {
  return guard(c, [&] {
    HOS_REQUIRE(dptr, HOS_E_INVALID, "null out pointer");
    hipError_t e = hipMalloc(dptr, nbytes);
    if (e != hipSuccess) throw Error(HOS_E_OOM, std::string("hipMalloc failed: ") + hipGetErrorString(e));
  });
}
int hos_hip_dev_free(hos_ctx* c, void* p) {
  return guard(c, [&] {
    HOS_HIP_CHECK(hipStreamSynchronize(c->stream));
    HOS_HIP_CHECK(hipFree(p));
  });
}
int hos_hip_h2d(hos_ctx* c, void* dst, const void* src, size_t n) {
  return guard(c, [&] {
    HOS_HIP_CHECK(hipMemcpyAsync(dst, src, n, hipMemcpyHostToDevice, c->stream));
    HOS_HIP_CHECK(hipStreamSynchronize(c->stream));
  });
}
int hos_hip_d2h(hos_ctx* c, void* dst, const void* src, size_t n) {
  return guard(c, [&] {
    HOS_HIP_CHECK(hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToHost, c->stream));
    HOS_HIP_CHECK(hipStreamSynchronize(c->stream));
  });
}

// Accessors the training model needs (peft.hip) — not part of the public ABI.
hipStream_t hos_internal_stream(hos_ctx* c) { return c->stream; }
int hos_internal_device(hos_ctx* c) { return c->device; }

}  // extern "C"

namespace hos {
DevMem& internal_scratch(hos_ctx* c, int slot) { return c->ops[slot]; }
DevMem& internal_ws(hos_ctx* c) {
  c->ws.ensure(hos_ctx::kWs);
  return c->ws;
}
const QWeight& internal_qweight(hos_ctx* c, uint64_t key) { return get_qw(c, key); }
void internal_set_error(hos_ctx* c, const std::string& e) { c->err = e; }
}  // namespace hos
