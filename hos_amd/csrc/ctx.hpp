// Host-side helpers shared by the C ABI translation units.
#pragma once
#include "kernels.hpp"

namespace hos {

// Owning device allocation that only grows.
struct DevMem {
  void* p = nullptr;
  size_t n = 0;
  DevMem() = default;
  DevMem(const DevMem&) = delete;
  DevMem& operator=(const DevMem&) = delete;
  DevMem(DevMem&& o) noexcept : p(o.p), n(o.n) {
    o.p = nullptr;
    o.n = 0;
  }
  ~DevMem();
  void reset();
  void ensure(size_t bytes);
};

void free_qweight(QWeight& w);
// Upload GGUF bytes and repack them on the device (synchronous).
void upload_qweight(hipStream_t st, const uint8_t* bytes, size_t nbytes, uint32_t type, size_t rows, size_t cols,
                    QWeight& w);

// f32 powi as compiler-rt's __powisf2 (Rust f32::powi, the reference's AdamW bias corrections):
// square-and-multiply over the exponent bits.
inline float powi_f32(float a, int b) {
  const bool recip = b < 0;
  float r = 1.0f;
  while (true) {
    if (b & 1) r *= a;
    b /= 2;
    if (b == 0) break;
    a *= a;
  }
  return recip ? 1.0f / r : r;
}

// Context internals for the op-level entry points (ops.hip).
DevMem& internal_scratch(hos_ctx* c, int slot);  // slot < 8, owned by the context
DevMem& internal_ws(hos_ctx* c);                  // the context's GEMM workspace (256 MB)
const QWeight& internal_qweight(hos_ctx* c, uint64_t key);
void internal_set_error(hos_ctx* c, const std::string& e);

}  // namespace hos

extern "C" {
hipStream_t hos_internal_stream(hos_ctx* c);
int hos_internal_device(hos_ctx* c);
}
