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

}  // namespace hos

extern "C" {
hipStream_t hos_internal_stream(hos_ctx* c);
int hos_internal_device(hos_ctx* c);
}
