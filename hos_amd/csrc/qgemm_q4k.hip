// qGEMM instantiations for GGUF_Q4_K (all tile shapes, both directions, precision modes 1-4).
#include "qgemm_impl.hpp"

namespace hos {

void qgemm_launch_q4k(bool dx, int passes, const QWeight& w, H16 a, long long lda, long long M, GemmEpi epi,
                        float* ws, size_t ws_bytes, hipStream_t st) {
  if (dx) {
    if (passes == 1) launch_typed<GGUF_Q4_K, true, 1>(w, a, lda, M, epi, ws, ws_bytes, st);
    else if (passes == 2) launch_typed<GGUF_Q4_K, true, 2>(w, a, lda, M, epi, ws, ws_bytes, st);
    else if (passes == 3) launch_typed<GGUF_Q4_K, true, 3>(w, a, lda, M, epi, ws, ws_bytes, st);
    else launch_typed<GGUF_Q4_K, true, 4>(w, a, lda, M, epi, ws, ws_bytes, st);
  } else {
    if (passes == 1) launch_typed<GGUF_Q4_K, false, 1>(w, a, lda, M, epi, ws, ws_bytes, st);
    else if (passes == 2) launch_typed<GGUF_Q4_K, false, 2>(w, a, lda, M, epi, ws, ws_bytes, st);
    else if (passes == 3) launch_typed<GGUF_Q4_K, false, 3>(w, a, lda, M, epi, ws, ws_bytes, st);
    else launch_typed<GGUF_Q4_K, false, 4>(w, a, lda, M, epi, ws, ws_bytes, st);
  }
}

}  // namespace hos

namespace hos {
void qgemm_grouped_q4k(bool dx, int passes, const QWeight& w, GroupSched gs, H16 a, long long lda, GemmEpi epi,
                      hipStream_t st) {
  if (dx) {
    if (passes == 1) launch_typed_grouped<GGUF_Q4_K, true, 1>(w, gs, a, lda, epi, st);
    else if (passes == 2) launch_typed_grouped<GGUF_Q4_K, true, 2>(w, gs, a, lda, epi, st);
    else if (passes == 3) launch_typed_grouped<GGUF_Q4_K, true, 3>(w, gs, a, lda, epi, st);
    else launch_typed_grouped<GGUF_Q4_K, true, 4>(w, gs, a, lda, epi, st);
  } else {
    if (passes == 1) launch_typed_grouped<GGUF_Q4_K, false, 1>(w, gs, a, lda, epi, st);
    else if (passes == 2) launch_typed_grouped<GGUF_Q4_K, false, 2>(w, gs, a, lda, epi, st);
    else if (passes == 3) launch_typed_grouped<GGUF_Q4_K, false, 3>(w, gs, a, lda, epi, st);
    else launch_typed_grouped<GGUF_Q4_K, false, 4>(w, gs, a, lda, epi, st);
  }
}
}  // namespace hos
