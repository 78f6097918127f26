// qGEMM instantiations for Q8_0 (also Q4_0 and Q5_0, repacked into this layout) weights (all tile shapes, both directions, precision modes 1-5).
#include "qgemm_impl.hpp"

HOS_QGEMM_INSTANTIATE(q8, GGUF_Q8_0)

namespace hos {
// The split-K reduction for callers outside the GEMM translation units (a consumer that cannot fuse deferred
// partials).
void launch_qgemm_split_reduce(const float* ws, int splits, long long M, int N, const float* rinv, const GemmEpi& epi,
                               hipStream_t st) {
  launch_splitk_reduce(ws, splits, M, N, rinv, epi, st);
}
}  // namespace hos
