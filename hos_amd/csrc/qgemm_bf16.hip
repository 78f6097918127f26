// qGEMM instantiations for BF16 weights (all tile shapes, both directions, precision modes 1-5).
#include "qgemm_impl.hpp"

HOS_QGEMM_INSTANTIATE(bf16, GGUF_BF16)
