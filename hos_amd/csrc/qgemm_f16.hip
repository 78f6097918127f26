// qGEMM instantiations for F16 weights (all tile shapes, both directions, precision modes 1-5).
#include "qgemm_impl.hpp"

HOS_QGEMM_INSTANTIATE(f16, GGUF_F16)
