// qGEMM instantiations for F32 weights (all tile shapes, both directions, precision modes 1-5).
#include "qgemm_impl.hpp"

HOS_QGEMM_INSTANTIATE(f32, GGUF_F32)
