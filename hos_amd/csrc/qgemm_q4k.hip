// qGEMM instantiations for Q4_K weights (all tile shapes, both directions, precision modes 1-5).
#include "qgemm_impl.hpp"

HOS_QGEMM_INSTANTIATE(q4k, GGUF_Q4_K)
