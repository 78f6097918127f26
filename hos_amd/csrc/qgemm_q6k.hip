// qGEMM instantiations for Q6_K weights (all tile shapes, both directions, precision modes 1-5).
#include "qgemm_impl.hpp"

HOS_QGEMM_INSTANTIATE(q6k, GGUF_Q6_K)
