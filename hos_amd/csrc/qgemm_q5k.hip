// qGEMM instantiations for Q5_K weights (all tile shapes, both directions, precision modes 1-5).
#include "qgemm_impl.hpp"

HOS_QGEMM_INSTANTIATE(q5k, GGUF_Q5_K)
