// qGEMM instantiations for Q8_0 (also Q4_0 and Q5_0, repacked into this layout) weights (all tile shapes, both directions, precision modes 1-4).
#include "qgemm_impl.hpp"

HOS_QGEMM_INSTANTIATE(q8, GGUF_Q8_0)
