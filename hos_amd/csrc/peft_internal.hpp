// Host-side access to a hos_peft's LoRA arena for the checkpoint code (not part of the C ABI).
#pragma once
#include <cstdint>
#include <functional>
#include <string>
#include <utility>
#include <vector>

#include "../../include/hos_hip.h"

namespace hos {

enum PeftBuf { PEFT_PARAM = 0, PEFT_GRAD = 1, PEFT_ADAM_M = 2, PEFT_ADAM_V = 3 };

struct PeftShape {
  int L, r;
  uint32_t targets;      // bitmask over q,k,v,o,gate,up,down
  int in[7], out[7];     // (in, out) of each target's projection
  uint64_t step;         // AdamW steps taken
  float lr, wd;          // last AdamW hyper-parameters
  int vocab, dim;
  bool rga;              // RGA adapters instead of LoRA
};

// RGA adapter tensors as (name, shape): PeftModel::adapter_tensors order (genome, wg, then per layer wr and
// each gene's down, up; src/peft.rs:741-760), or with param_order PeftModel::params order (wg, per layer wr,
// downs, ups, then the genome; src/peft.rs:283-311), which the optimizer state follows.
std::vector<std::pair<std::string, std::vector<uint32_t>>> peft_rga_tensors(const hos_peft* p, bool param_order);
// Copy one RGA tensor of `which` by name between the device and a host buffer (reference layout, n floats).
void peft_rga_io(hos_peft* p, PeftBuf which, const std::string& name, float* data, size_t n, bool upload);

// Copy one (layer, target) factor pair of `which` between the device and host buffers in the reference
// layout (A [in, r], B [r, out] row-major). Either pointer may be null.
void peft_factor_io(hos_peft* p, PeftBuf which, int layer, int target, float* A, float* B, bool upload);
PeftShape peft_shape(const hos_peft* p);
void peft_set_adam_state(hos_peft* p, uint64_t step, float lr, float wd);
void peft_token_embedding(hos_peft* p, std::vector<float>& out);
// Run f with the model's device current, mapping exceptions to a status code and last-error string.
int peft_call(hos_peft* p, const std::function<void()>& f);

}  // namespace hos
