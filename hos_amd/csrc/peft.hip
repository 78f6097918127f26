// Placeholder: the LoRA training model is not wired yet.
#include "ctx.hpp"

struct hos_peft {
  std::string err = "not implemented";
};

extern "C" {
int hos_peft_create(hos_ctx*, const hos_peft_cfg*, hos_peft** out) { if (out) *out = nullptr; return HOS_E_INVALID; }
void hos_peft_destroy(hos_peft* p) { delete p; }
const char* hos_peft_last_error(const hos_peft* p) { return p ? p->err.c_str() : "null"; }
int hos_peft_set_tensor(hos_peft*, const char*, const uint8_t*, size_t, uint32_t, size_t, size_t) { return HOS_E_INVALID; }
int hos_peft_set_lora(hos_peft*, int, int, const float*, const float*) { return HOS_E_INVALID; }
int hos_peft_get_lora(hos_peft*, int, int, float*, float*) { return HOS_E_INVALID; }
int hos_peft_get_lora_grad(hos_peft*, int, int, float*, float*) { return HOS_E_INVALID; }
int hos_peft_loss_grad(hos_peft*, const int32_t*, const int32_t*, int, int, float*) { return HOS_E_INVALID; }
int hos_peft_adamw(hos_peft*, float, float) { return HOS_E_INVALID; }
int hos_peft_step_dev(hos_peft*, const int32_t*, const int32_t*, int, int, float, float, float*) { return HOS_E_INVALID; }
int hos_peft_logits(hos_peft*, const int32_t*, int, float*) { return HOS_E_INVALID; }
int hos_peft_profile(hos_peft*, int) { return HOS_E_INVALID; }
int hos_peft_kernel_stats(hos_peft*, const char*, long long*, double*, double*, double*) { return HOS_E_INVALID; }
}
