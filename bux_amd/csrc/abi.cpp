// The library's error channel and version: a thread-local message behind each failed
// call's nonzero code.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>

#include "common.h"

namespace bux {

static thread_local char last_error[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list args;
  va_start(args, fmt);
  vsnprintf(last_error, sizeof(last_error), fmt, args);
  va_end(args);
  return code;
}

void clear_error() { last_error[0] = '\0'; }

int launched(const char* kernel) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return fail(BUX_E_LAUNCH, "%s: %s", kernel, hipGetErrorString(err));
  return BUX_OK;
}

}  // namespace bux

extern "C" const char* bux_last_error(void) { return bux::last_error; }

// 0.3.0: the float32 twins (bux_mx_quantize_f32, bux_glu_quantize_f32,
// bux_glu_backward_quantize_f32, bux_token_sums_f32) and bfloat16 GEMMs of any shape.
// 0.3.1: float32 twins of the bias ops (bux_expert_bias_add_f32, bux_expert_sums_f32,
// bux_token_sums_biased_f32, bux_expert_bias_weight_grad_f32) and of the expert norm
// (bux_expert_norm_forward_f32, bux_expert_norm_backward_f32).
// 0.3.2: float32 twins of the compute format's GEMMs (bux_bf16_grouped_rows_f32,
// bux_bf16_grouped_contract_f32) and of the activation (bux_glu_forward_f32,
// bux_glu_backward_f32): a float32 layer runs any pass outside MXFP8.
extern "C" int bux_version(void) { return 302; }
