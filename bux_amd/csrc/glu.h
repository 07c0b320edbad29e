// The experts' gated activation, one unit at a time, shared by the activation kernels
// and the kernels that quantize their results on the fly: h = act(gate) (up + offset) w
// and its gradients (src/bux/architecture/experts/moe.py:898-926, layers/mlp.py:20-35,
// common/functional.py:12-40). float32 throughout; the callers round once to bfloat16.
#pragma once

#include "common.h"

namespace bux {

struct Act {
  int kind;     // BUX_SWISH or BUX_QUICK_GELU
  float limit;  // <= 0: no clamp
  float offset;
};

// The gate's activation a(g) and its derivative: g sigmoid(alpha g). jax multiplies
// the bfloat16 gate by quick_gelu's 1.702 as a bfloat16 constant, 1.703125. The sigmoid
// takes the hardware's 2^x and reciprocal (v_exp_f32, v_rcp_f32: a few float32 ulps,
// far inside the one rounding to bfloat16 that follows); the precise library exp and
// an IEEE division made the activation kernels VALU-bound (24% slower forward).
__device__ __forceinline__ void activate(int kind, float g, float* a, float* da) {
  const float alpha = kind == BUX_QUICK_GELU ? 1.703125f : 1.0f;
  const float s = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-alpha * g * 1.44269504f));
  *a = g * s;
  *da = s + alpha * g * s * (1.0f - s);
}

// h of one unit from its (up, gate) pair and the row's weight.
__device__ __forceinline__ float glu_unit(const Act& act, float up, float gate, float w) {
  if (act.limit > 0.0f) {
    up = fminf(fmaxf(up, -act.limit), act.limit);
    gate = fminf(gate, act.limit);
  }
  float a, da;
  activate(act.kind, gate, &a, &da);
  return a * (up + act.offset) * w;
}

// The gradients of one unit's h, given dh = g: to up and gate, and the unit's term of
// the row weight's gradient. clip's and minimum's gradients are jax's: 1 inside, 1/2 at
// the limit, 0 outside.
__device__ __forceinline__ void glu_unit_grad(const Act& act, float up, float gate, float w,
                                              float g, float* d_up, float* d_gate, float* d_w) {
  float up_pass = 1.0f, gate_pass = 1.0f;
  if (act.limit > 0.0f) {
    const float au = fabsf(up);
    up_pass = au < act.limit ? 1.0f : (au == act.limit ? 0.5f : 0.0f);
    gate_pass = gate < act.limit ? 1.0f : (gate == act.limit ? 0.5f : 0.0f);
    up = fminf(fmaxf(up, -act.limit), act.limit);
    gate = fminf(gate, act.limit);
  }
  float a, da;
  activate(act.kind, gate, &a, &da);
  const float uo = up + act.offset;
  *d_up = g * w * a * up_pass;
  *d_gate = g * w * uo * da * gate_pass;
  *d_w = g * a * uo;
}

}  // namespace bux
