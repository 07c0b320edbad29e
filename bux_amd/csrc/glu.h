// The experts' activation, one unit at a time, shared by the activation kernels and
// the kernels that quantize their results on the fly: the reference's `activate`
// (src/bux/architecture/layers/mlp.py:20-35) of `activation` (common/functional.py:
// 12-40), times each row's weight (experts/moe.py:898-926). float32 throughout; the
// callers round once to bfloat16.
//
//   gated (gated_mlp):  h = a(min(gate, limit)) (cap(clip(up)) + up_offset) w
//   plain (mlp):        h = a(cap(clip(up))) w
//
// with clip(u) = u clipped to [-limit, limit] when clamped and cap(u) = c tanh(u / c)
// when soft-capped (up_softcap = c).
#pragma once

#include "common.h"

namespace bux {

struct Act {
  int kind;      // BUX_SWISH .. BUX_SITU
  int gated;     // act(gate) (up + offset), else act(up)
  int clamped;   // `limit` clips up to [-limit, limit] and the gate from above
  float limit;
  int capped;    // up = cap tanh(up / cap), after the clip
  float cap;
  float offset;  // added to the up branch of a gated unit
};

// The activation and gating as compile-time constants: each kernel is built once per
// pair, so that the units a lane computes interleave with no branch between them.
template <int KIND, bool GATED>
struct Kind {
  static constexpr int kind = KIND;
  static constexpr bool gated = GATED;
};

// Floating-point contraction: every function here fuses a * b + c into one FMA exactly
// where one expression holds it (contract(on), decided by the source), never by the
// code generator's choice, which may differ from one kernel to another: the plain, the
// quantizing and the fused GEMM-epilogue kernels inline these functions and must agree
// bit for bit. Their products do not fuse into a caller's sums either.
constexpr float LOG2E = 1.44269504088896341f;

// The hardware's 2^x and reciprocal (v_exp_f32, v_rcp_f32): a few float32 ulps, far
// inside the one rounding to bfloat16 that follows. (The library's precise exp and an
// IEEE division made the activation kernels VALU-bound, 24% slower for SwiGLU.)
__device__ __forceinline__ float fast_sigmoid(float x) {
#pragma clang fp contract(on)
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-x * LOG2E));
}
// tanh(x): below |x| = 1/8 its Taylor series to x^7 (the next term, 62 x^9 / 2835, is
// under 2e-9 of tanh there), else 1 - 2 / (e^{2x} + 1), +-1 where e^{2x} over- or
// underflows, a float32 ulp of 1 from exact (under 1e-6 of tanh from |x| = 1/8 on).
// Both forms are computed and one selected: no branch.
__device__ __forceinline__ float fast_tanh(float x) {
#pragma clang fp contract(on)
  const float x2 = x * x;
  const float series =
      x * (1.0f + x2 * (-1.0f / 3.0f + x2 * (2.0f / 15.0f - x2 * (17.0f / 315.0f))));
  const float far =
      1.0f - 2.0f * __builtin_amdgcn_rcpf(__builtin_amdgcn_exp2f(2.0f * x * LOG2E) + 1.0f);
  return fabsf(x) < 0.125f ? series : far;
}

// The activation a(x) and its derivative a'(x) (functional.py:12-40, their gradients
// as jax takes them: relu's is 0 at 0). F32: a layer in float32, whose weakly typed
// constants jax takes in float32.
template <int KIND, bool F32 = false>
__device__ __forceinline__ void activate(float x, float* a, float* da) {
#pragma clang fp contract(on)
  if constexpr (KIND == BUX_RELU) {
    *a = x > 0.0f ? x : 0.0f;
    *da = x > 0.0f ? 1.0f : 0.0f;
  } else if constexpr (KIND == BUX_RELU2) {
    const float r = x > 0.0f ? x : 0.0f;
    *a = r * r;
    *da = 2.0f * r;
  } else if constexpr (KIND == BUX_GELU) {
    // x Phi(x), Phi(x) = erfc(-x / sqrt 2) / 2 (1 + erf(x / sqrt 2) would cancel below
    // x = -4); Phi' = exp(-x^2 / 2) / sqrt(2 pi)
    const float phi = 0.5f * erfcf(-x * 0.70710678118654752f);
    *a = x * phi;
    *da = phi + x * 0.39894228040143268f * __builtin_amdgcn_exp2f(-0.5f * x * x * LOG2E);
  } else if constexpr (KIND == BUX_GELU_TANH) {
    // x (1 + tanh(z)) / 2, z = c (x + 0.044715 x^3), c = sqrt(2 / pi); 1 + tanh(z) taken
    // as 2 sigmoid(2 z), which does not cancel where tanh(z) nears -1:
    // a = x s, a' = s + 2 x s (1 - s) z', s = sigmoid(2 z)
    const float c = 0.79788456080286536f;
    const float s = fast_sigmoid(2.0f * c * (x + 0.044715f * x * x * x));
    *a = x * s;
    *da = s + 2.0f * x * s * (1.0f - s) * c * (1.0f + 3.0f * 0.044715f * x * x);
  } else if constexpr (KIND == BUX_SIGMOID) {
    const float s = fast_sigmoid(x);
    *a = s;
    *da = s * (1.0f - s);
  } else if constexpr (KIND == BUX_TANH) {
    const float t = fast_tanh(x);
    *a = t;
    *da = 1.0f - t * t;
  } else if constexpr (KIND == BUX_SOFTPLUS) {
    // log(1 + e^x) = max(x, 0) + log1p(e^-|x|), precise: far below 0 it is e^x itself
    *a = fmaxf(x, 0.0f) + log1pf(expf(-fabsf(x)));
    *da = fast_sigmoid(x);
  } else if constexpr (KIND == BUX_SITU) {
    // 4 tanh(x / 4) sigmoid(x)
    const float t = fast_tanh(0.25f * x), s = fast_sigmoid(x);
    *a = 4.0f * t * s;
    *da = (1.0f - t * t) * s + 4.0f * t * s * (1.0f - s);
  } else {
    static_assert(KIND == BUX_SWISH || KIND == BUX_QUICK_GELU, "no such activation");
    // swish: x sigmoid(x); quick_gelu: x sigmoid(1.702 x), jax multiplying the
    // bfloat16 gate by 1.702 as a bfloat16 constant, 1.703125 (a float32 gate by
    // 1.702's float32)
    constexpr float alpha = KIND == BUX_QUICK_GELU ? (F32 ? 1.702f : 1.703125f) : 1.0f;
    const float s = fast_sigmoid(alpha * x);
    *a = x * s;
    *da = s + alpha * x * s * (1.0f - s);
  }
}

// The up branch after its clip and soft cap, and its derivative to the up projection.
// clip is maximum, then minimum, and jax's gradient of each is 1/2 at a tie: 1 inside,
// 1/2 at the limit, 0 outside; at a limit of 0 an up of 0 ties both, 1/4.
__device__ __forceinline__ float up_branch(const Act& act, float up, float* dup) {
#pragma clang fp contract(on)
  float d = 1.0f;
  if (act.clamped) {
    const float au = fabsf(up);
    d = au < act.limit ? 1.0f : (au == act.limit ? (act.limit == 0.0f ? 0.25f : 0.5f) : 0.0f);
    up = fminf(fmaxf(up, -act.limit), act.limit);
  }
  if (act.capped) {
    const float t = fast_tanh(up / act.cap);
    d *= 1.0f - t * t;
    up = act.cap * t;
  }
  *dup = d;
  return up;
}

// h of one unit from its up projection (and gate, when gated) and the row's weight.
template <typename K, bool F32 = false>
__device__ __forceinline__ float glu_unit(const Act& act, float up, float gate, float w) {
#pragma clang fp contract(on)
  float dup, a, da;
  up = up_branch(act, up, &dup);
  if constexpr (!K::gated) {
    activate<K::kind, F32>(up, &a, &da);
    return a * w;
  } else {
    if (act.clamped) gate = fminf(gate, act.limit);
    activate<K::kind, F32>(gate, &a, &da);
    return a * (up + act.offset) * w;
  }
}

// The gradients of one unit's h, given dh = g: to up and (gated) gate, and the unit's
// term of the row weight's gradient.
template <typename K, bool F32 = false>
__device__ __forceinline__ void glu_unit_grad(const Act& act, float up, float gate, float w,
                                              float g, float* d_up, float* d_gate, float* d_w) {
#pragma clang fp contract(on)
  float dup, a, da;
  up = up_branch(act, up, &dup);
  if constexpr (!K::gated) {
    activate<K::kind, F32>(up, &a, &da);
    *d_up = g * w * da * dup;
    *d_gate = 0.0f;
    *d_w = g * a;
  } else {
    float gate_pass = 1.0f;
    if (act.clamped) {
      gate_pass = gate < act.limit ? 1.0f : (gate == act.limit ? 0.5f : 0.0f);
      gate = fminf(gate, act.limit);
    }
    activate<K::kind, F32>(gate, &a, &da);
    const float uo = up + act.offset;
    *d_up = g * w * a * dup;
    *d_gate = g * w * uo * da * gate_pass;
    *d_w = g * a * uo;
  }
}

// d weight of each of m rows from its `tiles` partial sums (one a 64 columns of d
// projected, rows past *filled 0), added in order and rounded once to bfloat16
// (quantize.hip's glu_weights_kernel).
int launch_glu_weights(const float* partials, int64_t m, int64_t tiles, const int32_t* filled,
                       uint16_t* d_weights, hipStream_t s);

// Calls f(Kind<act.kind, act.gated>{}) and returns what it returns.
template <int KIND, typename F>
int with_gating(const Act& act, F&& f) {
  return act.gated ? f(Kind<KIND, true>{}) : f(Kind<KIND, false>{});
}
template <typename F>
int with_kind(const Act& act, F&& f) {
  switch (act.kind) {
    case BUX_SWISH: return with_gating<BUX_SWISH>(act, f);
    case BUX_QUICK_GELU: return with_gating<BUX_QUICK_GELU>(act, f);
    case BUX_RELU: return with_gating<BUX_RELU>(act, f);
    case BUX_RELU2: return with_gating<BUX_RELU2>(act, f);
    case BUX_GELU: return with_gating<BUX_GELU>(act, f);
    case BUX_GELU_TANH: return with_gating<BUX_GELU_TANH>(act, f);
    case BUX_SIGMOID: return with_gating<BUX_SIGMOID>(act, f);
    case BUX_TANH: return with_gating<BUX_TANH>(act, f);
    case BUX_SOFTPLUS: return with_gating<BUX_SOFTPLUS>(act, f);
    default: return with_gating<BUX_SITU>(act, f);
  }
}

// The expert of sorted row i: the e with offsets[e] <= i < offsets[e + 1] (`experts` + 1
// nondecreasing offsets, bux_moe_permute's); -1 from offsets[experts] on.
__device__ __forceinline__ int32_t expert_of(const int32_t* __restrict__ offsets, int32_t experts,
                                             int64_t i) {
  if (i >= offsets[experts]) return -1;
  int32_t lo = 0, hi = experts;  // offsets[lo] <= i < offsets[hi]
  while (hi - lo > 1) {
    const int32_t mid = (lo + hi) >> 1;
    if (offsets[mid] <= i) lo = mid;
    else hi = mid;
  }
  return lo;
}

// The host's view of the activation, bux_ffn (include/bux_amd.h), checked.
inline int act_of(const char* name, const bux_ffn* ffn, Act* act) {
  if (ffn == nullptr) return fail(BUX_E_ARGUMENT, "%s: NULL ffn", name);
  if (ffn->activation < BUX_SWISH || ffn->activation > BUX_SITU)
    return fail(BUX_E_ARGUMENT, "%s: activation %d is none of BUX_SWISH .. BUX_SITU", name,
                ffn->activation);
  if (ffn->clamped && !(ffn->limit >= 0.0f))
    return fail(BUX_E_ARGUMENT, "%s: limit %g: a clamp's limit is at least 0", name, ffn->limit);
  if (ffn->capped && !(ffn->up_softcap > 0.0f))
    return fail(BUX_E_ARGUMENT, "%s: up_softcap %g: a soft cap is above 0", name,
                ffn->up_softcap);
  *act = Act{ffn->activation, ffn->gated != 0, ffn->clamped != 0, ffn->limit, ffn->capped != 0,
             ffn->up_softcap, ffn->up_offset};
  return BUX_OK;
}

}  // namespace bux
