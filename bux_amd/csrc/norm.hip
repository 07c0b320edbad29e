// The per-expert norm of the experts' outputs (experts/moe.py:871-872):
//
//   out[r] = weighted(norm(y[r] + down_bias[e(r)]), w[r])
//
// with the reference's Norm (layers/norm.py:14-78) in the tokens' dtype, bfloat16 (the
// model's parameters cast to it, train/trainer.py:129-140) or float32 (the _f32 entry
// points: every rounding below is then float32 arithmetic's own): gain = scale, or 1 + scale when
// zero-centered (rounded); with scale_input x = x * gain first; the statistics in float32
// (layernorm: x - mean(x), then times rsqrt(mean(x^2) + eps); rmsnorm: the second alone),
// the result rounded to bfloat16; then times the gain and plus the bias, each rounded;
// then times the row's weight, rounded. Every rounding the reference's bfloat16 ops make
// is made here, at the same place; the float32 sums are in another order.
//
// The backward is the VJP jax takes of that chain, in the same dtypes: the rows' upstream
// gradient is their token's (dy read by index), dn = g w; the weight's gradient the sum
// of g n; through the bias and gain (their gradients summed over the rows), the
// normalization's VJP in float32, and scale_input's gain. Rows in no expert (past the
// groups: the picks outside the experts, whose weights the layer zeroes) give 0.
//
// Forward: a workgroup a row, the row in registers (d <= 8192: 8 values a thread a 2048
// chunk), block sums through LDS. Backward: a workgroup takes ROWS rows one after another,
// each thread the same columns of every row, so that it adds its columns' gain and bias
// gradients over the rows in registers; one float32 partial a workgroup and column goes
// to the workspace, and norm_params_kernel adds the partials in workgroup order.

#include "common.h"
#include "glu.h"

namespace bux {
namespace {

constexpr int THREADS = 256;
constexpr int VEC = 8;
constexpr int MAX_CHUNKS = 4;  // d <= MAX_CHUNKS * THREADS * VEC = 8192
constexpr int ROWS = 64;       // rows a backward workgroup

// The sum of v over the workgroup (256 threads); `red` 4 floats of LDS. Every thread
// gets it; the LDS is free again when it returns.
__device__ __forceinline__ float block_sum(float v, float* red) {
#pragma unroll
  for (int s = 32; s >= 1; s >>= 1) v += __shfl_xor(v, s);
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[wave] = v;
  __syncthreads();
  const float t = (red[0] + red[1]) + (red[2] + red[3]);
  __syncthreads();
  return t;
}

// T: the layer's element type (uint16_t: bfloat16 bits; float).
template <typename T>
struct NormArgs {
  int kind;  // BUX_LAYERNORM or BUX_RMSNORM
  int affine, zero_centered, scale_input, biased;
  float eps;
  const T* scale;      // [d], or NULL (not affine)
  const T* bias;       // [d], or NULL
  const T* down_bias;  // [experts, d] or NULL
  const int32_t* offsets;
  int32_t experts;
};

// One thread's share of a row: columns c(i) = (i * THREADS + threadIdx.x) * VEC + j.
struct Row {
  float v[MAX_CHUNKS][VEC];
};

// The row's values through the norm's input side: y + down bias, rounded; with
// scale_input, times the gain, rounded (`in` before it, `x` after). Columns past d: 0.
template <typename T>
__device__ __forceinline__ void norm_input(const NormArgs<T>& a, const T* y_row, int32_t e,
                                           int64_t d, Row& in, Row& x, Row& gain) {
  // Each product rounds before it is added, as the reference's ops do (no FMA contraction).
#pragma clang fp contract(off)
  using E = Elem<T>;
#pragma unroll
  for (int i = 0; i < MAX_CHUNKS; ++i) {  // every chunk: past d, zeros
    const int64_t c = (static_cast<int64_t>(i) * THREADS + threadIdx.x) * VEC;
    float yv[VEC] = {0, 0, 0, 0, 0, 0, 0, 0}, b[VEC] = {0, 0, 0, 0, 0, 0, 0, 0};
    float s[VEC] = {1, 1, 1, 1, 1, 1, 1, 1};
    if (c < d) {
      E::load8(y_row + c, yv);
      if (a.down_bias) E::load8(a.down_bias + e * d + c, b);
      if (a.affine) E::load8(a.scale + c, s);
    }
#pragma unroll
    for (int j = 0; j < VEC; ++j) {
      const float g = a.affine && a.zero_centered ? E::round(1.0f + s[j]) : s[j];
      gain.v[i][j] = g;
      const float v = a.down_bias ? E::round(yv[j] + b[j]) : yv[j];
      in.v[i][j] = c < d ? v : 0.0f;
      x.v[i][j] = c < d ? (a.affine && a.scale_input ? E::round(v * g) : v) : 0.0f;
    }
  }
}

// mean (layernorm, else 0) and rsqrt(mean((x - mean)^2) + eps) of the row, float32.
template <typename T>
__device__ __forceinline__ void norm_stats(const NormArgs<T>& a, const Row& x, int64_t d, int chunks,
                                           float* red, float* mean, float* rs) {
  // Each product rounds before it is added, as the reference's ops do (no FMA contraction).
#pragma clang fp contract(off)
  float m = 0.0f;
  if (a.kind == BUX_LAYERNORM) {
    float t = 0.0f;
#pragma unroll
    for (int i = 0; i < MAX_CHUNKS; ++i)
#pragma unroll
      for (int j = 0; j < VEC; ++j) t += x.v[i][j];  // columns past d hold 0
    m = block_sum(t, red) / static_cast<float>(d);
  }
  float q = 0.0f;
#pragma unroll
  for (int i = 0; i < MAX_CHUNKS; ++i) {
    if (i >= chunks) break;
    const int64_t c = (static_cast<int64_t>(i) * THREADS + threadIdx.x) * VEC;
#pragma unroll
    for (int j = 0; j < VEC; ++j) {
      const float u = c + j < d ? x.v[i][j] - m : 0.0f;
      q += u * u;
    }
  }
  *mean = m;
  *rs = rsqrtf(block_sum(q, red) / static_cast<float>(d) + a.eps);
}

template <typename T>
__global__ __launch_bounds__(THREADS) void norm_forward_kernel(
    const T* __restrict__ y, int64_t d, NormArgs<T> a, const T* __restrict__ weights,
    T* __restrict__ out) {
  // Each product rounds before it is added, as the reference's ops do (no FMA contraction).
#pragma clang fp contract(off)
  using E = Elem<T>;
  __shared__ float red[4];
  const int64_t r = blockIdx.x;
  const int chunks = static_cast<int>((d + THREADS * VEC - 1) / (THREADS * VEC));
  const int32_t e = expert_of(a.offsets, a.experts, r);
  T* o = out + r * d;
  if (e < 0) {  // a row in no expert: 0 (a uniform branch: the whole workgroup's row)
    const float z[VEC] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < MAX_CHUNKS; ++i) {
      if (i >= chunks) break;
      const int64_t c = (static_cast<int64_t>(i) * THREADS + threadIdx.x) * VEC;
      if (c < d) E::store8(o + c, z);
    }
    return;
  }
  Row in, x, gain;
  norm_input(a, y + r * d, e, d, in, x, gain);
  float mean, rs;
  norm_stats(a, x, d, chunks, red, &mean, &rs);
  const float w = E::value(weights[r]);
#pragma unroll
  for (int i = 0; i < MAX_CHUNKS; ++i) {
    if (i >= chunks) break;
    const int64_t c = (static_cast<int64_t>(i) * THREADS + threadIdx.x) * VEC;
    if (c >= d) continue;
    float b[VEC] = {0, 0, 0, 0, 0, 0, 0, 0}, v[VEC];
    if (a.biased) E::load8(a.bias + c, b);
#pragma unroll
    for (int j = 0; j < VEC; ++j) {
      float n = E::round((x.v[i][j] - mean) * rs);
      if (a.affine && !a.scale_input) n = E::round(n * gain.v[i][j]);
      if (a.biased) n = E::round(n + b[j]);
      v[j] = n * w;
    }
    E::store8(o + c, v);
  }
}

// A workgroup takes rows [blockIdx.x ROWS, + ROWS): dv and the weights' gradient a row,
// and its columns' gain and bias gradients summed over its rows into partials[2][block][d].
template <typename T>
__global__ __launch_bounds__(THREADS) void norm_backward_kernel(
    const T* __restrict__ dy, const int32_t* __restrict__ index, int32_t index_div,
    int64_t sources, const T* __restrict__ y, int64_t m, int64_t d, NormArgs<T> a,
    const T* __restrict__ weights, T* __restrict__ dv, T* __restrict__ d_weights,
    float* __restrict__ partials) {
  // Each product rounds before it is added, as the reference's ops do (no FMA contraction).
#pragma clang fp contract(off)
  using E = Elem<T>;
  __shared__ float red[4];
  const int chunks = static_cast<int>((d + THREADS * VEC - 1) / (THREADS * VEC));
  Row d_gain, d_bias;
#pragma unroll
  for (int i = 0; i < MAX_CHUNKS; ++i)
#pragma unroll
    for (int j = 0; j < VEC; ++j) d_gain.v[i][j] = d_bias.v[i][j] = 0.0f;
  const int64_t r0 = static_cast<int64_t>(blockIdx.x) * ROWS;
  for (int64_t r = r0; r < r0 + ROWS && r < m; ++r) {
    const int32_t e = expert_of(a.offsets, a.experts, r);
    T* o = dv + r * d;
    if (e < 0) {  // uniform: the whole workgroup's row
      const float z[VEC] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
      for (int i = 0; i < MAX_CHUNKS; ++i) {
        if (i >= chunks) break;
        const int64_t c = (static_cast<int64_t>(i) * THREADS + threadIdx.x) * VEC;
        if (c < d) E::store8(o + c, z);
      }
      if (threadIdx.x == 0) d_weights[r] = E::make(0.0f);
      continue;
    }
    Row in, x, gain;
    norm_input(a, y + r * d, e, d, in, x, gain);
    float mean, rs;
    norm_stats(a, x, d, chunks, red, &mean, &rs);
    const float w = E::value(weights[r]);
    // dy's row: r, or by index (a row of 0 where that lies outside dy's sources rows)
    const int64_t src =
        index ? (index[r] < 0 ? -1 : static_cast<int64_t>(index[r] / index_div)) : r;
    const bool g_live = src >= 0 && (index == nullptr || src < sources);
    const T* g_row = dy + (g_live ? src : 0) * d;
    // dn = g w; the weight's gradient sum_c g n (products rounded, as T's ops);
    // dxn = dn (times the gain); and the two sums the normalization's VJP takes
    Row dxn;
    float wsum = 0.0f, s1 = 0.0f, s2 = 0.0f;
#pragma unroll
    for (int i = 0; i < MAX_CHUNKS; ++i) {
      if (i >= chunks) break;
      const int64_t c = (static_cast<int64_t>(i) * THREADS + threadIdx.x) * VEC;
      float g[VEC] = {0, 0, 0, 0, 0, 0, 0, 0}, b[VEC] = {0, 0, 0, 0, 0, 0, 0, 0};
      if (c < d) {
        if (g_live) E::load8(g_row + c, g);
        if (a.biased) E::load8(a.bias + c, b);
      }
#pragma unroll
      for (int j = 0; j < VEC; ++j) {
        const bool inside = c + j < d;
        const float u = x.v[i][j] - mean;
        const float xn = E::round(u * rs);  // the normalization's output
        float n = xn;
        if (a.affine && !a.scale_input) n = E::round(n * gain.v[i][j]);
        if (a.biased) n = E::round(n + b[j]);
        wsum += inside ? E::round(g[j] * n) : 0.0f;
        const float dn = E::round(g[j] * w);
        d_bias.v[i][j] += inside ? dn : 0.0f;
        float dx = dn;
        if (a.affine && !a.scale_input) {
          d_gain.v[i][j] += inside ? E::round(dn * xn) : 0.0f;
          dx = E::round(dn * gain.v[i][j]);
        }
        dxn.v[i][j] = inside ? dx : 0.0f;
        s1 += inside ? dx : 0.0f;
        s2 += inside ? dx * u : 0.0f;
      }
    }
    const float sum_w = block_sum(wsum, red);
    const float mean_dx = a.kind == BUX_LAYERNORM ? block_sum(s1, red) / static_cast<float>(d) : 0.0f;
    const float mean_dxu = block_sum(s2, red) / static_cast<float>(d);
    if (threadIdx.x == 0) d_weights[r] = E::make(sum_w);
#pragma unroll
    for (int i = 0; i < MAX_CHUNKS; ++i) {
      if (i >= chunks) break;
      const int64_t c = (static_cast<int64_t>(i) * THREADS + threadIdx.x) * VEC;
      if (c >= d) continue;
      float out[VEC];
#pragma unroll
      for (int j = 0; j < VEC; ++j) {
        const float u = x.v[i][j] - mean;
        // d x = rs (dxn - mean(dxn) - u rs^2 mean(dxn u)); rmsnorm: mean(dxn) left out
        float dx1 = E::round(rs * (dxn.v[i][j] - mean_dx - u * rs * rs * mean_dxu));
        if (a.affine && a.scale_input) {
          d_gain.v[i][j] += E::round(dx1 * in.v[i][j]);
          dx1 = E::round(dx1 * gain.v[i][j]);
        }
        out[j] = dx1;
      }
      E::store8(o + c, out);
    }
  }
  // this workgroup's column sums
  float* pg = partials + static_cast<int64_t>(blockIdx.x) * d;
  float* pb = partials + (static_cast<int64_t>(gridDim.x) + blockIdx.x) * d;
#pragma unroll
  for (int i = 0; i < MAX_CHUNKS; ++i) {
    if (i >= chunks) break;
    const int64_t c = (static_cast<int64_t>(i) * THREADS + threadIdx.x) * VEC;
    if (c >= d) continue;
#pragma unroll
    for (int j = 0; j < VEC; ++j) {
      pg[c + j] = d_gain.v[i][j];
      pb[c + j] = d_bias.v[i][j];
    }
  }
}

// d_gain[c] and d_bias[c]: the workgroups' partials added in workgroup order.
__global__ __launch_bounds__(THREADS) void norm_params_kernel(const float* __restrict__ partials,
                                                              int64_t blocks, int64_t d,
                                                              float* __restrict__ d_gain,
                                                              float* __restrict__ d_bias) {
  const int64_t c = static_cast<int64_t>(blockIdx.x) * THREADS + threadIdx.x;
  if (c >= d) return;
  float g = 0.0f, b = 0.0f;
  for (int64_t k = 0; k < blocks; ++k) {
    g += partials[k * d + c];
    b += partials[(blocks + k) * d + c];
  }
  if (d_gain) d_gain[c] = g;
  if (d_bias) d_bias[c] = b;
}

template <typename T>
int norm_args(const char* name, const bux_norm* norm, const T* scale, const T* bias,
              const T* down_bias, const int32_t* offsets, int32_t experts, NormArgs<T>* a) {
  if (norm == nullptr) return fail(BUX_E_ARGUMENT, "%s: NULL norm", name);
  if (norm->kind != BUX_LAYERNORM && norm->kind != BUX_RMSNORM)
    return fail(BUX_E_ARGUMENT, "%s: kind %d is neither BUX_LAYERNORM nor BUX_RMSNORM", name,
                norm->kind);
  if (!(norm->eps >= 0.0f)) return fail(BUX_E_ARGUMENT, "%s: eps %g", name, norm->eps);
  if (norm->affine && scale == nullptr) return fail(BUX_E_ARGUMENT, "%s: an affine norm needs its scale", name);
  if (norm->bias && bias == nullptr) return fail(BUX_E_ARGUMENT, "%s: a biased norm needs its bias", name);
  if (offsets == nullptr || experts < 1 || experts > (1 << 20))
    return fail(BUX_E_ARGUMENT, "%s: offsets of %d experts (1 .. 2^20, not NULL)", name, experts);
  *a = NormArgs<T>{norm->kind, norm->affine != 0, norm->zero_centered != 0, norm->scale_input != 0,
                   norm->bias != 0, norm->eps, scale, bias, down_bias, offsets, experts};
  return BUX_OK;
}

int norm_shape(const char* name, int64_t m, int64_t d) {
  BUX_CHECK(m >= 0 && m < (1LL << 31) && d > 0 && d % VEC == 0 && d <= MAX_CHUNKS * THREADS * VEC,
            "%s: bad shape m=%lld d=%lld (d a multiple of %d, at most %d)", name, (long long)m,
            (long long)d, VEC, MAX_CHUNKS * THREADS * VEC);
  return BUX_OK;
}

template <typename T>
int norm_forward(const char* name, const T* y, int64_t m, int64_t d, const T* down_bias,
                 const int32_t* offsets, int32_t experts, const bux_norm* norm, const T* scale,
                 const T* bias, const T* weights, T* out, void* stream) {
  if (int rc = norm_shape(name, m, d)) return rc;
  NormArgs<T> a;
  if (int rc = norm_args(name, norm, scale, bias, down_bias, offsets, experts, &a)) return rc;
  if (m == 0) return BUX_OK;
  BUX_CHECK(y && weights && out, "%s: NULL buffer", name);
  hipLaunchKernelGGL(norm_forward_kernel<T>, dim3(static_cast<unsigned>(m)), dim3(THREADS), 0,
                     as_stream(stream), y, d, a, weights, out);
  return launched("norm_forward_kernel");
}

size_t backward_workspace(int64_t m, int64_t d) {
  return static_cast<size_t>(2 * ceil_div(m, ROWS) * d) * sizeof(float);
}

template <typename T>
int norm_backward(const char* name, const T* dy, const int32_t* index, int32_t index_div,
                  int64_t sources, const T* y, int64_t m, int64_t d, const T* down_bias,
                  const int32_t* offsets, int32_t experts, const bux_norm* norm, const T* scale,
                  const T* bias, const T* weights, T* dv, T* d_weights, float* d_scale,
                  float* d_bias, void* workspace, size_t workspace_bytes, void* stream) {
  if (int rc = norm_shape(name, m, d)) return rc;
  BUX_CHECK(index == nullptr || index_div >= 1, "%s: index_div=%d", name, index_div);
  BUX_CHECK(index == nullptr || sources >= 0, "%s: sources=%lld", name, (long long)sources);
  NormArgs<T> a;
  if (int rc = norm_args(name, norm, scale, bias, down_bias, offsets, experts, &a)) return rc;
  BUX_CHECK((!a.affine || d_scale) && (!a.biased || d_bias),
            "%s: NULL d_scale or d_bias for a norm that has them", name);
  const size_t need = backward_workspace(m, d);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need))
    return fail(BUX_E_WORKSPACE, "%s: workspace of %zu bytes, %zu needed", name, workspace_bytes,
                need);
  hipStream_t s = as_stream(stream);
  const int64_t blocks = ceil_div(m, ROWS);
  if (m > 0) {
    BUX_CHECK(dy && y && weights && dv && d_weights, "%s: NULL buffer", name);
    hipLaunchKernelGGL(norm_backward_kernel<T>, dim3(static_cast<unsigned>(blocks)), dim3(THREADS),
                       0, s, dy, index, index_div, sources, y, m, d, a, weights, dv, d_weights,
                       static_cast<float*>(workspace));
    if (int rc = launched("norm_backward_kernel")) return rc;
  }
  if (!a.affine && !a.biased) return BUX_OK;
  // with no rows, the sums are 0: a workspace of no partials
  hipLaunchKernelGGL(norm_params_kernel, dim3(static_cast<unsigned>(ceil_div(d, THREADS))),
                     dim3(THREADS), 0, s, static_cast<const float*>(workspace), blocks, d,
                     a.affine ? d_scale : nullptr, a.biased ? d_bias : nullptr);
  return launched("norm_params_kernel");
}

}  // namespace
}  // namespace bux

extern "C" int bux_expert_norm_forward(const uint16_t* y, int64_t m, int64_t d,
                                       const uint16_t* down_bias, const int32_t* offsets,
                                       int32_t experts, const bux_norm* norm,
                                       const uint16_t* scale, const uint16_t* bias,
                                       const uint16_t* weights, uint16_t* out, void* stream) {
  bux::clear_error();
  return bux::norm_forward("bux_expert_norm_forward", y, m, d, down_bias, offsets, experts, norm,
                           scale, bias, weights, out, stream);
}

extern "C" int bux_expert_norm_forward_f32(const float* y, int64_t m, int64_t d,
                                           const float* down_bias, const int32_t* offsets,
                                           int32_t experts, const bux_norm* norm,
                                           const float* scale, const float* bias,
                                           const float* weights, float* out, void* stream) {
  bux::clear_error();
  return bux::norm_forward("bux_expert_norm_forward_f32", y, m, d, down_bias, offsets, experts,
                           norm, scale, bias, weights, out, stream);
}

extern "C" size_t bux_expert_norm_backward_workspace_size(int64_t m, int64_t d) {
  return bux::backward_workspace(m, d);
}

extern "C" int bux_expert_norm_backward(const uint16_t* dy, const int32_t* index, int32_t index_div,
                                        int64_t sources, const uint16_t* y, int64_t m, int64_t d,
                                        const uint16_t* down_bias, const int32_t* offsets,
                                        int32_t experts, const bux_norm* norm,
                                        const uint16_t* scale, const uint16_t* bias,
                                        const uint16_t* weights, uint16_t* dv,
                                        uint16_t* d_weights, float* d_scale, float* d_bias,
                                        void* workspace, size_t workspace_bytes, void* stream) {
  bux::clear_error();
  return bux::norm_backward("bux_expert_norm_backward", dy, index, index_div, sources, y, m, d,
                            down_bias, offsets, experts, norm, scale, bias, weights, dv,
                            d_weights, d_scale, d_bias, workspace, workspace_bytes, stream);
}

extern "C" int bux_expert_norm_backward_f32(const float* dy, const int32_t* index,
                                            int32_t index_div, int64_t sources, const float* y,
                                            int64_t m, int64_t d, const float* down_bias,
                                            const int32_t* offsets, int32_t experts,
                                            const bux_norm* norm, const float* scale,
                                            const float* bias, const float* weights, float* dv,
                                            float* d_weights, float* d_scale, float* d_bias,
                                            void* workspace, size_t workspace_bytes,
                                            void* stream) {
  bux::clear_error();
  return bux::norm_backward("bux_expert_norm_backward_f32", dy, index, index_div, sources, y, m,
                            d, down_bias, offsets, experts, norm, scale, bias, weights, dv,
                            d_weights, d_scale, d_bias, workspace, workspace_bytes, stream);
}
