// The token path's gathers and sums, and the experts' activation between the GEMMs.
//
//   token_rows  rows[i] = z[order[i] / k]           moe.py:991-1016, 1027-1032
//   token_sums  out[t] = sum_j y[inverse[t k + j]]  grouped_blockscaled.py:141-148,
//               in float32, picks in order, one rounding to bfloat16; an index outside
//               y's rows adds 0 (jnp.take's mode="fill").
//   glu         h = act(gate) (up + offset) w       moe.py:898-926, layers/mlp.py:20-35,
//               and its gradients                   common/functional.py:12-40
//
// All HBM-streaming: a lane moves 16 bytes (8 bfloat16) a load; a workgroup of 256
// lanes takes 2048 columns of a row. The activation computes in float32 and rounds
// once to bfloat16 (XLA fuses the elementwise chain and keeps float32 inside).

#include "common.h"
#include "glu.h"

namespace bux {
namespace {

constexpr int THREADS = 256;
constexpr int VEC = 8;  // bfloat16 a lane moves at once

__device__ __forceinline__ void unpack8(const uint4& r, float* v) {
  const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    v[2 * j] = bf16_to_f32(static_cast<uint16_t>(w[j] & 0xffffu));
    v[2 * j + 1] = bf16_to_f32(static_cast<uint16_t>(w[j] >> 16));
  }
}

__device__ __forceinline__ uint4 pack8(const float* v) {
  uint32_t w[4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
    w[j] = static_cast<uint32_t>(f32_to_bf16(v[2 * j])) |
           (static_cast<uint32_t>(f32_to_bf16(v[2 * j + 1])) << 16);
  return make_uint4(w[0], w[1], w[2], w[3]);
}

__global__ __launch_bounds__(THREADS) void token_rows_kernel(const uint16_t* __restrict__ z,
                                                             const int32_t* __restrict__ order,
                                                             int32_t k, int64_t width,
                                                             uint16_t* __restrict__ rows) {
  const int64_t chunks = (width + THREADS * VEC - 1) / (THREADS * VEC);
  const int64_t i = blockIdx.x / chunks;
  const int64_t c = ((blockIdx.x % chunks) * THREADS + threadIdx.x) * VEC;
  if (c >= width) return;
  const int64_t token = order[i] / k;
  *reinterpret_cast<uint4*>(rows + i * width + c) =
      *reinterpret_cast<const uint4*>(z + token * width + c);
}

// Rows narrower than a vector (a pick's weight, width 1): an element a lane.
__global__ __launch_bounds__(THREADS) void token_rows_narrow_kernel(
    const uint16_t* __restrict__ z, const int32_t* __restrict__ order, int64_t m, int32_t k,
    int64_t width, uint16_t* __restrict__ rows) {
  const int64_t e = static_cast<int64_t>(blockIdx.x) * THREADS + threadIdx.x;
  if (e >= m * width) return;
  const int64_t i = e / width, c = e % width;
  rows[e] = z[(order[i] / k) * width + c];
}

// KMAX > 0: the token's k <= KMAX picks' rows are all requested before the first is
// added (their indices first, then their rows); KMAX = 0: any k, one pick at a time.
// The additions are the same either way: picks in order, a row outside y skipped.
template <int KMAX>
__global__ __launch_bounds__(THREADS) void token_sums_kernel(const uint16_t* __restrict__ y,
                                                             int64_t y_rows,
                                                             const int32_t* __restrict__ inverse,
                                                             int32_t k, int64_t width,
                                                             uint16_t* __restrict__ out) {
  const int64_t chunks = (width + THREADS * VEC - 1) / (THREADS * VEC);
  const int64_t t = blockIdx.x / chunks;
  const int64_t c = ((blockIdx.x % chunks) * THREADS + threadIdx.x) * VEC;
  if (c >= width) return;
  float acc[VEC];
#pragma unroll
  for (int j = 0; j < VEC; ++j) acc[j] = 0.0f;
  if constexpr (KMAX > 0) {
    int64_t r[KMAX];
#pragma unroll
    for (int j = 0; j < KMAX; ++j) r[j] = j < k ? inverse[t * k + j] : -1;
    uint4 raw[KMAX];
#pragma unroll
    for (int j = 0; j < KMAX; ++j)
      raw[j] = (r[j] >= 0 && r[j] < y_rows) ? *reinterpret_cast<const uint4*>(y + r[j] * width + c)
                                            : make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int j = 0; j < KMAX; ++j) {
      if (r[j] < 0 || r[j] >= y_rows) continue;
      float v[VEC];
      unpack8(raw[j], v);
#pragma unroll
      for (int q = 0; q < VEC; ++q) acc[q] += v[q];
    }
  } else {
    for (int j = 0; j < k; ++j) {
      const int64_t r = inverse[t * k + j];
      if (r < 0 || r >= y_rows) continue;
      float v[VEC];
      unpack8(*reinterpret_cast<const uint4*>(y + r * width + c), v);
#pragma unroll
      for (int q = 0; q < VEC; ++q) acc[q] += v[q];
    }
  }
  *reinterpret_cast<uint4*>(out + t * width + c) = pack8(acc);
}

__global__ __launch_bounds__(THREADS) void glu_forward_kernel(
    const uint16_t* __restrict__ projected, const uint16_t* __restrict__ weights,
    const int32_t* __restrict__ filled_ptr, int64_t m, int64_t f, Act act,
    uint16_t* __restrict__ h) {
  // A lane takes 4 units (4 up-gate pairs, 16 bytes) of a row.
  const int64_t chunks = (f + THREADS * 4 - 1) / (THREADS * 4);
  const int64_t i = blockIdx.x / chunks;
  const int64_t u = ((blockIdx.x % chunks) * THREADS + threadIdx.x) * 4;
  if (u >= f) return;
  const int64_t filled = filled_ptr ? *filled_ptr : m;
  uint2 packed = make_uint2(0, 0);
  if (i < filled) {
    const uint4 r = *reinterpret_cast<const uint4*>(projected + (i * f + u) * 2);
    float p[8];
    unpack8(r, p);
    const float w = bf16_to_f32(weights[i]);
    float out[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) out[j] = glu_unit(act, p[2 * j], p[2 * j + 1], w);
    packed.x = f32_to_bf16(out[0]) | (static_cast<uint32_t>(f32_to_bf16(out[1])) << 16);
    packed.y = f32_to_bf16(out[2]) | (static_cast<uint32_t>(f32_to_bf16(out[3])) << 16);
  }
  *reinterpret_cast<uint2*>(h + i * f + u) = packed;
}

// One wave a row: d projected elementwise, d weight summed over the row's units.
__global__ __launch_bounds__(THREADS) void glu_backward_kernel(
    const uint16_t* __restrict__ projected, const uint16_t* __restrict__ weights,
    const uint16_t* __restrict__ dh, const int32_t* __restrict__ filled_ptr, int64_t m, int64_t f,
    Act act, uint16_t* __restrict__ d_projected, uint16_t* __restrict__ d_weights) {
  const int lane = threadIdx.x & 63;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * (THREADS / 64) + (threadIdx.x >> 6);
  if (i >= m) return;
  const int64_t filled = filled_ptr ? *filled_ptr : m;
  const bool live = i < filled;
  const float w = live ? bf16_to_f32(weights[i]) : 0.0f;
  float dw = 0.0f;
  for (int64_t u = 4 * lane; u < f; u += 256) {
    float p[8] = {0, 0, 0, 0, 0, 0, 0, 0}, g[4] = {0, 0, 0, 0};
    if (live) {
      unpack8(*reinterpret_cast<const uint4*>(projected + (i * f + u) * 2), p);
      const uint2 d = *reinterpret_cast<const uint2*>(dh + i * f + u);
      g[0] = bf16_to_f32(d.x & 0xffffu);
      g[1] = bf16_to_f32(d.x >> 16);
      g[2] = bf16_to_f32(d.y & 0xffffu);
      g[3] = bf16_to_f32(d.y >> 16);
    }
    float dp[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float term;
      glu_unit_grad(act, p[2 * j], p[2 * j + 1], w, g[j], &dp[2 * j], &dp[2 * j + 1], &term);
      dw += term;
    }
    *reinterpret_cast<uint4*>(d_projected + (i * f + u) * 2) = pack8(dp);
  }
#pragma unroll
  for (int s = 32; s >= 1; s >>= 1) dw += __shfl_xor(dw, s);
  if (lane == 0) d_weights[i] = f32_to_bf16(dw);
}

}  // namespace
}  // namespace bux

extern "C" int bux_token_rows(const uint16_t* z, const int32_t* order, int64_t m, int32_t k,
                              int64_t width, uint16_t* rows, void* stream) {
  using namespace bux;
  clear_error();
  BUX_CHECK(m >= 0 && m <= 2147483647LL && k >= 1 && width > 0,
            "bux_token_rows: bad shape m=%lld k=%d width=%lld", (long long)m, k, (long long)width);
  if (m == 0) return BUX_OK;
  BUX_CHECK(z && order && rows, "bux_token_rows: NULL buffer");
  if (width % VEC != 0) {
    BUX_CHECK(ceil_div(m * width, THREADS) < (1LL << 31), "bux_token_rows: too large");
    hipLaunchKernelGGL(token_rows_narrow_kernel, dim3(static_cast<unsigned>(ceil_div(m * width, THREADS))),
                       dim3(THREADS), 0, as_stream(stream), z, order, m, k, width, rows);
    return launched("token_rows_narrow_kernel");
  }
  BUX_CHECK(m * ceil_div(width, THREADS * VEC) < (1LL << 31), "bux_token_rows: too large");
  dim3 grid(static_cast<unsigned>(m * ceil_div(width, THREADS * VEC)));
  hipLaunchKernelGGL(token_rows_kernel, grid, dim3(THREADS), 0, as_stream(stream), z, order, k,
                     width, rows);
  return launched("token_rows_kernel");
}

extern "C" int bux_token_sums(const uint16_t* y, int64_t y_rows, const int32_t* inverse,
                              int64_t tokens, int32_t k, int64_t width, uint16_t* out,
                              void* stream) {
  using namespace bux;
  clear_error();
  BUX_CHECK(tokens >= 0 && tokens <= 2147483647LL && k >= 1 && width > 0 && y_rows >= 0,
            "bux_token_sums: bad shape tokens=%lld k=%d width=%lld", (long long)tokens, k,
            (long long)width);
  BUX_CHECK(width % VEC == 0, "bux_token_sums: width=%lld is not a multiple of %d",
            (long long)width, VEC);
  if (tokens == 0) return BUX_OK;
  BUX_CHECK(y && inverse && out, "bux_token_sums: NULL buffer");
  BUX_CHECK(tokens * ceil_div(width, THREADS * VEC) < (1LL << 31), "bux_token_sums: too large");
  dim3 grid(static_cast<unsigned>(tokens * ceil_div(width, THREADS * VEC)));
  if (k <= 8)
    hipLaunchKernelGGL(token_sums_kernel<8>, grid, dim3(THREADS), 0, as_stream(stream), y, y_rows,
                       inverse, k, width, out);
  else
    hipLaunchKernelGGL(token_sums_kernel<0>, grid, dim3(THREADS), 0, as_stream(stream), y, y_rows,
                       inverse, k, width, out);
  return launched("token_sums_kernel");
}

extern "C" int bux_glu_forward(const uint16_t* projected, const uint16_t* weights,
                               const int32_t* filled, int64_t m, int64_t f, int activation,
                               float limit, float up_offset, uint16_t* h, void* stream) {
  using namespace bux;
  clear_error();
  BUX_CHECK(m >= 0 && m <= 2147483647LL && f > 0 && f % 4 == 0,
            "bux_glu_forward: bad shape m=%lld f=%lld (f a multiple of 4)", (long long)m,
            (long long)f);
  BUX_CHECK(activation == BUX_SWISH || activation == BUX_QUICK_GELU,
            "bux_glu_forward: activation %d is neither BUX_SWISH nor BUX_QUICK_GELU", activation);
  if (m == 0) return BUX_OK;
  BUX_CHECK(projected && weights && h, "bux_glu_forward: NULL buffer");
  BUX_CHECK(m * ceil_div(f, THREADS * 4) < (1LL << 31), "bux_glu_forward: too large");
  dim3 grid(static_cast<unsigned>(m * ceil_div(f, THREADS * 4)));
  hipLaunchKernelGGL(glu_forward_kernel, grid, dim3(THREADS), 0, as_stream(stream), projected,
                     weights, filled, m, f, Act{activation, limit, up_offset}, h);
  return launched("glu_forward_kernel");
}

extern "C" int bux_glu_backward(const uint16_t* projected, const uint16_t* weights,
                                const uint16_t* dh, const int32_t* filled, int64_t m, int64_t f,
                                int activation, float limit, float up_offset,
                                uint16_t* d_projected, uint16_t* d_weights, void* stream) {
  using namespace bux;
  clear_error();
  BUX_CHECK(m >= 0 && m <= 2147483647LL && f > 0 && f % 4 == 0,
            "bux_glu_backward: bad shape m=%lld f=%lld (f a multiple of 4)", (long long)m,
            (long long)f);
  BUX_CHECK(activation == BUX_SWISH || activation == BUX_QUICK_GELU,
            "bux_glu_backward: activation %d is neither BUX_SWISH nor BUX_QUICK_GELU", activation);
  if (m == 0) return BUX_OK;
  BUX_CHECK(projected && weights && dh && d_projected && d_weights, "bux_glu_backward: NULL buffer");
  dim3 grid(static_cast<unsigned>(ceil_div(m, THREADS / 64)));
  hipLaunchKernelGGL(glu_backward_kernel, grid, dim3(THREADS), 0, as_stream(stream), projected,
                     weights, dh, filled, m, f, Act{activation, limit, up_offset}, d_projected,
                     d_weights);
  return launched("glu_backward_kernel");
}
