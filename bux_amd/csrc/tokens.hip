// The token path's gathers and sums, and the experts' activation between the GEMMs.
//
//   token_rows  rows[i] = z[order[i] / k]           moe.py:991-1016, 1027-1032
//               (a row of 0 where that row lies outside z, a negative index too: the
//               reference's orders never do, and no read leaves z)
//   token_sums  out[t] = sum_j y[inverse[t k + j]]  grouped_blockscaled.py:141-148,
//               in float32, picks in order, one rounding to bfloat16; an index outside
//               y's rows adds 0 (jnp.take's mode="fill").
//   glu         h = act(gate) (up + offset) w       moe.py:898-926, layers/mlp.py:20-35,
//               or act(up) w, and its gradients     common/functional.py:12-40
//   biases      the experts' up and down biases     moe.py:857-870, 876-885, 922-925
//               by expert, and their gradients
//
// All HBM-streaming: a lane moves 16 bytes (8 bfloat16) a load; a workgroup of 256
// lanes takes 2048 columns of a row. The activation computes in float32 and rounds
// once to bfloat16 (XLA fuses the elementwise chain and keeps float32 inside).

#include <type_traits>

#include "common.h"
#include "glu.h"

namespace bux {
namespace {

constexpr int THREADS = 256;
constexpr int VEC = 8;  // bfloat16 a lane moves at once

// 16 bytes of a row that this kernel alone reads, and once: the token sums' picked rows
// (each pick's row belongs to one token). Non-temporal loads: measured 10% faster at
// config 3's combines (0.116 -> 0.105 ms), where the picked rows were written just
// before by a GEMM; the other streaming kernels measured slower with them.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 read_once(const void* p) {
  const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return make_uint4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ float4 read_once_f(const void* p) {
  const uint4 v = read_once(p);
  return make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z),
                     __uint_as_float(v.w));
}

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

// Four bfloat16 to the low halves of four words (a plain unit's up where a gated
// unit's pair would be, its gate 0).
__device__ __forceinline__ uint4 spread4(const uint2& r) {
  return make_uint4(r.x & 0xffffu, r.x >> 16, r.y & 0xffffu, r.y >> 16);
}

// The row of z that pick `at` (an index entry) reads: at / k, or -1 (a row of 0) when
// that lies outside z's `tokens` rows, a negative entry included.
__device__ __forceinline__ int64_t source_row(int32_t at, int32_t k, int64_t tokens) {
  if (at < 0) return -1;
  const int64_t src = at / k;
  return src < tokens ? src : -1;
}

__global__ __launch_bounds__(THREADS) void token_rows_kernel(const uint16_t* __restrict__ z,
                                                             int64_t tokens,
                                                             const int32_t* __restrict__ order,
                                                             int32_t k, int64_t width,
                                                             uint16_t* __restrict__ rows) {
  const int64_t chunks = (width + THREADS * VEC - 1) / (THREADS * VEC);
  const int64_t i = blockIdx.x / chunks;
  const int64_t c = ((blockIdx.x % chunks) * THREADS + threadIdx.x) * VEC;
  if (c >= width) return;
  const int64_t token = source_row(order[i], k, tokens);
  *reinterpret_cast<uint4*>(rows + i * width + c) =
      token < 0 ? make_uint4(0, 0, 0, 0) : *reinterpret_cast<const uint4*>(z + token * width + c);
}

// Rows narrower than a vector (a pick's weight, width 1): an element a lane.
__global__ __launch_bounds__(THREADS) void token_rows_narrow_kernel(
    const uint16_t* __restrict__ z, int64_t tokens, const int32_t* __restrict__ order, int64_t m,
    int32_t k, int64_t width, uint16_t* __restrict__ rows) {
  const int64_t e = static_cast<int64_t>(blockIdx.x) * THREADS + threadIdx.x;
  if (e >= m * width) return;
  const int64_t i = e / width, c = e % width;
  const int64_t token = source_row(order[i], k, tokens);
  rows[e] = token < 0 ? uint16_t{0} : z[token * width + c];
}

// KMAX > 0: the token's k <= KMAX picks' rows are all requested before the first is
// added (their indices first, then their rows); KMAX = 0: any k, one pick at a time.
// The additions are the same either way: picks in order, a row outside y skipped.
// With BIAS, a second sum beside: each pick's bias[e(r)] * weights[r] (rounded to
// bfloat16), the picks of rows in no expert adding 0; out = the two sums, each rounded
// to bfloat16, added and rounded. T: the layer's element type.
template <typename T>
struct PickBias {
  const T* bias;
  const int32_t* offsets;
  int32_t experts;
  const T* weights;
};

template <int KMAX, bool BIAS>
__global__ __launch_bounds__(THREADS) void token_sums_kernel(const uint16_t* __restrict__ y,
                                                             int64_t y_rows,
                                                             const int32_t* __restrict__ inverse,
                                                             int32_t k, int64_t width,
                                                             PickBias<uint16_t> pb,
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
      raw[j] = (r[j] >= 0 && r[j] < y_rows) ? read_once(y + r[j] * width + c) : make_uint4(0, 0, 0, 0);
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
      unpack8(read_once(y + r * width + c), v);
#pragma unroll
      for (int q = 0; q < VEC; ++q) acc[q] += v[q];
    }
  }
  if constexpr (BIAS) {
    float bsum[VEC] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int j = 0; j < k; ++j) {
      const int64_t r = inverse[t * k + j];
      if (r < 0 || r >= y_rows) continue;
      const int32_t e = expert_of(pb.offsets, pb.experts, r);
      if (e < 0) continue;
      const float w = bf16_to_f32(pb.weights[r]);
      float b[VEC];
      unpack8(*reinterpret_cast<const uint4*>(pb.bias + e * width + c), b);
#pragma unroll
      for (int q = 0; q < VEC; ++q) bsum[q] += bf16_to_f32(f32_to_bf16(b[q] * w));
    }
#pragma unroll
    for (int q = 0; q < VEC; ++q)
      acc[q] = bf16_to_f32(f32_to_bf16(acc[q])) + bf16_to_f32(f32_to_bf16(bsum[q]));
  }
  *reinterpret_cast<uint4*>(out + t * width + c) = pack8(acc);
}

// token_sums_kernel for a layer in float32: float32 rows, the picks added in the same
// order, the float32 sum stored as it is (the reference's sum_by_token casts its float32
// sum back to y's dtype, grouped_blockscaled.py:148); with BIAS the picks' float32
// products bias[e(r)] * weights[r] summed beside and added. A lane moves 8 floats (32
// bytes) a pick.
template <int KMAX, bool BIAS>
__global__ __launch_bounds__(THREADS) void token_sums_f32_kernel(const float* __restrict__ y,
                                                                 int64_t y_rows,
                                                                 const int32_t* __restrict__ inverse,
                                                                 int32_t k, int64_t width,
                                                                 PickBias<float> pb,
                                                                 float* __restrict__ out) {
  // Each product rounds before it is added, as the reference's ops do (no FMA contraction).
#pragma clang fp contract(off)
  const int64_t chunks = (width + THREADS * VEC - 1) / (THREADS * VEC);
  const int64_t t = blockIdx.x / chunks;
  const int64_t c = ((blockIdx.x % chunks) * THREADS + threadIdx.x) * VEC;
  if (c >= width) return;
  float4 acc[2] = {make_float4(0, 0, 0, 0), make_float4(0, 0, 0, 0)};
  auto add = [&](const float4* row) {
    const float4 a = read_once_f(row), b = read_once_f(row + 1);
    acc[0].x += a.x; acc[0].y += a.y; acc[0].z += a.z; acc[0].w += a.w;
    acc[1].x += b.x; acc[1].y += b.y; acc[1].z += b.z; acc[1].w += b.w;
  };
  if constexpr (KMAX > 0) {
    int64_t r[KMAX];
#pragma unroll
    for (int j = 0; j < KMAX; ++j) r[j] = j < k ? inverse[t * k + j] : -1;
#pragma unroll
    for (int j = 0; j < KMAX; ++j)
      if (r[j] >= 0 && r[j] < y_rows) add(reinterpret_cast<const float4*>(y + r[j] * width + c));
  } else {
    for (int j = 0; j < k; ++j) {
      const int64_t r = inverse[t * k + j];
      if (r >= 0 && r < y_rows) add(reinterpret_cast<const float4*>(y + r * width + c));
    }
  }
  if constexpr (BIAS) {
    float bsum[VEC] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int j = 0; j < k; ++j) {
      const int64_t r = inverse[t * k + j];
      if (r < 0 || r >= y_rows) continue;
      const int32_t e = expert_of(pb.offsets, pb.experts, r);
      if (e < 0) continue;
      const float w = pb.weights[r];
      float b[VEC];
      Elem<float>::load8(pb.bias + e * width + c, b);
#pragma unroll
      for (int q = 0; q < VEC; ++q) bsum[q] += b[q] * w;
    }
    acc[0].x += bsum[0]; acc[0].y += bsum[1]; acc[0].z += bsum[2]; acc[0].w += bsum[3];
    acc[1].x += bsum[4]; acc[1].y += bsum[5]; acc[1].z += bsum[6]; acc[1].w += bsum[7];
  }
  float4* o = reinterpret_cast<float4*>(out + t * width + c);
  o[0] = acc[0];
  o[1] = acc[1];
}

// A row's 4 units from u on, as a lane takes them: gated, 8 values (4 up-gate pairs, up j
// at v[2 j]); plain, up j at v[2 j] and 0 beside it. T the layer's element type.
template <typename T, bool GATED>
__device__ __forceinline__ void load_units(const T* projected, int64_t i, int64_t f, int64_t u,
                                           float* v) {
  if constexpr (GATED) {
    Elem<T>::load8(projected + (i * f + u) * 2, v);
  } else if constexpr (std::is_same<T, float>::value) {
    const float4 r = *reinterpret_cast<const float4*>(projected + i * f + u);
    v[0] = r.x; v[2] = r.y; v[4] = r.z; v[6] = r.w;
    v[1] = v[3] = v[5] = v[7] = 0.0f;
  } else {
    unpack8(spread4(*reinterpret_cast<const uint2*>(projected + i * f + u)), v);
  }
}

// 4 values of a row (8 bytes of bfloat16, 16 of float32), stored or loaded.
__device__ __forceinline__ void store4(uint16_t* p, const float* v) {
  *reinterpret_cast<uint2*>(p) =
      make_uint2(f32_to_bf16(v[0]) | (static_cast<uint32_t>(f32_to_bf16(v[1])) << 16),
                 f32_to_bf16(v[2]) | (static_cast<uint32_t>(f32_to_bf16(v[3])) << 16));
}
__device__ __forceinline__ void store4(float* p, const float* v) {
  *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ void load4(const uint16_t* p, float* v) {
  const uint2 d = *reinterpret_cast<const uint2*>(p);
  v[0] = bf16_to_f32(d.x & 0xffffu);
  v[1] = bf16_to_f32(d.x >> 16);
  v[2] = bf16_to_f32(d.y & 0xffffu);
  v[3] = bf16_to_f32(d.y >> 16);
}
__device__ __forceinline__ void load4(const float* p, float* v) {
  const float4 d = *reinterpret_cast<const float4*>(p);
  v[0] = d.x; v[1] = d.y; v[2] = d.z; v[3] = d.w;
}

// A lane takes 4 units of a row: 16 bytes of projected gated (4 up-gate pairs), 8 plain
// (32 and 16 for float32). T the layer's element type: the activation computes in
// float32 and rounds once to T.
template <typename K, typename T>
__global__ __launch_bounds__(THREADS) void glu_forward_kernel(
    const T* __restrict__ projected, const T* __restrict__ weights,
    const int32_t* __restrict__ filled_ptr, int64_t m, int64_t f, Act act, T* __restrict__ h) {
  constexpr bool F32 = std::is_same<T, float>::value;
  const int64_t chunks = (f + THREADS * 4 - 1) / (THREADS * 4);
  const int64_t i = blockIdx.x / chunks;
  const int64_t u = ((blockIdx.x % chunks) * THREADS + threadIdx.x) * 4;
  if (u >= f) return;
  const int64_t filled = filled_ptr ? *filled_ptr : m;
  float out[4] = {0, 0, 0, 0};
  if (i < filled) {
    float p[8];
    load_units<T, K::gated>(projected, i, f, u, p);
    const float w = Elem<T>::value(weights[i]);
#pragma unroll
    for (int j = 0; j < 4; ++j) out[j] = glu_unit<K, F32>(act, p[2 * j], p[2 * j + 1], w);
  }
  store4(h + i * f + u, out);
}

// One wave a row: d projected elementwise, d weight summed over the row's units.
template <typename K, typename T>
__global__ __launch_bounds__(THREADS) void glu_backward_kernel(
    const T* __restrict__ projected, const T* __restrict__ weights, const T* __restrict__ dh,
    const int32_t* __restrict__ filled_ptr, int64_t m, int64_t f, Act act,
    T* __restrict__ d_projected, T* __restrict__ d_weights) {
  constexpr bool F32 = std::is_same<T, float>::value;
  const int lane = threadIdx.x & 63;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * (THREADS / 64) + (threadIdx.x >> 6);
  if (i >= m) return;
  const int64_t filled = filled_ptr ? *filled_ptr : m;
  const bool live = i < filled;
  const float w = live ? Elem<T>::value(weights[i]) : 0.0f;
  float dw = 0.0f;
  for (int64_t u = 4 * lane; u < f; u += 256) {
    float p[8] = {0, 0, 0, 0, 0, 0, 0, 0}, g[4] = {0, 0, 0, 0};
    if (live) {
      load_units<T, K::gated>(projected, i, f, u, p);
      load4(dh + i * f + u, g);
    }
    float dp[8] = {0, 0, 0, 0, 0, 0, 0, 0};  // rows past `filled`: +0 (not 0 x offset)
    if (live) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float term;
        glu_unit_grad<K, F32>(act, p[2 * j], p[2 * j + 1], w, g[j], &dp[2 * j], &dp[2 * j + 1],
                              &term);
        dw += term;
      }
    }
    if constexpr (K::gated) {
      Elem<T>::store8(d_projected + (i * f + u) * 2, dp);
    } else {
      const float up[4] = {dp[0], dp[2], dp[4], dp[6]};
      store4(d_projected + i * f + u, up);
    }
  }
#pragma unroll
  for (int s = 32; s >= 1; s >>= 1) dw += __shfl_xor(dw, s);
  if (lane == 0) d_weights[i] = Elem<T>::make(dw);
}

// --- The experts' biases --------------------------------------------------------------

// The bias kernels take the layer's element type T (uint16_t: bfloat16 bits, each op
// rounded to bfloat16; float: float32 ops).

// x[i] += bias[e(i)] in place, 8 columns a lane; rows in no expert add 0.
template <typename T>
__global__ __launch_bounds__(THREADS) void expert_bias_add_kernel(
    T* __restrict__ x, int64_t width, const T* __restrict__ bias,
    const int32_t* __restrict__ offsets, int32_t experts) {
  using E = Elem<T>;
  const int64_t chunks = (width + THREADS * VEC - 1) / (THREADS * VEC);
  const int64_t i = blockIdx.x / chunks;
  const int64_t c = ((blockIdx.x % chunks) * THREADS + threadIdx.x) * VEC;
  if (c >= width) return;
  const int32_t e = expert_of(offsets, experts, i);
  float v[VEC], b[VEC] = {0, 0, 0, 0, 0, 0, 0, 0};
  T* at = x + i * width + c;
  E::load8(at, v);
  if (e >= 0) E::load8(bias + e * width + c, b);
#pragma unroll
  for (int q = 0; q < VEC; ++q) v[q] += b[q];
  E::store8(at, v);
}

// out[e] = sum over e's rows of v_r (x[src(r)], times weights[r] rounded to T if
// weights). Workgroup (e, column chunk): wave w adds rows w, w + 4, ... of e in order,
// lanes 8 columns each; the four waves' sums are added in wave order. Deterministic.
constexpr int SUM_COLS = 64 * VEC;  // a workgroup's columns
template <typename T>
__global__ __launch_bounds__(THREADS) void expert_sums_kernel(
    const T* __restrict__ x, const int32_t* __restrict__ index, int32_t index_div,
    int64_t sources, const T* __restrict__ weights, int64_t m, int64_t width,
    const int32_t* __restrict__ offsets, int32_t experts, float* __restrict__ out) {
  // Each product rounds before it is added, as the reference's ops do (no FMA contraction).
#pragma clang fp contract(off)
  using E = Elem<T>;
  __shared__ float part[THREADS / 64][SUM_COLS];
  const int64_t chunks = (width + SUM_COLS - 1) / SUM_COLS;
  const int64_t e = blockIdx.x / chunks;
  const int64_t c0 = (blockIdx.x % chunks) * SUM_COLS;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t c = c0 + lane * VEC;
  // rows inside [0, m) only, whatever the offsets say
  const int64_t lo = offsets[e] > 0 ? offsets[e] : 0;
  const int64_t hi = offsets[e + 1] < m ? offsets[e + 1] : m;
  float acc[VEC] = {0, 0, 0, 0, 0, 0, 0, 0};
  if (c < width) {
    for (int64_t r = lo + wave; r < hi; r += THREADS / 64) {
      const int64_t src = index ? source_row(index[r], index_div, sources) : r;
      if (src < 0) continue;  // a row of 0
      float v[VEC];
      E::load8(x + src * width + c, v);
      if (weights) {
        const float w = E::value(weights[r]);
#pragma unroll
        for (int q = 0; q < VEC; ++q) v[q] = E::round(v[q] * w);
      }
#pragma unroll
      for (int q = 0; q < VEC; ++q) acc[q] += v[q];
    }
  }
#pragma unroll
  for (int q = 0; q < VEC; ++q) part[wave][lane * VEC + q] = acc[q];
  __syncthreads();
  // thread t: column t and t + 256 of the chunk
  for (int j = threadIdx.x; j < SUM_COLS; j += THREADS) {
    const int64_t col = c0 + j;
    if (col >= width) continue;
    float sum = part[0][j];
#pragma unroll
    for (int w = 1; w < THREADS / 64; ++w) sum += part[w][j];
    out[e * width + col] = sum;
  }
}

// d_weights[r] += sum_c dy[src(r)][c] bias[e(r)][c]: one wave a row, lanes 8 columns a
// step, each lane's products (rounded to T) in column order, then the lanes by
// xor-shuffles; the sum rounded to T, added and rounded.
template <typename T>
__global__ __launch_bounds__(THREADS) void expert_bias_weight_grad_kernel(
    const T* __restrict__ dy, const int32_t* __restrict__ index, int32_t index_div,
    int64_t sources, int64_t m, int64_t width, const T* __restrict__ bias,
    const int32_t* __restrict__ offsets, int32_t experts, T* __restrict__ d_weights) {
  // Each product rounds before it is added, as the reference's ops do (no FMA contraction).
#pragma clang fp contract(off)
  using E = Elem<T>;
  const int lane = threadIdx.x & 63;
  const int64_t r = static_cast<int64_t>(blockIdx.x) * (THREADS / 64) + (threadIdx.x >> 6);
  if (r >= m) return;
  const int32_t e = expert_of(offsets, experts, r);
  float sum = 0.0f;
  const int64_t src = e < 0 ? -1 : index ? source_row(index[r], index_div, sources) : r;
  if (src >= 0) {
    for (int64_t c = lane * VEC; c < width; c += 64 * VEC) {
      float g[VEC], b[VEC];
      E::load8(dy + src * width + c, g);
      E::load8(bias + e * width + c, b);
#pragma unroll
      for (int q = 0; q < VEC; ++q) sum += E::round(g[q] * b[q]);
    }
  }
#pragma unroll
  for (int s = 32; s >= 1; s >>= 1) sum += __shfl_xor(sum, s);
  if (lane == 0) d_weights[r] = E::make(E::value(d_weights[r]) + E::round(sum));
}

}  // namespace
}  // namespace bux

extern "C" int bux_token_rows(const uint16_t* z, int64_t tokens, const int32_t* order, int64_t m,
                              int32_t k, int64_t width, uint16_t* rows, void* stream) {
  using namespace bux;
  clear_error();
  BUX_CHECK(m >= 0 && m <= 2147483647LL && k >= 1 && width > 0 && tokens >= 0,
            "bux_token_rows: bad shape tokens=%lld m=%lld k=%d width=%lld", (long long)tokens,
            (long long)m, k, (long long)width);
  if (m == 0) return BUX_OK;
  BUX_CHECK(z && order && rows, "bux_token_rows: NULL buffer");
  if (width % VEC != 0) {
    BUX_CHECK(ceil_div(m * width, THREADS) < (1LL << 31), "bux_token_rows: too large");
    hipLaunchKernelGGL(token_rows_narrow_kernel, dim3(static_cast<unsigned>(ceil_div(m * width, THREADS))),
                       dim3(THREADS), 0, as_stream(stream), z, tokens, order, m, k, width, rows);
    return launched("token_rows_narrow_kernel");
  }
  BUX_CHECK(m * ceil_div(width, THREADS * VEC) < (1LL << 31), "bux_token_rows: too large");
  dim3 grid(static_cast<unsigned>(m * ceil_div(width, THREADS * VEC)));
  hipLaunchKernelGGL(token_rows_kernel, grid, dim3(THREADS), 0, as_stream(stream), z, tokens,
                     order, k, width, rows);
  return launched("token_rows_kernel");
}

namespace bux {
namespace {
int token_sums(const char* name, const uint16_t* y, int64_t y_rows, const int32_t* inverse,
               int64_t tokens, int32_t k, int64_t width, const PickBias<uint16_t>* pb,
               uint16_t* out, void* stream) {
  BUX_CHECK(tokens >= 0 && tokens <= 2147483647LL && k >= 1 && width > 0 && y_rows >= 0,
            "%s: bad shape tokens=%lld k=%d width=%lld", name, (long long)tokens, k,
            (long long)width);
  BUX_CHECK(width % VEC == 0, "%s: width=%lld is not a multiple of %d", name, (long long)width,
            VEC);
  if (tokens == 0) return BUX_OK;
  BUX_CHECK(y && inverse && out, "%s: NULL buffer", name);
  BUX_CHECK(tokens * ceil_div(width, THREADS * VEC) < (1LL << 31), "%s: too large", name);
  dim3 grid(static_cast<unsigned>(tokens * ceil_div(width, THREADS * VEC)));
  const PickBias<uint16_t> none{nullptr, nullptr, 0, nullptr};
  hipStream_t s = as_stream(stream);
  if (pb)
    hipLaunchKernelGGL((token_sums_kernel<0, true>), grid, dim3(THREADS), 0, s, y, y_rows,
                       inverse, k, width, *pb, out);
  else if (k <= 8)
    hipLaunchKernelGGL((token_sums_kernel<8, false>), grid, dim3(THREADS), 0, s, y, y_rows,
                       inverse, k, width, none, out);
  else
    hipLaunchKernelGGL((token_sums_kernel<0, false>), grid, dim3(THREADS), 0, s, y, y_rows,
                       inverse, k, width, none, out);
  return launched("token_sums_kernel");
}

int token_sums_f32(const char* name, const float* y, int64_t y_rows, const int32_t* inverse,
                   int64_t tokens, int32_t k, int64_t width, const PickBias<float>* pb,
                   float* out, void* stream) {
  BUX_CHECK(tokens >= 0 && tokens <= 2147483647LL && k >= 1 && width > 0 && y_rows >= 0,
            "%s: bad shape tokens=%lld k=%d width=%lld", name, (long long)tokens, k,
            (long long)width);
  BUX_CHECK(width % VEC == 0, "%s: width=%lld is not a multiple of %d", name, (long long)width,
            VEC);
  if (tokens == 0) return BUX_OK;
  BUX_CHECK(y && inverse && out, "%s: NULL buffer", name);
  BUX_CHECK(tokens * ceil_div(width, THREADS * VEC) < (1LL << 31), "%s: too large", name);
  dim3 grid(static_cast<unsigned>(tokens * ceil_div(width, THREADS * VEC)));
  hipStream_t s = as_stream(stream);
  const PickBias<float> none{nullptr, nullptr, 0, nullptr};
  if (pb)
    hipLaunchKernelGGL((token_sums_f32_kernel<0, true>), grid, dim3(THREADS), 0, s, y, y_rows,
                       inverse, k, width, *pb, out);
  else if (k <= 8)
    hipLaunchKernelGGL((token_sums_f32_kernel<8, false>), grid, dim3(THREADS), 0, s, y, y_rows,
                       inverse, k, width, none, out);
  else
    hipLaunchKernelGGL((token_sums_f32_kernel<0, false>), grid, dim3(THREADS), 0, s, y, y_rows,
                       inverse, k, width, none, out);
  return launched("token_sums_f32_kernel");
}

int experts_ok(const char* name, const int32_t* offsets, int32_t experts) {
  BUX_CHECK(offsets != nullptr && experts >= 1 && experts <= (1 << 20),
            "%s: offsets of %d experts (1 .. 2^20, not NULL)", name, experts);
  return BUX_OK;
}

template <typename T>
int bias_add(const char* name, T* x, int64_t m, int64_t width, const T* bias,
             const int32_t* offsets, int32_t experts, void* stream) {
  BUX_CHECK(m >= 0 && width > 0 && width % VEC == 0,
            "%s: bad shape m=%lld width=%lld (a multiple of %d)", name, (long long)m,
            (long long)width, VEC);
  if (int rc = experts_ok(name, offsets, experts)) return rc;
  if (m == 0) return BUX_OK;
  BUX_CHECK(x && bias, "%s: NULL buffer", name);
  BUX_CHECK(m * ceil_div(width, THREADS * VEC) < (1LL << 31), "%s: too large", name);
  dim3 grid(static_cast<unsigned>(m * ceil_div(width, THREADS * VEC)));
  hipLaunchKernelGGL(expert_bias_add_kernel<T>, grid, dim3(THREADS), 0, as_stream(stream), x,
                     width, bias, offsets, experts);
  return launched("expert_bias_add_kernel");
}

template <typename T>
int expert_sums(const char* name, const T* x, const int32_t* index, int32_t index_div,
                int64_t sources, const T* weights, int64_t m, int64_t width,
                const int32_t* offsets, int32_t experts, float* out, void* stream) {
  BUX_CHECK(m >= 0 && width > 0 && width % VEC == 0,
            "%s: bad shape m=%lld width=%lld (a multiple of %d)", name, (long long)m,
            (long long)width, VEC);
  BUX_CHECK(index == nullptr || index_div >= 1, "%s: index_div=%d", name, index_div);
  BUX_CHECK(index == nullptr || sources >= 0, "%s: sources=%lld", name, (long long)sources);
  if (int rc = experts_ok(name, offsets, experts)) return rc;
  BUX_CHECK(out != nullptr && (m == 0 || x != nullptr), "%s: NULL buffer", name);
  // every expert's sum is written (0 for none); rows at or past m add nothing
  const int64_t chunks = ceil_div(width, SUM_COLS);
  BUX_CHECK(experts * chunks < (1LL << 31), "%s: too large", name);
  hipLaunchKernelGGL(expert_sums_kernel<T>, dim3(static_cast<unsigned>(experts * chunks)),
                     dim3(THREADS), 0, as_stream(stream), x, index, index_div, sources, weights,
                     m, width, offsets, experts, out);
  return launched("expert_sums_kernel");
}

template <typename T>
int bias_weight_grad(const char* name, const T* dy, const int32_t* index, int32_t index_div,
                     int64_t sources, int64_t m, int64_t width, const T* bias,
                     const int32_t* offsets, int32_t experts, T* d_weights, void* stream) {
  BUX_CHECK(m >= 0 && width > 0 && width % VEC == 0,
            "%s: bad shape m=%lld width=%lld (a multiple of %d)", name, (long long)m,
            (long long)width, VEC);
  BUX_CHECK(index == nullptr || index_div >= 1, "%s: index_div=%d", name, index_div);
  BUX_CHECK(index == nullptr || sources >= 0, "%s: sources=%lld", name, (long long)sources);
  if (int rc = experts_ok(name, offsets, experts)) return rc;
  if (m == 0) return BUX_OK;
  BUX_CHECK(dy && bias && d_weights, "%s: NULL buffer", name);
  hipLaunchKernelGGL(expert_bias_weight_grad_kernel<T>,
                     dim3(static_cast<unsigned>(ceil_div(m, THREADS / 64))), dim3(THREADS), 0,
                     as_stream(stream), dy, index, index_div, sources, m, width, bias, offsets,
                     experts, d_weights);
  return launched("expert_bias_weight_grad_kernel");
}
}  // namespace
}  // namespace bux

extern "C" int bux_token_sums(const uint16_t* y, int64_t y_rows, const int32_t* inverse,
                              int64_t tokens, int32_t k, int64_t width, uint16_t* out,
                              void* stream) {
  using namespace bux;
  clear_error();
  return token_sums("bux_token_sums", y, y_rows, inverse, tokens, k, width, nullptr, out, stream);
}

extern "C" int bux_token_sums_f32(const float* y, int64_t y_rows, const int32_t* inverse,
                                  int64_t tokens, int32_t k, int64_t width, float* out,
                                  void* stream) {
  using namespace bux;
  clear_error();
  return token_sums_f32("bux_token_sums_f32", y, y_rows, inverse, tokens, k, width, nullptr, out,
                        stream);
}

extern "C" int bux_token_sums_biased(const uint16_t* y, int64_t y_rows, const int32_t* inverse,
                                     int64_t tokens, int32_t k, int64_t width,
                                     const uint16_t* bias, const int32_t* offsets,
                                     int32_t experts, const uint16_t* weights, uint16_t* out,
                                     void* stream) {
  using namespace bux;
  clear_error();
  if (int rc = experts_ok("bux_token_sums_biased", offsets, experts)) return rc;
  BUX_CHECK(tokens == 0 || (bias && weights), "bux_token_sums_biased: NULL bias or weights");
  const PickBias<uint16_t> pb{bias, offsets, experts, weights};
  return token_sums("bux_token_sums_biased", y, y_rows, inverse, tokens, k, width, &pb, out,
                    stream);
}

extern "C" int bux_token_sums_biased_f32(const float* y, int64_t y_rows, const int32_t* inverse,
                                         int64_t tokens, int32_t k, int64_t width,
                                         const float* bias, const int32_t* offsets,
                                         int32_t experts, const float* weights, float* out,
                                         void* stream) {
  using namespace bux;
  clear_error();
  if (int rc = experts_ok("bux_token_sums_biased_f32", offsets, experts)) return rc;
  BUX_CHECK(tokens == 0 || (bias && weights), "bux_token_sums_biased_f32: NULL bias or weights");
  const PickBias<float> pb{bias, offsets, experts, weights};
  return token_sums_f32("bux_token_sums_biased_f32", y, y_rows, inverse, tokens, k, width, &pb,
                        out, stream);
}

extern "C" int bux_expert_bias_add(uint16_t* x, int64_t m, int64_t width, const uint16_t* bias,
                                   const int32_t* offsets, int32_t experts, void* stream) {
  bux::clear_error();
  return bux::bias_add("bux_expert_bias_add", x, m, width, bias, offsets, experts, stream);
}

extern "C" int bux_expert_bias_add_f32(float* x, int64_t m, int64_t width, const float* bias,
                                       const int32_t* offsets, int32_t experts, void* stream) {
  bux::clear_error();
  return bux::bias_add("bux_expert_bias_add_f32", x, m, width, bias, offsets, experts, stream);
}

extern "C" int bux_expert_sums(const uint16_t* x, const int32_t* index, int32_t index_div,
                               int64_t sources, const uint16_t* weights, int64_t m,
                               int64_t width, const int32_t* offsets, int32_t experts,
                               float* out, void* stream) {
  bux::clear_error();
  return bux::expert_sums("bux_expert_sums", x, index, index_div, sources, weights, m, width,
                          offsets, experts, out, stream);
}

extern "C" int bux_expert_sums_f32(const float* x, const int32_t* index, int32_t index_div,
                                   int64_t sources, const float* weights, int64_t m,
                                   int64_t width, const int32_t* offsets, int32_t experts,
                                   float* out, void* stream) {
  bux::clear_error();
  return bux::expert_sums("bux_expert_sums_f32", x, index, index_div, sources, weights, m, width,
                          offsets, experts, out, stream);
}

extern "C" int bux_expert_bias_weight_grad(const uint16_t* dy, const int32_t* index,
                                           int32_t index_div, int64_t sources, int64_t m,
                                           int64_t width, const uint16_t* bias,
                                           const int32_t* offsets, int32_t experts,
                                           uint16_t* d_weights, void* stream) {
  bux::clear_error();
  return bux::bias_weight_grad("bux_expert_bias_weight_grad", dy, index, index_div, sources, m,
                               width, bias, offsets, experts, d_weights, stream);
}

extern "C" int bux_expert_bias_weight_grad_f32(const float* dy, const int32_t* index,
                                               int32_t index_div, int64_t sources, int64_t m,
                                               int64_t width, const float* bias,
                                               const int32_t* offsets, int32_t experts,
                                               float* d_weights, void* stream) {
  bux::clear_error();
  return bux::bias_weight_grad("bux_expert_bias_weight_grad_f32", dy, index, index_div, sources,
                               m, width, bias, offsets, experts, d_weights, stream);
}

namespace bux {
namespace {
template <typename T>
int glu_forward(const char* name, const T* projected, const T* weights, const int32_t* filled,
                int64_t m, int64_t f, const bux_ffn* ffn, T* h, void* stream) {
  BUX_CHECK(m >= 0 && m <= 2147483647LL && f > 0 && f % 4 == 0,
            "%s: bad shape m=%lld f=%lld (f a multiple of 4)", name, (long long)m, (long long)f);
  Act act;
  if (int rc = act_of(name, ffn, &act)) return rc;
  if (m == 0) return BUX_OK;
  BUX_CHECK(projected && weights && h, "%s: NULL buffer", name);
  BUX_CHECK(m * ceil_div(f, THREADS * 4) < (1LL << 31), "%s: too large", name);
  dim3 grid(static_cast<unsigned>(m * ceil_div(f, THREADS * 4)));
  return with_kind(act, [&](auto kind) {
    hipLaunchKernelGGL((glu_forward_kernel<decltype(kind), T>), grid, dim3(THREADS), 0,
                       as_stream(stream), projected, weights, filled, m, f, act, h);
    return launched("glu_forward_kernel");
  });
}

template <typename T>
int glu_backward(const char* name, const T* projected, const T* weights, const T* dh,
                 const int32_t* filled, int64_t m, int64_t f, const bux_ffn* ffn, T* d_projected,
                 T* d_weights, void* stream) {
  BUX_CHECK(m >= 0 && m <= 2147483647LL && f > 0 && f % 4 == 0,
            "%s: bad shape m=%lld f=%lld (f a multiple of 4)", name, (long long)m, (long long)f);
  Act act;
  if (int rc = act_of(name, ffn, &act)) return rc;
  if (m == 0) return BUX_OK;
  BUX_CHECK(projected && weights && dh && d_projected && d_weights, "%s: NULL buffer", name);
  dim3 grid(static_cast<unsigned>(ceil_div(m, THREADS / 64)));
  return with_kind(act, [&](auto kind) {
    hipLaunchKernelGGL((glu_backward_kernel<decltype(kind), T>), grid, dim3(THREADS), 0,
                       as_stream(stream), projected, weights, dh, filled, m, f, act, d_projected,
                       d_weights);
    return launched("glu_backward_kernel");
  });
}
}  // namespace
}  // namespace bux

extern "C" int bux_glu_forward(const uint16_t* projected, const uint16_t* weights,
                               const int32_t* filled, int64_t m, int64_t f, const bux_ffn* ffn,
                               uint16_t* h, void* stream) {
  bux::clear_error();
  return bux::glu_forward("bux_glu_forward", projected, weights, filled, m, f, ffn, h, stream);
}

extern "C" int bux_glu_forward_f32(const float* projected, const float* weights,
                                   const int32_t* filled, int64_t m, int64_t f,
                                   const bux_ffn* ffn, float* h, void* stream) {
  bux::clear_error();
  return bux::glu_forward("bux_glu_forward_f32", projected, weights, filled, m, f, ffn, h, stream);
}

extern "C" int bux_glu_backward(const uint16_t* projected, const uint16_t* weights,
                                const uint16_t* dh, const int32_t* filled, int64_t m, int64_t f,
                                const bux_ffn* ffn, uint16_t* d_projected, uint16_t* d_weights,
                                void* stream) {
  bux::clear_error();
  return bux::glu_backward("bux_glu_backward", projected, weights, dh, filled, m, f, ffn,
                           d_projected, d_weights, stream);
}

extern "C" int bux_glu_backward_f32(const float* projected, const float* weights,
                                    const float* dh, const int32_t* filled, int64_t m, int64_t f,
                                    const bux_ffn* ffn, float* d_projected, float* d_weights,
                                    void* stream) {
  bux::clear_error();
  return bux::glu_backward("bux_glu_backward_f32", projected, weights, dh, filled, m, f, ffn,
                           d_projected, d_weights, stream);
}
