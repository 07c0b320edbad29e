// MXFP8 as rows of bytes, what an expert-parallel dispatch sends: each token quantized
// along its width in blocks of 32 (the a-4 spec) and written as one row of d + d/32
// bytes, its E4M3 codes then its scales' E8M0 bytes; and back, each row dequantized to
// bfloat16.
//
//   pack    packed[i] = mx_packed(mx_quantize(x[index[i] / div]))   experts.py:624, 659-663,
//           (x[i] without an index)                                 blockscaled.py:372-375
//   unpack  out[i] = bf16(dequantized(mx_unpacked(packed[i], d)))   experts.py:666-672,
//                                                                   blockscaled.py:223-229,
//                                                                   378-380
//
// pack: a lane takes a block of 32 values, 64 bytes of bfloat16 in (four 16-byte
// loads), 32 codes and a scale byte out; a wave takes 64 blocks of a row, a workgroup 4
// waves. Quantizing a token once per pick rather than once gives the same bytes (the
// quantizer is a function of the row) and reads the token's further copies from L2.
// (Four lanes a block, each load and store one run, measured slower here: 4 code and 4
// scale stores a row where this form has 2 and 1.)
// unpack: four neighbouring lanes take a block, a lane 8 codes in and 16 bytes of
// bfloat16 out; a wave takes 16 consecutive blocks at a time, so that each load and
// store moves one run (512 bytes of codes, 1 KiB of bfloat16), 4 such runs with their
// loads in flight together. Unpacking is exact: a code times a power of two holds in float32 and, with
// at most 4 significant bits, in bfloat16 (a product past float32's range is inf in
// both, as the reference's float32 product is). HBM-bound.

#include "common.h"

namespace bux {
namespace {

constexpr int THREADS = 256;

__device__ __forceinline__ void unpack8(const uint4& r, float* v) {
  const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    v[2 * j] = bf16_to_f32(static_cast<uint16_t>(w[j] & 0xffffu));
    v[2 * j + 1] = bf16_to_f32(static_cast<uint16_t>(w[j] >> 16));
  }
}

// Stores `bytes` (a multiple of 4) from `src` words at `dst`, 16 bytes at a time where
// both row alignment allows (`align` 16), else 4.
template <int ALIGN>
__device__ __forceinline__ void store_words(uint8_t* dst, const uint32_t* w, int words) {
  if (ALIGN == 16) {
    for (int i = 0; i < words; i += 4)
      *reinterpret_cast<uint4*>(dst + 4 * i) = make_uint4(w[i], w[i + 1], w[i + 2], w[i + 3]);
  } else if (ALIGN == 4) {
    for (int i = 0; i < words; ++i) *reinterpret_cast<uint32_t*>(dst + 4 * i) = w[i];
  } else {
    for (int i = 0; i < 4 * words; ++i) dst[i] = static_cast<uint8_t>(w[i / 4] >> (8 * (i % 4)));
  }
}

// ALIGN: the byte alignment every packed row starts at (16, 4 or 1).
template <int ALIGN>
__global__ __launch_bounds__(THREADS) void pack_kernel(const uint16_t* __restrict__ x,
                                                       const int32_t* __restrict__ index,
                                                       int32_t div, int64_t n, int64_t m,
                                                       int64_t d, uint8_t* __restrict__ packed) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * (THREADS / 64) + (threadIdx.x >> 6);
  if (i >= m) return;
  // a negative index reads zeros, as one past x does (C's division would take -1 / k
  // to row 0)
  const int64_t src = index ? (index[i] < 0 ? -1 : index[i] / div) : i;
  const bool live = src >= 0 && src < n;
  const int64_t blocks = d / 32, row_bytes = d + blocks;
  uint8_t* out = packed + i * row_bytes;
  for (int64_t b = threadIdx.x & 63; b < blocks; b += 64) {
    float v[32];
    if (live) {
      const uint4* p = reinterpret_cast<const uint4*>(x + src * d + 32 * b);
#pragma unroll
      for (int q = 0; q < 4; ++q) unpack8(p[q], v + 8 * q);
    } else {
#pragma unroll
      for (int j = 0; j < 32; ++j) v[j] = 0.0f;
    }
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < 32; ++j) amax = fmaxf(amax, fabsf(v[j]));
    const int e = scale_exponent_bf16(amax);
    const float down = power_of_two_down(e);
    uint32_t w[8];
#pragma unroll
    for (int j = 0; j < 8; ++j)
      w[j] = e4m3x4(clip448(v[4 * j] * down), clip448(v[4 * j + 1] * down),
                    clip448(v[4 * j + 2] * down), clip448(v[4 * j + 3] * down));
    store_words<ALIGN>(out + 32 * b, w, 8);
    out[d + b] = static_cast<uint8_t>(e + 127);
  }
}

// A wave takes RUNS runs of 16 blocks, one after another in memory, their loads issued
// together: run r (of the m rows' ceil(d / 512) runs each) is row r / runs_a_row, blocks
// 16 (r % runs_a_row) on; lane l takes block l / 4 of it (`on`: the block is in the
// row), values 8 (l % 4) .. of the block.
constexpr int RUNS = 4;
struct Run {
  int64_t row, b;
  int q;
  bool on;
};
__device__ __forceinline__ Run run_of(int64_t m, int64_t blocks, int j) {
  const int64_t runs_a_row = (blocks + 15) / 16;
  const int64_t wave = static_cast<int64_t>(blockIdx.x) * (THREADS / 64) + (threadIdx.x >> 6);
  const int64_t r = wave * RUNS + j;
  const int lane = threadIdx.x & 63;
  Run u;
  u.row = r / runs_a_row;
  u.b = (r % runs_a_row) * 16 + (lane >> 2);
  u.q = lane & 3;
  u.on = u.row < m && u.b < blocks;
  return u;
}

// 8 bytes of a packed row at `p`, which is 8-byte aligned when the rows start
// ALIGN-aligned (16), else 4-aligned (4) or not (1).
template <int ALIGN>
__device__ __forceinline__ uint2 load8(const uint8_t* p) {
  if (ALIGN == 16) return *reinterpret_cast<const uint2*>(p);
  if (ALIGN == 4) return make_uint2(reinterpret_cast<const uint32_t*>(p)[0], reinterpret_cast<const uint32_t*>(p)[1]);
  uint32_t w[2] = {0, 0};
#pragma unroll
  for (int i = 0; i < 8; ++i) w[i / 4] |= static_cast<uint32_t>(p[i]) << (8 * (i % 4));
  return make_uint2(w[0], w[1]);
}

// 2^(s - 127) for an E8M0 byte s: 0 gives 2^-127 (a float32 subnormal), 255 NaN.
__device__ __forceinline__ float e8m0(uint32_t s) {
  if (s == 0) return __uint_as_float(0x00400000u);
  if (s == 255) return __uint_as_float(0x7fc00000u);
  return __uint_as_float(s << 23);
}

template <int ALIGN>
__global__ __launch_bounds__(THREADS) void unpack_kernel(const uint8_t* __restrict__ packed,
                                                         int64_t m, int64_t d,
                                                         uint16_t* __restrict__ out) {
  const int64_t blocks = d / 32, row_bytes = d + blocks;
  Run u[RUNS];
  uint2 c[RUNS];
  uint32_t sb[RUNS];
#pragma unroll
  for (int j = 0; j < RUNS; ++j) {
    u[j] = run_of(m, blocks, j);
    const uint8_t* row = packed + u[j].row * row_bytes;
    c[j] = u[j].on ? load8<ALIGN>(row + 32 * u[j].b + 8 * u[j].q) : make_uint2(0, 0);
    sb[j] = u[j].on ? row[d + u[j].b] : 0u;
  }
#pragma unroll
  for (int j = 0; j < RUNS; ++j) {
    if (!u[j].on) continue;
    const float scale = e8m0(sb[j]);
    const uint32_t w[2] = {c[j].x, c[j].y};
    uint32_t o[4];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      // v_cvt_pk_f32_fp8: two E4M3 codes (the word's low or high half) to two floats
      const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(w[i]), false);
      const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(w[i]), true);
      o[2 * i] = static_cast<uint32_t>(f32_to_bf16(lo[0] * scale)) |
                 (static_cast<uint32_t>(f32_to_bf16(lo[1] * scale)) << 16);
      o[2 * i + 1] = static_cast<uint32_t>(f32_to_bf16(hi[0] * scale)) |
                     (static_cast<uint32_t>(f32_to_bf16(hi[1] * scale)) << 16);
    }
    *reinterpret_cast<uint4*>(out + u[j].row * d + 32 * u[j].b + 8 * u[j].q) =
        make_uint4(o[0], o[1], o[2], o[3]);
  }
}

int alignment(int64_t d) {
  const int64_t row_bytes = d + d / 32;
  return row_bytes % 16 == 0 ? 16 : (row_bytes % 4 == 0 ? 4 : 1);
}

}  // namespace
}  // namespace bux

extern "C" int bux_mx_pack_rows(const uint16_t* x, const int32_t* index, int32_t index_div,
                                int64_t n, int64_t m, int64_t d, uint8_t* packed, void* stream) {
  using namespace bux;
  clear_error();
  BUX_CHECK(n >= 0 && m >= 0 && d > 0 && d % 32 == 0 && d < (1LL << 31),
            "bux_mx_pack_rows: n=%lld m=%lld d=%lld (d a positive multiple of 32)",
            (long long)n, (long long)m, (long long)d);
  BUX_CHECK(index || m <= n, "bux_mx_pack_rows: m=%lld rows of x's %lld without an index",
            (long long)m, (long long)n);
  BUX_CHECK(!index || index_div >= 1, "bux_mx_pack_rows: index_div=%d", index_div);
  BUX_CHECK(m == 0 || ((x || n == 0) && packed), "bux_mx_pack_rows: NULL buffer");
  if (m == 0) return BUX_OK;
  const dim3 grid(static_cast<unsigned>(ceil_div(m, THREADS / 64)));
  hipStream_t s = as_stream(stream);
  switch (alignment(d)) {
    case 16: hipLaunchKernelGGL(pack_kernel<16>, grid, dim3(THREADS), 0, s, x, index, index_div, n, m, d, packed); break;
    case 4: hipLaunchKernelGGL(pack_kernel<4>, grid, dim3(THREADS), 0, s, x, index, index_div, n, m, d, packed); break;
    default: hipLaunchKernelGGL(pack_kernel<1>, grid, dim3(THREADS), 0, s, x, index, index_div, n, m, d, packed);
  }
  return launched("pack_kernel");
}

extern "C" int bux_mx_unpack_rows(const uint8_t* packed, int64_t m, int64_t d, uint16_t* out,
                                  void* stream) {
  using namespace bux;
  clear_error();
  BUX_CHECK(m >= 0 && d > 0 && d % 32 == 0 && d < (1LL << 31),
            "bux_mx_unpack_rows: m=%lld d=%lld (d a positive multiple of 32)", (long long)m,
            (long long)d);
  BUX_CHECK(m == 0 || (packed && out), "bux_mx_unpack_rows: NULL buffer");
  if (m == 0) return BUX_OK;
  const int64_t runs = m * ceil_div(d / 32, 16);
  BUX_CHECK(ceil_div(runs, THREADS / 64) < (1LL << 31), "bux_mx_unpack_rows: m=%lld d=%lld is too large for one launch",
            (long long)m, (long long)d);
  const dim3 grid(static_cast<unsigned>(ceil_div(runs, RUNS * (THREADS / 64))));
  hipStream_t s = as_stream(stream);
  switch (alignment(d)) {
    case 16: hipLaunchKernelGGL(unpack_kernel<16>, grid, dim3(THREADS), 0, s, packed, m, d, out); break;
    case 4: hipLaunchKernelGGL(unpack_kernel<4>, grid, dim3(THREADS), 0, s, packed, m, d, out); break;
    default: hipLaunchKernelGGL(unpack_kernel<1>, grid, dim3(THREADS), 0, s, packed, m, d, out);
  }
  return launched("unpack_kernel");
}
