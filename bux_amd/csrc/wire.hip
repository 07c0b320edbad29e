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
// A lane takes a block of 32 values: 64 bytes of bfloat16 in (four 16-byte loads), 32
// codes and a scale byte out (or the reverse); a wave takes 64 blocks of a row, a
// workgroup 4 waves. Quantizing a token once per pick rather than once gives the same
// bytes (the quantizer is a function of the row) and reads the token's further copies
// from L2. Unpacking is exact: a code times a power of two holds in float32 and, with
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
  const int64_t src = index ? index[i] / div : i;
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
  const int64_t i = static_cast<int64_t>(blockIdx.x) * (THREADS / 64) + (threadIdx.x >> 6);
  if (i >= m) return;
  const int64_t blocks = d / 32, row_bytes = d + blocks;
  const uint8_t* row = packed + i * row_bytes;
  for (int64_t b = threadIdx.x & 63; b < blocks; b += 64) {
    uint32_t w[8];
    const uint8_t* c = row + 32 * b;
    if (ALIGN == 16) {
      const uint4 lo = *reinterpret_cast<const uint4*>(c), hi = *reinterpret_cast<const uint4*>(c + 16);
      w[0] = lo.x; w[1] = lo.y; w[2] = lo.z; w[3] = lo.w;
      w[4] = hi.x; w[5] = hi.y; w[6] = hi.z; w[7] = hi.w;
    } else if (ALIGN == 4) {
#pragma unroll
      for (int j = 0; j < 8; ++j) w[j] = reinterpret_cast<const uint32_t*>(c)[j];
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j)
        w[j] = static_cast<uint32_t>(c[4 * j]) | (static_cast<uint32_t>(c[4 * j + 1]) << 8) |
               (static_cast<uint32_t>(c[4 * j + 2]) << 16) |
               (static_cast<uint32_t>(c[4 * j + 3]) << 24);
    }
    const float scale = e8m0(row[d + b]);
    uint32_t o[16];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      // v_cvt_pk_f32_fp8: two E4M3 codes (the word's low or high half) to two floats
      const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(w[j]), false);
      const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(w[j]), true);
      o[2 * j] = static_cast<uint32_t>(f32_to_bf16(lo[0] * scale)) |
                 (static_cast<uint32_t>(f32_to_bf16(lo[1] * scale)) << 16);
      o[2 * j + 1] = static_cast<uint32_t>(f32_to_bf16(hi[0] * scale)) |
                     (static_cast<uint32_t>(f32_to_bf16(hi[1] * scale)) << 16);
    }
    uint4* dst = reinterpret_cast<uint4*>(out + i * d + 32 * b);
#pragma unroll
    for (int q = 0; q < 4; ++q) dst[q] = make_uint4(o[4 * q], o[4 * q + 1], o[4 * q + 2], o[4 * q + 3]);
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
  const dim3 grid(static_cast<unsigned>(ceil_div(m, THREADS / 64)));
  hipStream_t s = as_stream(stream);
  switch (alignment(d)) {
    case 16: hipLaunchKernelGGL(unpack_kernel<16>, grid, dim3(THREADS), 0, s, packed, m, d, out); break;
    case 4: hipLaunchKernelGGL(unpack_kernel<4>, grid, dim3(THREADS), 0, s, packed, m, d, out); break;
    default: hipLaunchKernelGGL(unpack_kernel<1>, grid, dim3(THREADS), 0, s, packed, m, d, out);
  }
  return launched("unpack_kernel");
}
