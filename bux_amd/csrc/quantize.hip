// MXFP8 1x32 quantization of a matrix and of its transpose in one pass over it
// (a stack of matrices, one at a time; or rows gathered by index).
//
// Semantics: src/bux/architecture/precision/blockscaled.py:282-356 (mx_twice,
// mx_quantize, _in_e4m3, _ceil_log2, _power_of_two) as grouped_blockscaled._quantized
// (grouped_blockscaled.py:296-317) applies them, and grouped_triton.quantized_twice
// (grouped_triton.py:44-101) for rows read by index. Per block of 32 values v (bfloat16,
// widened exactly to float32):
//   e      = ceil_log2(max|v| / 448) clipped to [-126, 126]   scale byte e + 127
//   code_i = RNE_E4M3(clip(v_i * 2^-e, -448, 448))
// v_i * 2^-e is exact in float32 as in bfloat16 (a power of two, no overflow), so the
// float32 product gives the reference's bfloat16 product's code.
//
// The copies are written in the grouped GEMMs' tiled layout (include/bux_amd.h): codes
// [K/64][rows][64] and scale bytes [K/128][rows][4], K padded to whole 128s by codes of
// 0 and scale bytes of 1 (2^-126): the row copy's K is x's columns, the column copy's
// K is the height.
//
// One workgroup of 256 threads (4 waves) takes a tile of 128 rows by 64 columns:
//   - loads: thread t reads 16 bytes (8 values) of row t/8 + 32 i, columns 8 (t % 8):
//     each row's 128 bytes in one coalesced burst of 8 lanes;
//   - the row copy: a block of 32 columns is 4 neighbouring lanes, reduced by two
//     xor-shuffles; each lane writes its 8 codes as one 8-byte store (8 lanes a row's
//     64 bytes of a K chunk, consecutive rows consecutive);
//   - the column copy: the tile goes through LDS; wave w takes rows 32w..32w+31, lane
//     l column l, reading one LDS row per step (all lanes on one row: no bank
//     conflicts), and writes its 32 codes of x^T's row l as two 16-byte stores (half
//     of the row's 64-byte K chunk; the other wave of the pair writes the other half).
// HBM traffic per element: 2 bytes read, 2 x (1 + 1/32) bytes written.

#include "common.h"

namespace bux {
namespace {

constexpr int TILE_ROWS = 128;
constexpr int TILE_COLS = 64;
constexpr int THREADS = 256;

__global__ __launch_bounds__(THREADS) void quantize_kernel(
    const uint16_t* __restrict__ x, const int32_t* __restrict__ index, int32_t index_div,
    int64_t rows, int64_t cols, int64_t height, const int32_t* __restrict__ filled_ptr, int flags,
    uint8_t* __restrict__ values, uint8_t* __restrict__ scales, uint8_t* __restrict__ t_values,
    uint8_t* __restrict__ t_scales) {
  __shared__ uint16_t tile[TILE_ROWS][TILE_COLS];

  const int t = threadIdx.x;
  // Column tiles run fastest, so that neighbouring workgroups read one band of rows.
  // They cover the K padding of the row copy too (columns read as 0 there).
  const int64_t cols_pad = (cols + 127) / 128 * 128;
  const int64_t col_tiles = cols_pad / TILE_COLS;
  const int64_t col0 = (static_cast<int64_t>(blockIdx.x) % col_tiles) * TILE_COLS;
  const int64_t row0 = (static_cast<int64_t>(blockIdx.x) / col_tiles) * TILE_ROWS;
  const int64_t g = blockIdx.y;
  const int64_t filled = filled_ptr ? static_cast<int64_t>(*filled_ptr) : height;
  const uint16_t* xg = index ? x : x + g * rows * cols;

  const int chunk = t & 7;  // 8 values of columns col0 + 8 chunk
  const int64_t col = col0 + 8 * chunk;
  const bool col_in = col < cols;  // cols is a multiple of 32: a chunk is all in or out

  uint4 raw[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t r = row0 + (t >> 3) + 32 * i;
    int64_t src = -1;
    if (r < rows && r < filled) {
      if (index) {
        const int32_t at = index[r];
        src = at < 0 ? -1 : at / index_div;
      } else {
        src = r;
      }
    }
    raw[i] = make_uint4(0, 0, 0, 0);
    if (src >= 0 && col_in) raw[i] = *reinterpret_cast<const uint4*>(xg + src * cols + col);
  }

  if (flags & BUX_MX_ROWS) {
    uint8_t* vg = values + g * height * cols_pad;
    uint8_t* sg = scales + g * height * (cols_pad / 32);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t r = row0 + (t >> 3) + 32 * i;
      const uint32_t w[4] = {raw[i].x, raw[i].y, raw[i].z, raw[i].w};
      float v[8];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        v[2 * j] = bf16_to_f32(static_cast<uint16_t>(w[j] & 0xffffu));
        v[2 * j + 1] = bf16_to_f32(static_cast<uint16_t>(w[j] >> 16));
      }
      float amax = 0.0f;
#pragma unroll
      for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(v[j]));
      amax = fmaxf(amax, __shfl_xor(amax, 1));
      amax = fmaxf(amax, __shfl_xor(amax, 2));
      const int e = scale_exponent(amax);
      const float down = power_of_two_down(e);
      uint2 codes;
      codes.x = e4m3x4(clip448(v[0] * down), clip448(v[1] * down), clip448(v[2] * down),
                       clip448(v[3] * down));
      codes.y = e4m3x4(clip448(v[4] * down), clip448(v[5] * down), clip448(v[6] * down),
                       clip448(v[7] * down));
      if (r < height) {  // padding columns too: codes 0, scale byte 1
        *reinterpret_cast<uint2*>(vg + ((col >> 6) * height + r) * 64 + (col & 63)) = codes;
        const int64_t b = col >> 5;
        if ((chunk & 3) == 0) sg[((b >> 2) * height + r) * 4 + (b & 3)] = static_cast<uint8_t>(e + 127);
      }
    }
  }

  if (!(flags & BUX_MX_COLUMNS)) return;

#pragma unroll
  for (int i = 0; i < 4; ++i) {
    *reinterpret_cast<uint4*>(&tile[(t >> 3) + 32 * i][8 * chunk]) = raw[i];
  }
  __syncthreads();

  const int wave = t >> 6;
  const int lane = t & 63;
  const int64_t c = col0 + lane;
  const int64_t rb = row0 + 32 * wave;  // the block's first row (below kt: tiles cover it)
  const int64_t kt = (height + 127) / 128 * 128;  // the column copy's K, padded
  if (c >= cols) return;
  float v[32];
  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < 32; ++j) {
    v[j] = bf16_to_f32(tile[32 * wave + j][lane]);
    amax = fmaxf(amax, fabsf(v[j]));
  }
  const int e = scale_exponent(amax);
  const float down = power_of_two_down(e);
  uint32_t w[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    w[j] = e4m3x4(clip448(v[4 * j] * down), clip448(v[4 * j + 1] * down),
                  clip448(v[4 * j + 2] * down), clip448(v[4 * j + 3] * down));
  }
  // x^T's row c, K (x's rows) from rb: 32 bytes of its 64-byte chunk rb / 64
  uint8_t* out = t_values + g * cols * kt + ((rb >> 6) * cols + c) * 64 + (rb & 63);
  reinterpret_cast<uint4*>(out)[0] = make_uint4(w[0], w[1], w[2], w[3]);
  reinterpret_cast<uint4*>(out)[1] = make_uint4(w[4], w[5], w[6], w[7]);
  t_scales[g * cols * (kt / 32) + ((rb >> 7) * cols + c) * 4 + ((rb >> 5) & 3)] =
      static_cast<uint8_t>(e + 127);
}

}  // namespace
}  // namespace bux

extern "C" int bux_mx_quantize(const uint16_t* x, const int32_t* index, int32_t index_div,
                               int64_t groups, int64_t rows, int64_t cols, int64_t height,
                               const int32_t* filled, int flags, uint8_t* values, uint8_t* scales,
                               uint8_t* t_values, uint8_t* t_scales, void* stream) {
  using namespace bux;
  clear_error();
  BUX_CHECK(x != nullptr, "bux_mx_quantize: x is NULL");
  BUX_CHECK(groups >= 1 && rows >= 0 && cols > 0 && height >= rows,
            "bux_mx_quantize: bad shape groups=%lld rows=%lld cols=%lld height=%lld",
            (long long)groups, (long long)rows, (long long)cols, (long long)height);
  BUX_CHECK(index == nullptr || index_div >= 1, "bux_mx_quantize: index_div=%d", index_div);
  BUX_CHECK(cols % 32 == 0, "bux_mx_quantize: cols=%lld is not a multiple of 32", (long long)cols);
  BUX_CHECK(height % 32 == 0, "bux_mx_quantize: height=%lld is not a multiple of 32",
            (long long)height);
  BUX_CHECK(flags != 0 && (flags & ~(BUX_MX_ROWS | BUX_MX_COLUMNS)) == 0,
            "bux_mx_quantize: flags=%d must be BUX_MX_ROWS and/or BUX_MX_COLUMNS", flags);
  BUX_CHECK(!(flags & BUX_MX_ROWS) || (values && scales),
            "bux_mx_quantize: BUX_MX_ROWS needs values and scales");
  BUX_CHECK(!(flags & BUX_MX_COLUMNS) || (t_values && t_scales),
            "bux_mx_quantize: BUX_MX_COLUMNS needs t_values and t_scales");
  BUX_CHECK(index == nullptr || groups == 1, "bux_mx_quantize: index takes one matrix, not %lld",
            (long long)groups);
  BUX_CHECK(groups <= 65535, "bux_mx_quantize: %lld matrices exceed one launch", (long long)groups);
  if (height == 0) return BUX_OK;
  const int64_t tiles = ceil_div(height, TILE_ROWS) * (ceil_div(cols, 128) * 128 / TILE_COLS);
  BUX_CHECK(tiles <= (1LL << 23), "bux_mx_quantize: %lld x %lld is too large for one launch",
            (long long)height, (long long)cols);
  dim3 grid(static_cast<unsigned>(tiles), static_cast<unsigned>(groups));
  hipLaunchKernelGGL(quantize_kernel, grid, dim3(THREADS), 0, as_stream(stream), x, index,
                     index_div, rows, cols, height, filled, flags, values, scales, t_values,
                     t_scales);
  return launched("quantize_kernel");
}
