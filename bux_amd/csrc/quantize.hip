// MXFP8 1x32 quantization of a matrix and of its transpose in one pass over it
// (a stack of matrices, one at a time; or rows gathered by index).
//
// Semantics: src/bux/architecture/precision/blockscaled.py:282-356 (mx_twice,
// mx_quantize, _in_e4m3, _ceil_log2, _power_of_two) as grouped_blockscaled._quantized
// (grouped_blockscaled.py:296-317) applies them, and grouped_triton.quantized_twice
// (grouped_triton.py:44-101) for rows read by index. Per block of 32 values v (bfloat16
// widened exactly to float32, or float32 for a layer in float32):
//   e      = ceil_log2(max|v| / 448) clipped to [-126, 126]   scale byte e + 127
//   code_i = RNE_E4M3(clip(v_i * 2^-e, -448, 448))
// v_i * 2^-e is exact in float32 as in bfloat16 (a power of two, no overflow), so the
// float32 product gives the reference's bfloat16 product's code. The exponent of a
// bfloat16 block comes from its maximum's bits; of a float32 block, from the float32
// quotient max / 448 (a float32 maximum has mantissa bits the shortcut would drop).
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
//     64 bytes of a K chunk, consecutive rows consecutive: a store instruction writes
//     512 bytes in one run; pairs of lanes swapping halves for 16-byte stores measured
//     no faster);
//   - the column copy: the tile goes through LDS; four neighbouring lanes take a
//     column, lane q its rows 16 q .. 16 q + 15 of each half of 64 rows (a block of 32
//     is a pair of lanes, reduced by one xor-shuffle), and write its 16 codes of x^T's
//     row as one 16-byte store: a wave's store is 16 of x^T's rows' 64-byte K chunks,
//     1 KiB in one run. Lane 0 of the four writes the column's 4 scale bytes of the
//     tile's 128 rows as one word. The tile's 16-byte chunks are swizzled by row (chunk
//     c of row r at c ^ 2 ((r / 16) % 4)), so that the four lanes' rows, 16 apart, read
//     different banks.
// HBM traffic per element: 2 bytes read (4 of float32), 2 x (1 + 1/32) bytes written; the
// codes go out as non-temporal stores (below).
//
// With BUX_MX_TILES the scale is one per 32 x 32 tile of x instead (the mxfp8_2d
// recipe's weights, blockscaled.py:294-309): xor-shuffles reduce each tile's largest
// magnitude over a wave's rows of it and the waves' maxima meet in LDS, so both copies
// take the tile's scale and hold the same codes, transposed.
//
// The values come from a source: a matrix (or a stack, or rows read by index), or the
// experts' activation computed on the fly from its inputs (h of the forward, d projected
// of the backward), so that the activation's bfloat16 result is quantized without a
// round trip through HBM; those values are the ones the activation kernels would store
// (float32 arithmetic, one rounding to bfloat16), and can be stored too.

#include <type_traits>

#include "common.h"
#include "glu.h"

namespace bux {
namespace {

constexpr int TILE_ROWS = 128;
constexpr int TILE_COLS = 64;
constexpr int THREADS = 256;

// The copies' codes go out as non-temporal stores: both copies' stores write whole runs
// (512 bytes and 1 KiB an instruction), which the GEMMs read a kernel later, and keeping
// them out of the caches' way leaves the source rows there (rows read by index are read
// once for each of a token's picks). The scale bytes, 2 or 4 of them a row, stay
// ordinary stores, which L2 merges into lines. Measured at c3 in the step: W_up's copies
// 6% faster, the step 1%.
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void stream_codes(uint8_t* at, uint32_t a, uint32_t b) {
  __builtin_nontemporal_store(u32x2{a, b}, reinterpret_cast<u32x2*>(at));
}
__device__ __forceinline__ void stream_codes(uint8_t* at, uint32_t a, uint32_t b, uint32_t c,
                                             uint32_t d) {
  __builtin_nontemporal_store(u32x4{a, b, c, d}, reinterpret_cast<u32x4*>(at));
}

// Eight bfloat16 of a uint4 as floats.
__device__ __forceinline__ void floats8(const uint4& r, float* v) {
  const uint32_t q[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    v[2 * j] = bf16_to_f32(static_cast<uint16_t>(q[j] & 0xffffu));
    v[2 * j + 1] = bf16_to_f32(static_cast<uint16_t>(q[j] >> 16));
  }
}

// Eight values of a source's type V: bfloat16 (V = uint16_t, 16 bytes) or float32 (V =
// float, 32 bytes), as a thread loads, stores and widens them.
template <typename V>
struct Pack8;
template <>
struct Pack8<uint16_t> {
  typedef uint4 type;
  __device__ static __forceinline__ type zero() { return make_uint4(0, 0, 0, 0); }
  __device__ static __forceinline__ type load(const uint16_t* p) { return *reinterpret_cast<const uint4*>(p); }
  __device__ static __forceinline__ void store(uint16_t* p, const type& x) { *reinterpret_cast<uint4*>(p) = x; }
  __device__ static __forceinline__ void floats(const type& x, float* v) { floats8(x, v); }
  // the 8 values of v as the type holds them (rounded to bfloat16, nearest even)
  __device__ static __forceinline__ type of(const float* v) {
    return make_uint4(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]),
                      pack_bf16x2(v[6], v[7]));
  }
  __device__ static __forceinline__ float widen(uint16_t x) { return bf16_to_f32(x); }
  __device__ static __forceinline__ uint16_t narrow(float x) { return f32_to_bf16(x); }
  // the scale exponent of a block whose largest magnitude (a value of the type) is amax
  __device__ static __forceinline__ int exponent(float amax) { return scale_exponent_bf16(amax); }
};
template <>
struct Pack8<float> {
  struct type {
    uint4 lo, hi;
  };
  __device__ static __forceinline__ type zero() { return type{make_uint4(0, 0, 0, 0), make_uint4(0, 0, 0, 0)}; }
  __device__ static __forceinline__ type load(const float* p) {
    const uint4* q = reinterpret_cast<const uint4*>(p);
    return type{q[0], q[1]};
  }
  __device__ static __forceinline__ void store(float* p, const type& x) {
    uint4* q = reinterpret_cast<uint4*>(p);
    q[0] = x.lo;
    q[1] = x.hi;
  }
  __device__ static __forceinline__ void floats(const type& x, float* v) {
    const uint32_t w[8] = {x.lo.x, x.lo.y, x.lo.z, x.lo.w, x.hi.x, x.hi.y, x.hi.z, x.hi.w};
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = __uint_as_float(w[j]);
  }
  __device__ static __forceinline__ type of(const float* v) {
    return type{make_uint4(__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]),
                           __float_as_uint(v[3])),
                make_uint4(__float_as_uint(v[4]), __float_as_uint(v[5]), __float_as_uint(v[6]),
                           __float_as_uint(v[7]))};
  }
  __device__ static __forceinline__ float widen(float x) { return x; }
  __device__ static __forceinline__ float narrow(float x) { return x; }
  __device__ static __forceinline__ int exponent(float amax) { return scale_exponent(amax); }
};

// A matrix of bfloat16 (matrix g of a stack), or its rows read by index. With
// `halves`, its columns are read as a GLU's halves (grouped_cudnn.halves_of,
// grouped_cudnn.py:150-155): column c of the copies is, in each 64, the gate (odd column)
// of pair c % 32 for c % 64 < 32, else that pair's up (even column).
template <typename V>
struct MatrixOf {
  typedef V Value;
  static constexpr bool kPartials = false;
  const V* x;
  const int32_t* index;
  int32_t index_div;
  int64_t sources;  // with an index, x's rows: a source row outside [0, sources) reads 0
  int64_t rows, cols;
  bool halves;
  // The tiles go in XCD runs (quantize_kernel); rows read by index take them a column
  // tile at a time, its row tiles one after another: an XCD then works on one or two
  // column tiles at once, and those columns of every token (c3: 16384 tokens x 128
  // bytes, 2 MiB) stay in its L2 for all k of a token's picks, which lie in k places
  // of the index. (Column tiles fastest, an XCD held four at once, 8 MiB, and the
  // tokens came from beyond L2 5.2 times over.)
  __device__ __forceinline__ bool xcd_runs() const { return true; }
  __device__ __forceinline__ bool by_columns() const { return index != nullptr; }
  // Columns [col, col + 8) of row r of matrix g; `live`: r holds values and the
  // columns are the matrix's (`inside`: the columns are; padding past them is not).
  __device__ __forceinline__ typename Pack8<V>::type load(int64_t g, int64_t r, int64_t col,
                                                          bool live, bool, float*) const {
    if (!live) return Pack8<V>::zero();
    int64_t src = r;
    if (index) {
      const int32_t at = index[r];
      if (at < 0) return Pack8<V>::zero();
      // a power-of-two divisor (every top-k bux's configs use) by a shift
      src = (index_div & (index_div - 1)) == 0 ? (at >> (31 - __builtin_clz(index_div)))
                                               : at / index_div;
      if (src >= sources) return Pack8<V>::zero();
    }
    const V* row = (index ? x : x + g * rows * cols) + src * cols;
    if (!halves) return Pack8<V>::load(row + col);
    // 8 columns of one half: 16 consecutive columns of pairs, every other one (a gate
    // is a pair's second, an up its first)
    const int64_t q = col & 63;
    const typename Pack8<V>::type lo = Pack8<V>::load(row + (col - q) + 2 * (q & 31));
    const typename Pack8<V>::type hi = Pack8<V>::load(row + (col - q) + 2 * (q & 31) + 8);
    if constexpr (std::is_same<V, uint16_t>::value) {
      const int shift = q < 32 ? 16 : 0;  // bits: a gate is a pair's high half, an up its low
      const uint32_t w[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
      uint32_t o[4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        o[j] = ((w[2 * j] >> shift) & 0xffffu) | (((w[2 * j + 1] >> shift) & 0xffffu) << 16);
      return make_uint4(o[0], o[1], o[2], o[3]);
    } else {
      const uint32_t w[16] = {lo.lo.x, lo.lo.y, lo.lo.z, lo.lo.w, lo.hi.x, lo.hi.y, lo.hi.z, lo.hi.w,
                              hi.lo.x, hi.lo.y, hi.lo.z, hi.lo.w, hi.hi.x, hi.hi.y, hi.hi.z, hi.hi.w};
      const int pick = q < 32 ? 1 : 0;
      return typename Pack8<V>::type{
          make_uint4(w[pick], w[2 + pick], w[4 + pick], w[6 + pick]),
          make_uint4(w[8 + pick], w[10 + pick], w[12 + pick], w[14 + pick])};
    }
  }
  __device__ __forceinline__ void partial(int64_t, int64_t, float) const {}
};
typedef MatrixOf<uint16_t> Matrix;

// h = act(gate) (up + offset) w, or act(up) w, from projected ((m, f, 2) gated, (m, f)
// plain) and the rows' weights; columns are units. Rows past `filled` give 0. With `h`,
// the values are stored there too.
template <typename K, typename V = uint16_t>
struct GluForward {
  typedef V Value;
  static constexpr bool kPartials = false;
  __device__ __forceinline__ bool xcd_runs() const { return true; }
  __device__ __forceinline__ bool by_columns() const { return false; }
  const V* projected;
  const V* weights;
  V* h;
  Act act;
  int64_t m, f;
  __device__ __forceinline__ typename Pack8<V>::type load(int64_t, int64_t r, int64_t col,
                                                          bool live, bool inside, float*) const {
    typename Pack8<V>::type out = Pack8<V>::zero();
    if (live) {
      const float w = Pack8<V>::widen(weights[r]);
      float v[8];
      if constexpr (K::gated) {
        const V* p = projected + (r * f + col) * 2;
        float pair[16];
        Pack8<V>::floats(Pack8<V>::load(p), pair);
        Pack8<V>::floats(Pack8<V>::load(p + 8), pair + 8);
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = glu_unit<K, std::is_same<V, float>::value>(act, pair[2 * j], pair[2 * j + 1], w);
      } else {
        float up[8];
        Pack8<V>::floats(Pack8<V>::load(projected + r * f + col), up);
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = glu_unit<K, std::is_same<V, float>::value>(act, up[j], 0.0f, w);
      }
      out = Pack8<V>::of(v);
    }
    if (h && r < m && inside) Pack8<V>::store(h + r * f + col, out);
    return out;
  }
  __device__ __forceinline__ void partial(int64_t, int64_t, float) const {}
};

// d projected from projected, the rows' weights and dh (m, f); columns are projected's
// p f (gated: (up, gate) pairs, p = 2; plain: units, p = 1). Each workgroup also leaves
// its 64 columns' share of each row's d weight (the sum of its units' terms) in
// `partials` (m rows of `tiles`), which glu_weights_kernel sums in order. With
// `d_projected`, the values are stored there too.
template <typename K, typename V = uint16_t>
struct GluBackward {
  typedef V Value;
  static constexpr bool kPartials = true;
  __device__ __forceinline__ bool xcd_runs() const { return true; }
  __device__ __forceinline__ bool by_columns() const { return false; }
  static constexpr int P = K::gated ? 2 : 1;
  const V* projected;
  const V* weights;
  const V* dh;
  V* d_projected;
  float* partials;
  Act act;
  int64_t m, f, tiles;
  // dh's 4 values from p (bfloat16: 8 bytes; float32: 16)
  __device__ static __forceinline__ void four(const V* p, float* g) {
    if constexpr (std::is_same<V, uint16_t>::value) {
      const uint2 d = *reinterpret_cast<const uint2*>(p);
      g[0] = bf16_to_f32(d.x & 0xffffu);
      g[1] = bf16_to_f32(d.x >> 16);
      g[2] = bf16_to_f32(d.y & 0xffffu);
      g[3] = bf16_to_f32(d.y >> 16);
    } else {
      const float4 d = *reinterpret_cast<const float4*>(p);
      g[0] = d.x;
      g[1] = d.y;
      g[2] = d.z;
      g[3] = d.w;
    }
  }
  __device__ __forceinline__ typename Pack8<V>::type load(int64_t, int64_t r, int64_t col,
                                                          bool live, bool inside,
                                                          float* dw) const {
    typename Pack8<V>::type out = Pack8<V>::zero();
    *dw = 0.0f;
    if (live) {
      float p[8], v[8], sum = 0.0f;
      Pack8<V>::floats(Pack8<V>::load(projected + r * f * P + col), p);
      const float w = Pack8<V>::widen(weights[r]);
      if constexpr (K::gated) {
        float g[4];
        four(dh + r * f + col / 2, g);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          float term;
          glu_unit_grad<K, std::is_same<V, float>::value>(act, p[2 * j], p[2 * j + 1], w, g[j], &v[2 * j], &v[2 * j + 1], &term);
          sum += term;
        }
      } else {
        float g[8];
        Pack8<V>::floats(Pack8<V>::load(dh + r * f + col), g);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          float term, none;
          glu_unit_grad<K, std::is_same<V, float>::value>(act, p[j], 0.0f, w, g[j], &v[j], &none, &term);
          sum += term;
        }
      }
      *dw = sum;
      out = Pack8<V>::of(v);
    }
    if (d_projected && r < m && inside) Pack8<V>::store(d_projected + r * f * P + col, out);
    return out;
  }
  __device__ __forceinline__ void partial(int64_t r, int64_t tile, float v) const {
    if (r < m) partials[r * tiles + tile] = v;
  }
};

// Workgroup b of n as the b-th tile of a numbering in which XCD x = b % 8 holds a
// contiguous run: n = 8 q + r tiles, XCD x the q + (x < r) of them from x q + min(x, r).
__device__ __forceinline__ int64_t xcd_run(uint32_t b, uint32_t n) {
  const uint32_t q = n / 8, r = n % 8, x = b % 8;
  return static_cast<int64_t>(x) * q + (x < r ? x : r) + b / 8;
}

template <typename Source>
__global__ __launch_bounds__(THREADS) void quantize_kernel(
    Source src, int64_t rows, int64_t cols, int64_t height, const int32_t* __restrict__ filled_ptr,
    int flags, uint8_t* __restrict__ values, uint8_t* __restrict__ scales,
    uint8_t* __restrict__ t_values, uint8_t* __restrict__ t_scales) {
  typedef typename Source::Value V;
  typedef Pack8<V> P8;
  __shared__ V tile[TILE_ROWS][TILE_COLS];
  // where column `col` of row `row` sits in the tile: its group of 8 values (16 bytes of
  // bfloat16, 32 of float32) swizzled
  const auto at = [&](int row, int col) -> V& {
    return tile[row][(((col >> 3) ^ (2 * ((row >> 4) & 3))) << 3) | (col & 7)];
  };

  const int t = threadIdx.x;
  // The tiles are renumbered so that each XCD (workgroup id % 8) takes a contiguous run
  // of them, neighbouring tiles then sharing its L2. Column tiles run fastest, so that
  // neighbouring tiles read one band of rows (two 64-column tiles of d projected read the
  // two halves of one 128-byte line of dh a row; measured at c3: W_up's copies 10% faster,
  // the activations' 4%); rows read by index take row tiles fastest (Matrix::by_columns:
  // quantize x and dy by index 8% and 4% faster in the c3 step). They cover the K
  // padding of the row copy too (columns read as 0 there).
  const int64_t cols_pad = (cols + 127) / 128 * 128;
  const int64_t col_tiles = cols_pad / TILE_COLS;
  const int64_t tile_id = src.xcd_runs() ? xcd_run(blockIdx.x, gridDim.x) : blockIdx.x;
  const int64_t row_tiles = gridDim.x / col_tiles;
  const int64_t col_tile = src.by_columns() ? tile_id / row_tiles : tile_id % col_tiles;
  const int64_t col0 = col_tile * TILE_COLS;
  const int64_t row0 = (src.by_columns() ? tile_id % row_tiles : tile_id / col_tiles) * TILE_ROWS;
  const int64_t g = blockIdx.y;
  const int64_t filled = filled_ptr ? static_cast<int64_t>(*filled_ptr) : height;

  const int chunk = t & 7;  // 8 values of columns col0 + 8 chunk
  const int64_t col = col0 + 8 * chunk;
  const bool col_in = col < cols;  // cols is a multiple of 32: a chunk is all in or out

  typename P8::type raw[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t r = row0 + (t >> 3) + 32 * i;
    float part = 0.0f;
    raw[i] = src.load(g, r, col, r < rows && r < filled && col_in, col_in, &part);
    if constexpr (Source::kPartials) {
      // the 8 lanes of the row: a fixed order of additions
      part += __shfl_xor(part, 1);
      part += __shfl_xor(part, 2);
      part += __shfl_xor(part, 4);
      if (chunk == 0) src.partial(r, col_tile, part);
    }
  }

  // BUX_MX_TILES: a scale per 32 x 32 tile, both copies. A thread's 8 values of row
  // (t / 8) + 32 i lie in tile (i, chunk / 4); xor-shuffles reduce each tile's largest
  // magnitude over a wave's 8 rows of it, and the 4 waves' maxima meet in LDS (with the
  // tile itself, which the column copy reads), so both copies take the tile's scale.
  __shared__ float tile_max[THREADS / 64][TILE_ROWS / 32][TILE_COLS / 32];
  const bool tiles = (flags & BUX_MX_TILES) != 0;
  if (tiles) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      P8::store(&at((t >> 3) + 32 * i, 8 * chunk), raw[i]);
      float w[8];
      P8::floats(raw[i], w);
      float m = 0.0f;
#pragma unroll
      for (int j = 0; j < 8; ++j) m = fmaxf(m, fabsf(w[j]));
      m = fmaxf(m, __shfl_xor(m, 1));
      m = fmaxf(m, __shfl_xor(m, 2));
      m = fmaxf(m, __shfl_xor(m, 8));
      m = fmaxf(m, __shfl_xor(m, 16));
      m = fmaxf(m, __shfl_xor(m, 32));
      if ((t & 59) == 0) tile_max[t >> 6][i][(t >> 2) & 1] = m;  // lanes 0 and 4 of a wave
    }
    __syncthreads();
  }
  // the scale exponent of tile (i, b)
  auto tile_e = [&](int i, int b) {
    float m = tile_max[0][i][b];
#pragma unroll
    for (int w = 1; w < THREADS / 64; ++w) m = fmaxf(m, tile_max[w][i][b]);
    return P8::exponent(m);
  };

  if (flags & BUX_MX_ROWS) {
    uint8_t* vg = values + g * height * cols_pad;
    uint8_t* sg = scales + g * height * (cols_pad / 32);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t r = row0 + (t >> 3) + 32 * i;
      float v[8];
      P8::floats(raw[i], v);
      float amax = 0.0f;
#pragma unroll
      for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(v[j]));
      amax = fmaxf(amax, __shfl_xor(amax, 1));
      amax = fmaxf(amax, __shfl_xor(amax, 2));
      const int e = tiles ? tile_e(i, chunk >> 2) : P8::exponent(amax);
      const float down = power_of_two_down(e);
      uint2 codes;
      codes.x = e4m3x4(clip448(v[0] * down), clip448(v[1] * down), clip448(v[2] * down),
                       clip448(v[3] * down));
      codes.y = e4m3x4(clip448(v[4] * down), clip448(v[5] * down), clip448(v[6] * down),
                       clip448(v[7] * down));
      if (r < height) {  // padding columns too: codes 0, scale byte 1
        stream_codes(vg + ((col >> 6) * height + r) * 64 + (col & 63), codes.x, codes.y);
        const int64_t b = col >> 5;
        if ((chunk & 3) == 0) sg[((b >> 2) * height + r) * 4 + (b & 3)] = static_cast<uint8_t>(e + 127);
      }
    }
  }

  if (!(flags & BUX_MX_COLUMNS)) return;

  if (!tiles) {
#pragma unroll
    for (int i = 0; i < 4; ++i) P8::store(&at((t >> 3) + 32 * i, 8 * chunk), raw[i]);
    __syncthreads();
  }

  // x^T's row c (of x's column c), K (x's rows) from row0: lane q of its four holds K
  // 64 h + 16 q .. + 15 in half h; a block of 32 is the pair q / 2.
  const int q = t & 3, lc = t >> 2;
  const int64_t c = col0 + lc;
  const int64_t kt = (height + 127) / 128 * 128;  // the column copy's K, padded (tiles cover it)
  const bool col_out = c < cols;
  uint8_t* out = t_values + g * cols * kt + ((row0 >> 6) * cols + c) * 64 + 16 * q;
  uint32_t word = 0;  // lane 0's scale bytes of the 4 blocks
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    float v[16];
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      v[j] = P8::widen(at(64 * h + 16 * q + j, lc));
      amax = fmaxf(amax, fabsf(v[j]));
    }
    amax = fmaxf(amax, __shfl_xor(amax, 1));
    const int e = tiles ? tile_e(2 * h + (q >> 1), lc >> 5) : P8::exponent(amax);
    const float down = power_of_two_down(e);
    uint32_t w[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      w[j] = e4m3x4(clip448(v[4 * j] * down), clip448(v[4 * j + 1] * down),
                    clip448(v[4 * j + 2] * down), clip448(v[4 * j + 3] * down));
    if (col_out) stream_codes(out + h * cols * 64, w[0], w[1], w[2], w[3]);
    // block 2 h from this pair (q 0, 1), block 2 h + 1 from the other (q 2, 3)
    const uint32_t b = static_cast<uint32_t>(e + 127);
    const uint32_t other = static_cast<uint32_t>(__shfl_xor(static_cast<int>(b), 2));
    word |= (b | (other << 8)) << (16 * h);
  }
  if (col_out && q == 0)
    *reinterpret_cast<uint32_t*>(t_scales + g * cols * (kt / 32) + ((row0 >> 7) * cols + c) * 4) = word;
}

// d weight of each row: its workgroups' partial sums, added in column order, rounded
// once to V (bfloat16; float32 keeps the sum); rows past `filled` give 0.
template <typename V>
__global__ __launch_bounds__(THREADS) void glu_weights_kernel(const float* __restrict__ partials,
                                                              int64_t m, int64_t tiles,
                                                              const int32_t* __restrict__ filled_ptr,
                                                              V* __restrict__ d_weights) {
  const int64_t r = static_cast<int64_t>(blockIdx.x) * THREADS + threadIdx.x;
  if (r >= m) return;
  const int64_t filled = filled_ptr ? static_cast<int64_t>(*filled_ptr) : m;
  float sum = 0.0f;
  if (r < filled) {
    // tiles is even (two 64-column tiles a 128 of d projected): pairs, added in order
    const float2* row = reinterpret_cast<const float2*>(partials + r * tiles);
    for (int64_t c = 0; c < tiles / 2; ++c) {
      const float2 v = row[c];
      sum += v.x;
      sum += v.y;
    }
  }
  d_weights[r] = Pack8<V>::narrow(sum);
}

// Checks shared by the entry points, then the launch over `groups` matrices.
template <typename Source>
int launch_quantize(const char* name, const Source& src, int64_t groups, int64_t rows, int64_t cols,
                    int64_t height, const int32_t* filled, int flags, uint8_t* values,
                    uint8_t* scales, uint8_t* t_values, uint8_t* t_scales, hipStream_t s) {
  BUX_CHECK(groups >= 1 && rows >= 0 && cols > 0 && height >= rows,
            "%s: bad shape groups=%lld rows=%lld cols=%lld height=%lld", name, (long long)groups,
            (long long)rows, (long long)cols, (long long)height);
  BUX_CHECK(cols % 32 == 0, "%s: cols=%lld is not a multiple of 32", name, (long long)cols);
  BUX_CHECK(height % 32 == 0, "%s: height=%lld is not a multiple of 32", name, (long long)height);
  BUX_CHECK((flags & (BUX_MX_ROWS | BUX_MX_COLUMNS)) != 0 &&
                (flags & ~(BUX_MX_ROWS | BUX_MX_COLUMNS | BUX_MX_TILES)) == 0,
            "%s: flags=%d must be BUX_MX_ROWS and/or BUX_MX_COLUMNS (with BUX_MX_TILES)", name,
            flags);
  BUX_CHECK(!(flags & BUX_MX_ROWS) || (values && scales), "%s: BUX_MX_ROWS needs values and scales",
            name);
  BUX_CHECK(!(flags & BUX_MX_COLUMNS) || (t_values && t_scales),
            "%s: BUX_MX_COLUMNS needs t_values and t_scales", name);
  BUX_CHECK(groups <= 65535, "%s: %lld matrices exceed one launch", name, (long long)groups);
  if (height == 0) return BUX_OK;
  const int64_t tiles = ceil_div(height, TILE_ROWS) * (ceil_div(cols, 128) * 128 / TILE_COLS);
  BUX_CHECK(tiles <= (1LL << 23), "%s: %lld x %lld is too large for one launch", name,
            (long long)height, (long long)cols);
  dim3 grid(static_cast<unsigned>(tiles), static_cast<unsigned>(groups));
  hipLaunchKernelGGL(quantize_kernel<Source>, grid, dim3(THREADS), 0, s, src, rows, cols, height,
                     filled, flags, values, scales, t_values, t_scales);
  return launched(name);
}

}  // namespace

template <typename V>
int launch_glu_weights(const float* partials, int64_t m, int64_t tiles, const int32_t* filled,
                       V* d_weights, hipStream_t s) {
  if (m == 0) return BUX_OK;
  hipLaunchKernelGGL(glu_weights_kernel<V>, dim3(static_cast<unsigned>(ceil_div(m, THREADS))),
                     dim3(THREADS), 0, s, partials, m, tiles, filled, d_weights);
  return launched("glu_weights_kernel");
}
int launch_glu_weights(const float* partials, int64_t m, int64_t tiles, const int32_t* filled,
                       uint16_t* d_weights, hipStream_t s) {
  return launch_glu_weights<uint16_t>(partials, m, tiles, filled, d_weights, s);
}

}  // namespace bux

namespace bux {
namespace {
template <typename V>
int mx_quantize(const char* name, const V* x, const int32_t* index, int32_t index_div,
                int64_t sources, int64_t groups, int64_t rows, int64_t cols, int64_t height,
                const int32_t* filled, int flags, uint8_t* values, uint8_t* scales,
                uint8_t* t_values, uint8_t* t_scales, void* stream) {
  clear_error();
  BUX_CHECK(x != nullptr, "%s: x is NULL", name);
  BUX_CHECK(index == nullptr || index_div >= 1, "%s: index_div=%d", name, index_div);
  BUX_CHECK(index == nullptr || groups == 1, "%s: index takes one matrix, not %lld", name,
            (long long)groups);
  BUX_CHECK(index == nullptr || sources >= 0, "%s: sources=%lld", name, (long long)sources);
  const bool halves = (flags & BUX_MX_HALVES) != 0;
  BUX_CHECK(!halves || cols % 64 == 0, "%s: BUX_MX_HALVES needs cols=%lld a multiple of 64", name,
            (long long)cols);
  const MatrixOf<V> source{x, index, index_div, sources, rows, cols, halves};
  return launch_quantize(name, source, groups, rows, cols, height, filled, flags & ~BUX_MX_HALVES,
                         values, scales, t_values, t_scales, as_stream(stream));
}
}  // namespace
}  // namespace bux

extern "C" int bux_mx_quantize(const uint16_t* x, const int32_t* index, int32_t index_div,
                               int64_t sources, int64_t groups, int64_t rows, int64_t cols,
                               int64_t height, const int32_t* filled, int flags, uint8_t* values,
                               uint8_t* scales, uint8_t* t_values, uint8_t* t_scales,
                               void* stream) {
  return bux::mx_quantize("bux_mx_quantize", x, index, index_div, sources, groups, rows, cols,
                          height, filled, flags, values, scales, t_values, t_scales, stream);
}

extern "C" int bux_mx_quantize_f32(const float* x, const int32_t* index, int32_t index_div,
                                   int64_t sources, int64_t groups, int64_t rows, int64_t cols,
                                   int64_t height, const int32_t* filled, int flags,
                                   uint8_t* values, uint8_t* scales, uint8_t* t_values,
                                   uint8_t* t_scales, void* stream) {
  return bux::mx_quantize("bux_mx_quantize_f32", x, index, index_div, sources, groups, rows, cols,
                          height, filled, flags, values, scales, t_values, t_scales, stream);
}

namespace bux {
namespace {
// The copies an activation's quantizer writes: along the rows where `values` is given,
// the transpose where `t_values` is (a copy not wanted: NULL; at least one).
int copies(const uint8_t* values, const uint8_t* t_values) {
  return (values ? BUX_MX_ROWS : 0) | (t_values ? BUX_MX_COLUMNS : 0);
}

template <typename V>
int glu_quantize(const char* name, const V* projected, const V* weights, const int32_t* filled,
                 int64_t m, int64_t f, const bux_ffn* ffn, int64_t height, V* h, uint8_t* values,
                 uint8_t* scales, uint8_t* t_values, uint8_t* t_scales, void* stream) {
  clear_error();
  Act act;
  if (int rc = act_of(name, ffn, &act)) return rc;
  BUX_CHECK(m == 0 || (projected && weights), "%s: NULL input", name);
  return with_kind(act, [&](auto kind) {
    using K = decltype(kind);
    const GluForward<K, V> src{projected, weights, h, act, m, f};
    return launch_quantize(name, src, 1, m, f, height, filled, copies(values, t_values),
                           values, scales, t_values, t_scales, as_stream(stream));
  });
}
}  // namespace
}  // namespace bux

extern "C" int bux_glu_quantize(const uint16_t* projected, const uint16_t* weights,
                                const int32_t* filled, int64_t m, int64_t f, const bux_ffn* ffn,
                                int64_t height, uint16_t* h, uint8_t* values, uint8_t* scales,
                                uint8_t* t_values, uint8_t* t_scales, void* stream) {
  return bux::glu_quantize("bux_glu_quantize", projected, weights, filled, m, f, ffn, height, h,
                           values, scales, t_values, t_scales, stream);
}

extern "C" int bux_glu_quantize_f32(const float* projected, const float* weights,
                                    const int32_t* filled, int64_t m, int64_t f,
                                    const bux_ffn* ffn, int64_t height, float* h, uint8_t* values,
                                    uint8_t* scales, uint8_t* t_values, uint8_t* t_scales,
                                    void* stream) {
  return bux::glu_quantize("bux_glu_quantize_f32", projected, weights, filled, m, f, ffn, height,
                           h, values, scales, t_values, t_scales, stream);
}

extern "C" size_t bux_glu_backward_quantize_workspace_size(int64_t m, int64_t f) {
  using namespace bux;
  // a float a row and a 64-column tile of d projected, gated (the wider)
  return static_cast<size_t>(m) * static_cast<size_t>(ceil_div(2 * f, 128) * 2) * sizeof(float);
}

namespace bux {
namespace {
template <typename V>
int glu_backward_quantize(const char* name, const V* projected, const V* weights, const V* dh,
                          const int32_t* filled, int64_t m, int64_t f, const bux_ffn* ffn,
                          int64_t height, V* d_projected, uint8_t* values, uint8_t* scales,
                          uint8_t* t_values, uint8_t* t_scales, V* d_weights, void* workspace,
                          size_t workspace_bytes, void* stream) {
  clear_error();
  Act act;
  if (int rc = act_of(name, ffn, &act)) return rc;
  BUX_CHECK(m == 0 || (projected && weights && dh && d_weights), "%s: NULL input or d_weights",
            name);
  const size_t need = bux_glu_backward_quantize_workspace_size(m, f);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need))
    return fail(BUX_E_WORKSPACE, "%s: workspace of %zu bytes, %zu needed", name, workspace_bytes,
                need);
  const int64_t cols = (act.gated ? 2 : 1) * f;
  const int64_t tiles = ceil_div(cols, 128) * 2;
  float* partials = static_cast<float*>(workspace);
  hipStream_t s = as_stream(stream);
  const int rc = with_kind(act, [&](auto kind) {
    using K = decltype(kind);
    const GluBackward<K, V> src{projected, weights, dh, d_projected, partials, act, m, f, tiles};
    return launch_quantize(name, src, 1, m, cols, height, filled, copies(values, t_values),
                           values, scales, t_values, t_scales, s);
  });
  if (rc != BUX_OK) return rc;
  return launch_glu_weights<V>(partials, m, tiles, filled, d_weights, s);
}
}  // namespace
}  // namespace bux

extern "C" int bux_glu_backward_quantize(const uint16_t* projected, const uint16_t* weights,
                                         const uint16_t* dh, const int32_t* filled, int64_t m,
                                         int64_t f, const bux_ffn* ffn, int64_t height,
                                         uint16_t* d_projected, uint8_t* values, uint8_t* scales,
                                         uint8_t* t_values, uint8_t* t_scales,
                                         uint16_t* d_weights, void* workspace,
                                         size_t workspace_bytes, void* stream) {
  return bux::glu_backward_quantize("bux_glu_backward_quantize", projected, weights, dh, filled,
                                    m, f, ffn, height, d_projected, values, scales, t_values,
                                    t_scales, d_weights, workspace, workspace_bytes, stream);
}

extern "C" int bux_glu_backward_quantize_f32(const float* projected, const float* weights,
                                             const float* dh, const int32_t* filled, int64_t m,
                                             int64_t f, const bux_ffn* ffn, int64_t height,
                                             float* d_projected, uint8_t* values,
                                             uint8_t* scales, uint8_t* t_values,
                                             uint8_t* t_scales, float* d_weights,
                                             void* workspace, size_t workspace_bytes,
                                             void* stream) {
  return bux::glu_backward_quantize("bux_glu_backward_quantize_f32", projected, weights, dh,
                                    filled, m, f, ffn, height, d_projected, values, scales,
                                    t_values, t_scales, d_weights, workspace, workspace_bytes,
                                    stream);
}
