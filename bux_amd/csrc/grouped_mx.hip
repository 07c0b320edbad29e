// Grouped MXFP8 GEMMs on CDNA4's block-scaled MFMA (v_mfma_scale_f32_32x32x64_f8f6f4):
// E4M3 x E4M3 with an E8M0 scale per 32 of what they contract, float32 accumulation.
//
//   rows      y[i] = a[i] b[g(i)]^T for each group g's rows i      grouped_mxfp8.py:116-154
//             (fprop x W and dgrad dy W^T); rows past sum(sizes) are 0.
//   contract  dw[g] = a[:, rows of g] b[:, rows of g]^T           grouped_mxfp8.py:185-210
//             (wgrad); a block of 32 rows that another group shares counts as 0 in a
//             (the reference's _edges, grouped_mxfp8.py:240-256).
//
// Both operands arrive row-major with what they contract contiguous (the canonical
// MXFP8 layout: codes (r, K), scale bytes (r, K/32)), so one mainloop serves both:
// C[r][c] = sum_k A[r][k] B[c][k] over a tile of 128 x 128 outputs.
//
// Workgroup: 256 lanes in 4 waves (2 x 2), each wave 64 x 64 outputs as 2 x 2 MFMAs of
// 32 x 32, two MFMAs of K = 64 per step of K = 128 bytes. A step's A and B tiles
// (16 KiB each) and their scales (one word a row) are double-buffered in LDS: the next
// step's global loads are in flight while the MFMAs read the current one. In LDS each
// row's eight 16-byte chunks sit at chunk ^ swizzle(row), so that the lanes reading one
// chunk of consecutive rows spread over every bank.
//
// MFMA lane layout (32 x 32 x 64), measured on the MI355X: lane l holds row l % 32 of A
// (column l % 32 of B); lane half h = l / 32 holds 16 bytes of each of the two blocks of
// 32 in K, block 0 in register bytes 0..15 and block 1 in bytes 16..31, and its scale
// operand (the register's low byte) scales block h of its row. A and B load alike, so
// the order of K inside a block is immaterial. The accumulator's 16 registers of lane l
// are rows 8 (j / 4) + 4 (l / 32) + j % 4, column l % 32.
//
// Ragged rows: a tile list like the reference's tiles_of (grouped_mxfp8.py:157-182),
// built on the device from `sizes` so the host never synchronises: each tile of 128
// rows that a group has rows in, once for each group in it (a tile two groups share
// runs twice and each stores its own rows), and the rows past the groups as a group
// of their own that stores 0.

#include "common.h"

namespace bux {
namespace {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int BM = 128;  // rows of a tile (A's)
constexpr int BN = 128;  // columns of a tile (B's rows)
constexpr int BK = 128;  // bytes of K a step
constexpr int THREADS = 256;
constexpr int MAX_GROUPS = 4096;

struct Tile {
  int32_t group, lo, hi;
};

// --- the device-side prologue: group starts and the ragged tile list ----------------

// Exclusive scan of data[0, n) in LDS by one workgroup of THREADS lanes; returns the
// total. `partial` is THREADS ints of LDS.
__device__ int32_t block_scan(int32_t* data, int n, int32_t* partial) {
  const int t = threadIdx.x;
  const int per = (n + THREADS - 1) / THREADS;
  const int lo = t * per, hi = lo + per < n ? lo + per : n;
  int32_t sum = 0;
  for (int i = lo; i < hi; ++i) sum += data[i];
  partial[t] = sum;
  __syncthreads();
  for (int step = 1; step < THREADS; step <<= 1) {
    const int32_t add = t >= step ? partial[t - step] : 0;
    __syncthreads();
    partial[t] += add;
    __syncthreads();
  }
  int32_t run = t > 0 ? partial[t - 1] : 0;
  for (int i = lo; i < hi; ++i) {
    const int32_t c = data[i];
    data[i] = run;
    run += c;
  }
  const int32_t total = partial[THREADS - 1];
  __syncthreads();
  return total;
}

// starts[g] for g <= groups (starts[groups] = sum of sizes), then, if `tiles`, the
// tile list of `slots` entries over `rows` rows (the last group the rows from the
// sum of sizes to `height`).
//
// Two rules for a group's tiles of `tile_rows`: the tiles of the rows' absolute grid
// that the group has rows in (a tile two groups share is listed for each), or, with
// `from_start`, tiles from the group's first row on (the last one partial; the rows
// past it belong to the next group or past the groups, and are computed but not stored).
__global__ __launch_bounds__(THREADS) void prologue_kernel(const int32_t* __restrict__ sizes,
                                                           int32_t groups, int64_t height,
                                                           int64_t slots, int tile_rows,
                                                           bool from_start,
                                                           int32_t* __restrict__ starts_out,
                                                           Tile* __restrict__ tiles) {
  __shared__ int32_t starts[MAX_GROUPS + 2];
  __shared__ int32_t before[MAX_GROUPS + 2];
  __shared__ int32_t partial[THREADS];
  const int t = threadIdx.x;
  for (int g = t; g < groups; g += THREADS) starts[g] = sizes[g];
  __syncthreads();
  const int32_t filled = block_scan(starts, groups, partial);
  if (t == 0) starts[groups] = filled;
  __syncthreads();
  for (int g = t; g <= groups; g += THREADS) starts_out[g] = starts[g];
  if (tiles == nullptr) return;
  // The rows past the groups, up to height, are group `groups`.
  const int all = groups + 1;
  auto size_of = [&](int g) -> int64_t {
    if (g < groups) return sizes[g];
    return height > filled ? height - filled : 0;
  };
  const int64_t tr = tile_rows;
  auto count_of = [&](int64_t s, int64_t start) -> int64_t {
    if (s <= 0) return 0;
    return from_start ? (s + tr - 1) / tr : (start + s + tr - 1) / tr - start / tr;
  };
  for (int g = t; g < all; g += THREADS)
    before[g] = static_cast<int32_t>(count_of(size_of(g), starts[g]));
  __syncthreads();
  const int32_t used = block_scan(before, all, partial);
  for (int g = t; g < all; g += THREADS) {
    const int64_t s = size_of(g), start = starts[g], end = start + s;
    const int64_t count = count_of(s, start);
    // Sizes summing past the rows there are would list more tiles than there are
    // slots: those are dropped, never written past the list.
    for (int64_t j = 0; j < count && before[g] + j < slots; ++j) {
      const int64_t lo = from_start ? start + j * tr : (start / tr + j) * tr;
      Tile out;
      out.group = g;
      out.lo = static_cast<int32_t>(start > lo ? start : lo);
      out.hi = static_cast<int32_t>(end < lo + tr ? end : lo + tr);
      tiles[before[g] + j] = out;
    }
  }
  for (int64_t i = used + t; i < slots; i += THREADS) tiles[i] = Tile{0, 0, 0};
}

// --- the mainloop --------------------------------------------------------------------

struct Operand {
  const uint8_t* values;  // row r's byte k at values[r * ld + k]
  const uint8_t* scales;  // row r's block b at scales[r * (ld / 32) + b]
  int64_t ld;             // bytes of K a row (a multiple of 32)
  int64_t rows;           // rows there are: loads past them read 0
};

// Where a row's 16-byte chunk c of a 128-byte LDS row sits: chunk c ^ swizzle(row).
// gfx950's LDS serves ds_read_b128 16 lanes at a time over 64 banks of 4 bytes (256
// bytes): the 16 consecutive rows that 16 lanes read at one logical chunk must cover
// all 16 places of 16 bytes in 256, which rows r and r ^ 1 (apart by 128 bytes) and
// (r / 2) % 8 do. Measured on the MI355X: 193 bytes a clock, against 112 for c ^ (r % 8).
__device__ __forceinline__ int swizzle(int row) { return (row >> 1) & 7; }

struct Lds {
  uint8_t a[2][BM * BK];
  uint8_t b[2][BN * BK];
  uint32_t as[2][BM];
  uint32_t bs[2][BN];
};

__device__ __forceinline__ uint4 zero_outside(uint4 v, int64_t k0, int64_t lo, int64_t hi) {
  if (k0 >= lo && k0 + 16 <= hi) return v;
  if (k0 + 16 <= lo || k0 >= hi) return make_uint4(0, 0, 0, 0);
  uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    uint32_t keep = 0;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const int64_t k = k0 + 4 * q + b;
      if (k >= lo && k < hi) keep |= 0xffu << (8 * b);
    }
    w[q] &= keep;
  }
  return make_uint4(w[0], w[1], w[2], w[3]);
}

// The scale word (4 blocks of 32) of row `row` at K step `kt`; a block past the row's
// or a row past the operand's reads 127 (2^0), which its values, 0, ignore.
__device__ __forceinline__ uint32_t load_scales(const Operand& op, int64_t row, int64_t kt) {
  const int64_t blocks = op.ld / 32;
  if (row >= op.rows || kt * 4 >= blocks) return 0x7f7f7f7fu;
  const uint8_t* p = op.scales + row * blocks + kt * 4;
  if ((blocks & 3) == 0) return *reinterpret_cast<const uint32_t*>(p);
  uint32_t w = 0;
#pragma unroll
  for (int b = 0; b < 4; ++b) w |= (kt * 4 + b < blocks ? static_cast<uint32_t>(p[b]) : 0x7fu) << (8 * b);
  return w;
}

struct Staged {
  uint4 a[4], b[4];
  uint32_t scale;  // lanes 0..127: A's row; 128..255: B's
};

// Global -> registers for K step kt: lane t takes 16 bytes of rows t/8 + 32 i at
// chunk t % 8. With `mask`, A's bytes outside K [mlo, mhi) read 0.
__device__ __forceinline__ void fetch(Staged& s, const Operand& A, int64_t a_row0, const Operand& B,
                                      int64_t b_row0, int64_t kt, bool mask, int64_t mlo,
                                      int64_t mhi) {
  const int t = threadIdx.x;
  const int chunk = t & 7;
  const int64_t k0 = kt * BK + 16 * chunk;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t r = (t >> 3) + 32 * i;
    const int64_t ra = a_row0 + r, rb = b_row0 + r;
    s.a[i] = make_uint4(0, 0, 0, 0);
    s.b[i] = make_uint4(0, 0, 0, 0);
    if (k0 < A.ld && ra < A.rows) s.a[i] = *reinterpret_cast<const uint4*>(A.values + ra * A.ld + k0);
    if (k0 < B.ld && rb < B.rows) s.b[i] = *reinterpret_cast<const uint4*>(B.values + rb * B.ld + k0);
    if (mask) s.a[i] = zero_outside(s.a[i], k0, mlo, mhi);
  }
  s.scale = t < BM ? load_scales(A, a_row0 + t, kt) : load_scales(B, b_row0 + (t - BM), kt);
}

__device__ __forceinline__ void stage(const Staged& s, Lds& lds, int buf) {
  const int t = threadIdx.x;
  const int chunk = t & 7;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = (t >> 3) + 32 * i;
    const int at = r * BK + ((chunk ^ swizzle(r)) << 4);
    *reinterpret_cast<uint4*>(&lds.a[buf][at]) = s.a[i];
    *reinterpret_cast<uint4*>(&lds.b[buf][at]) = s.b[i];
  }
  if (t < BM) lds.as[buf][t] = s.scale;
  else lds.bs[buf][t - BM] = s.scale;
}

// A's (or B's) operand for one MFMA: 32 bytes of row `row` at K sub-step `sub` (64
// bytes of K). The MFMA takes each register's bytes 0..15 of both lane halves as its
// first block of 32 (scaled by lane half 0's scale) and bytes 16..31 as its second
// (lane half 1's): lane half h holds K chunks h and 2 + h of the sub-step.
__device__ __forceinline__ v8i operand(const uint8_t* tile, int row, int sub, int half) {
  const int c0 = sub * 4 + half;
  const uint4 lo = *reinterpret_cast<const uint4*>(tile + row * BK + (((c0) ^ swizzle(row)) << 4));
  const uint4 hi = *reinterpret_cast<const uint4*>(tile + row * BK + (((c0 + 2) ^ swizzle(row)) << 4));
  v8i v;
  v[0] = lo.x; v[1] = lo.y; v[2] = lo.z; v[3] = lo.w;
  v[4] = hi.x; v[5] = hi.y; v[6] = hi.z; v[7] = hi.w;
  return v;
}

__device__ __forceinline__ void multiply(const Lds& lds, int buf, v16f acc[2][2]) {
  const int t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int half = lane >> 5;
#pragma unroll
  for (int sub = 0; sub < 2; ++sub) {
    v8i a[2], b[2];
    int sa[2], sb[2];
    const int shift = 8 * (sub * 2 + half);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int ra = wm * 64 + i * 32 + (lane & 31);
      const int rb = wn * 64 + i * 32 + (lane & 31);
      a[i] = operand(lds.a[buf], ra, sub, half);
      b[i] = operand(lds.b[buf], rb, sub, half);
      sa[i] = static_cast<int>((lds.as[buf][ra] >> shift) & 0xffu);
      sb[i] = static_cast<int>((lds.bs[buf][rb] >> shift) & 0xffu);
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a[i], b[j], acc[i][j], 0, 0, 0,
                                                                   sa[i], 0, sb[j]);
  }
}

// acc += A[a_row0 + r] . B[b_row0 + c] over K steps [kt_begin, kt_end).
__device__ __forceinline__ void mainloop(const Operand& A, int64_t a_row0, const Operand& B,
                                         int64_t b_row0, int64_t kt_begin, int64_t kt_end,
                                         bool mask, int64_t mlo, int64_t mhi, Lds& lds,
                                         v16f acc[2][2]) {
  Staged s;
  if (kt_begin >= kt_end) return;
  fetch(s, A, a_row0, B, b_row0, kt_begin, mask, mlo, mhi);
  stage(s, lds, 0);
  __syncthreads();
  for (int64_t kt = kt_begin; kt < kt_end; ++kt) {
    const int buf = static_cast<int>((kt - kt_begin) & 1);
    const bool more = kt + 1 < kt_end;
    if (more) fetch(s, A, a_row0, B, b_row0, kt + 1, mask, mlo, mhi);
    multiply(lds, buf, acc);
    if (more) stage(s, lds, buf ^ 1);
    __syncthreads();
  }
}

template <typename T>
__device__ __forceinline__ T from_f32(float v);
template <>
__device__ __forceinline__ uint16_t from_f32<uint16_t>(float v) { return f32_to_bf16(v); }
template <>
__device__ __forceinline__ float from_f32<float>(float v) { return v; }

// Stores the tile's outputs at rows [row_lo, row_hi) and columns below n_cols:
// out[(row) * ld + col], row = row0 + tile row, col = col0 + tile column.
template <typename T>
__device__ __forceinline__ void store(const v16f acc[2][2], T* out, int64_t ld, int64_t row0,
                                      int64_t col0, int64_t row_lo, int64_t row_hi, int64_t n_cols) {
  const int t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  const int wm = wave >> 1, wn = wave & 1;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int64_t col = col0 + wn * 64 + j * 32 + (lane & 31);
      if (col >= n_cols) continue;
#pragma unroll
      for (int q = 0; q < 16; ++q) {
        const int64_t row = row0 + wm * 64 + i * 32 + 8 * (q >> 2) + 4 * (lane >> 5) + (q & 3);
        if (row >= row_lo && row < row_hi) out[row * ld + col] = from_f32<T>(acc[i][j][q]);
      }
    }
}

template <typename T>
__device__ void store_zeros(T* out, int64_t ld, int64_t row_lo, int64_t row_hi, int64_t col0,
                            int64_t n_cols) {
  const int64_t width = (col0 + BN < n_cols ? col0 + BN : n_cols) - col0;
  for (int64_t i = threadIdx.x; i < (row_hi - row_lo) * width; i += THREADS)
    out[(row_lo + i / width) * ld + col0 + i % width] = from_f32<T>(0.0f);
}

template <typename T>
__global__ __launch_bounds__(THREADS) void rows_kernel(Operand A, Operand B, int32_t groups,
                                                       int64_t n, int64_t height,
                                                       const Tile* __restrict__ tiles,
                                                       int64_t col_tiles, T* __restrict__ y) {
  extern __shared__ __align__(16) uint8_t smem[];
  Lds& lds = *reinterpret_cast<Lds*>(smem);
  const int64_t slot = blockIdx.x / col_tiles;
  const int64_t col0 = (blockIdx.x % col_tiles) * BN;
  Tile tile = tiles[slot];
  // Rows of y stop at height whatever the sizes say.
  if (tile.hi > height) tile.hi = static_cast<int32_t>(height);
  if (tile.lo >= tile.hi) return;
  if (tile.group >= groups) {  // rows past the groups
    store_zeros(y, n, tile.lo, tile.hi, col0, n);
    return;
  }
  const int64_t row0 = static_cast<int64_t>(tile.lo) / BM * BM;
  Operand b = B;
  b.values += static_cast<int64_t>(tile.group) * B.rows * B.ld;
  b.scales += static_cast<int64_t>(tile.group) * B.rows * (B.ld / 32);
  v16f acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int q = 0; q < 16; ++q) acc[i][j][q] = 0.0f;
  mainloop(A, row0, b, col0, 0, (A.ld + BK - 1) / BK, false, 0, 0, lds, acc);
  store(acc, y, n, row0, col0, tile.lo, tile.hi, n);
}

template <typename T>
__global__ __launch_bounds__(THREADS) void contract_kernel(Operand A, Operand B, int32_t groups,
                                                           const int32_t* __restrict__ starts,
                                                           int64_t d_tiles, int64_t f_tiles,
                                                           T* __restrict__ dw) {
  extern __shared__ __align__(16) uint8_t smem[];
  Lds& lds = *reinterpret_cast<Lds*>(smem);
  const int64_t per_group = d_tiles * f_tiles;
  const int64_t g = blockIdx.x / per_group;
  const int64_t rest = blockIdx.x % per_group;
  const int64_t row0 = (rest / f_tiles) * BM;  // rows of dw[g]: A's rows (d)
  const int64_t col0 = (rest % f_tiles) * BN;  // columns of dw[g]: B's rows (f)
  const int64_t start = starts[g], end = starts[g + 1];
  T* out = dw + g * A.rows * B.rows;
  v16f acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int q = 0; q < 16; ++q) acc[i][j][q] = 0.0f;
  if (end > start) {
    // A's bytes outside the group's rows read 0 only in its first and last steps.
    const int64_t kt_begin = start / BK, kt_end = (end + BK - 1) / BK;
    const bool ragged = (start % BK) != 0 || (end % BK) != 0;
    if (!ragged) {
      mainloop(A, row0, B, col0, kt_begin, kt_end, false, 0, 0, lds, acc);
    } else {
      mainloop(A, row0, B, col0, kt_begin, kt_begin + 1, true, start, end, lds, acc);
      if (kt_end - kt_begin > 2)
        mainloop(A, row0, B, col0, kt_begin + 1, kt_end - 1, false, 0, 0, lds, acc);
      if (kt_end - kt_begin > 1)
        mainloop(A, row0, B, col0, kt_end - 1, kt_end, true, start, end, lds, acc);
    }
  }
  store(acc, out, B.rows, row0, col0, row0, A.rows, B.rows);
}

// --- v2: 256 x 256 tiles, a 4-stage pipeline of direct-to-LDS loads ----------------
//
// For K a whole number of 128-byte steps. A workgroup of 4 waves takes 256 x 256
// outputs, each wave 128 x 128 as 4 x 4 MFMAs of 32 x 32 (256 accumulator registers:
// one wave a SIMD). K goes in steps of 64 bytes (one MFMA deep). Each step's A and B
// tiles (16 KiB each) and scale words go from global memory straight into LDS
// (buffer_load ... lds, 16 bytes a lane, no registers on the way) in a ring of 4
// stages, issued 4 steps ahead of their MFMAs. A wave keeps two sets of operand
// registers: while the MFMAs of step k run on one, its LDS reads of step k + 1 fill
// the other, and the workgroup's one barrier a step (after which step k + 2's stage is
// visible and step k + 1's has been read by every wave) sits between them. Each lane's
// source address is chosen so that LDS holds each 64-byte row's chunks at
// chunk ^ swizzle64(row). The MFMA takes B's rows as its first operand and A's as its
// second, so that a lane's accumulators are 4 runs of 4 consecutive output columns of
// one output row: the epilogue stores 8 (bf16) or 16 (f32) contiguous bytes a run.
//
// Ragged rows: a group's tiles start at its first row (`prologue_kernel`'s
// from_start rule), so no tile computes two groups; a tile's rows past its group are
// computed from whatever rows follow (the next group's, or the padding) and not
// stored. Workgroups are renumbered so that each XCD (a workgroup's id modulo 8) takes
// a contiguous run of tiles, which share A's rows and a group's B in its L2.

constexpr int BM2 = 256, BN2 = 256, BK2 = 64, STAGES = 4;
constexpr int SCALE_K = 128;  // bytes of K a scale word (4 blocks) covers

struct Lds2 {
  uint8_t a[STAGES][BM2 * BK2];
  uint8_t b[STAGES][BN2 * BK2];
  uint32_t as[STAGES][BM2];  // each row's scale word of the 128 bytes of K the step is in
  uint32_t bs[STAGES][BN2];
};

// Where a 64-byte LDS row's 16-byte chunk c sits: c ^ swizzle64(row). The 16 lanes
// that ds_read_b128 serves together read one chunk of 16 consecutive rows; rows r,
// r + 1, r + 2, r + 3 lie 64 bytes apart and (r / 4) % 4 spreads each such four over
// the 4 chunk places: 16 places of 16 bytes in 256, every bank once.
__device__ __forceinline__ int swizzle64(int row) { return (row >> 2) & 3; }

typedef int i32x4 __attribute__((ext_vector_type(4)));

// buffer_load_dword{,x4} ... lds: lane i's 4 (16) bytes at the resource's base + voffset +
// soffset land in LDS at M0 + 4 (16) i; offsets past the resource's size read 0. Written
// as inline assembly so that the compiler does not track these loads: left to itself it
// waits for every load in flight (vmcnt(0)) before any LDS read that might alias their
// destinations, which undoes the pipeline. The mainloop counts them itself
// (wait_loads), and nothing else in it touches vector memory.
__device__ __forceinline__ void load_lds16(i32x4 rsrc, uint32_t lds, int voffset, int soffset) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
               :: "s"(lds), "v"(voffset), "s"(rsrc), "s"(soffset) : "memory", "m0");
}
__device__ __forceinline__ void load_lds4(i32x4 rsrc, uint32_t lds, int voffset, int soffset) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, %3 offen lds"
               :: "s"(lds), "v"(voffset), "s"(rsrc), "s"(soffset) : "memory", "m0");
}

// A raw buffer resource (stride 0) over `bytes` bytes from `base`.
__device__ __forceinline__ i32x4 resource(const void* base, int64_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  i32x4 r;
  r[0] = __builtin_amdgcn_readfirstlane(static_cast<int>(a & 0xffffffffu));
  r[1] = __builtin_amdgcn_readfirstlane(static_cast<int>((a >> 32) & 0xffffu));
  r[2] = __builtin_amdgcn_readfirstlane(static_cast<int>(bytes > 0xffffffffLL ? 0xffffffffLL : bytes));
  r[3] = 0x00020000;
  return r;
}

// The LDS address of `p` (a location in the workgroup's LDS), as a scalar.
__device__ __forceinline__ uint32_t lds_at(const void* p) {
  return __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(reinterpret_cast<uintptr_t>(
      (__attribute__((address_space(3))) const void*)(p))));
}

// What a workgroup's lanes load for one operand's 256 rows from `row0` on: a resource
// over those rows (rows past the operand's read 0), and each lane's byte offsets in it
// for its 4 instructions of 16-byte chunks (16 rows an instruction, 4 lanes a row) and
// its scale word (64 rows an instruction).
struct Loads {
  i32x4 values, scales;
  int voff[4];
  int soff;
};

constexpr int LOADS_A_STEP = 10;  // load instructions a wave issues a step

__device__ __forceinline__ Loads loads_for(const Operand& op, int64_t row0) {
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  const int64_t rows = op.rows - row0, blocks = op.ld / 32;
  Loads ld;
  ld.values = resource(op.values + row0 * op.ld, rows * op.ld);
  ld.scales = resource(op.scales + row0 * blocks, rows * blocks);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = (w * 4 + i) * 16 + (l >> 2);
    ld.voff[i] = static_cast<int>(r * op.ld + 16 * ((l & 3) ^ swizzle64(r)));
  }
  ld.soff = static_cast<int>((w * 64 + l) * blocks);
  return ld;
}

// Direct load number q (0..9) of K step ks (64 bytes from 64 ks) into stage `st`: q < 8
// a 16-row slice of A's (even q) or B's (odd q) tile, 8 and 9 the scale words of A's
// and B's 64 rows of this wave.
__device__ __forceinline__ void issue_one(const Loads& la, const Loads& lb, int64_t ks, Lds2& lds,
                                         int st, int q) {
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (q < 8) {
    const int i = q >> 1, r0 = (w * 4 + i) * 16;
    const int k0 = static_cast<int>(ks * BK2);
    if ((q & 1) == 0) load_lds16(la.values, lds_at(&lds.a[st][r0 * BK2]), la.voff[i], k0);
    else load_lds16(lb.values, lds_at(&lds.b[st][r0 * BK2]), lb.voff[i], k0);
  } else {
    const int s0 = static_cast<int>(ks / 2 * 4);
    if (q == 8) load_lds4(la.scales, lds_at(&lds.as[st][w * 64]), la.soff, s0);
    else load_lds4(lb.scales, lds_at(&lds.bs[st][w * 64]), lb.soff, s0);
  }
}

// All 10 direct loads of K step ks into stage `st`.
__device__ __forceinline__ void issue2(const Loads& la, const Loads& lb, int64_t ks, Lds2& lds,
                                      int st) {
#pragma unroll
  for (int q = 0; q < LOADS_A_STEP; ++q) issue_one(la, lb, ks, lds, st, q);
}

// The workgroup barrier of the pipeline: this wave's LDS reads and writes are done,
// then s_barrier. Unlike __syncthreads it does not wait for the direct loads in flight
// (a fence would: vmcnt(0)), which wait_loads() waits for step by step.
__device__ __forceinline__ void barrier_lds() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Waits until at most `steps` steps' loads of this wave are in flight.
__device__ __forceinline__ void wait_loads(int64_t steps) {
  if (steps >= 3) asm volatile("s_waitcnt vmcnt(30)" ::: "memory");
  else if (steps == 2) asm volatile("s_waitcnt vmcnt(20)" ::: "memory");
  else if (steps == 1) asm volatile("s_waitcnt vmcnt(10)" ::: "memory");
  else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// Zeroes A's bytes of K outside [lo, hi) in stage `st`, step ks (a wgrad's edge steps):
// lane t takes row t.
__device__ __forceinline__ void mask2(Lds2& lds, int st, int64_t ks, int64_t lo, int64_t hi) {
  const int r = threadIdx.x;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int64_t k0 = ks * BK2 + 16 * c;
    if (k0 >= lo && k0 + 16 <= hi) continue;
    uint4* at = reinterpret_cast<uint4*>(&lds.a[st][r * BK2 + ((c ^ swizzle64(r)) << 4)]);
    *at = zero_outside(*at, k0, lo, hi);
  }
}

// A wave's operands of one step: 4 blocks of 32 rows of A and of B, and their scales.
struct Frag {
  v8i a[4], b[4];
  int sa[4], sb[4];
};

// 32 bytes of row `row` (lane half `half`): K chunks half and 2 + half of the step, the
// MFMA's two blocks of 32 (see operand()).
__device__ __forceinline__ v8i operand64(const uint8_t* tile, int row, int half) {
  const int sw = swizzle64(row);
  const uint4 lo = *reinterpret_cast<const uint4*>(tile + row * BK2 + ((half ^ sw) << 4));
  const uint4 hi = *reinterpret_cast<const uint4*>(tile + row * BK2 + (((2 + half) ^ sw) << 4));
  v8i v;
  v[0] = lo.x; v[1] = lo.y; v[2] = lo.z; v[3] = lo.w;
  v[4] = hi.x; v[5] = hi.y; v[6] = hi.z; v[7] = hi.w;
  return v;
}

// Part p (0..3) of a wave's operands of step ks from stage `st`: A's and B's 32-row
// block p and their scales.
__device__ __forceinline__ void read_part(Frag& f, const Lds2& lds, int st, int64_t ks, int p) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1, half = lane >> 5;
  // The step's two blocks are bytes 2 (ks % 2) and 2 (ks % 2) + 1 of the scale word;
  // lane half h scales block h.
  const int shift = 8 * ((static_cast<int>(ks & 1) << 1) + half);
  const int ra = wm * 128 + p * 32 + (lane & 31), rb = wn * 128 + p * 32 + (lane & 31);
  f.a[p] = operand64(lds.a[st], ra, half);
  f.b[p] = operand64(lds.b[st], rb, half);
  f.sa[p] = static_cast<int>((lds.as[st][ra] >> shift) & 0xffu);
  f.sb[p] = static_cast<int>((lds.bs[st][rb] >> shift) & 0xffu);
}

__device__ __forceinline__ void read_frag(Frag& f, const Lds2& lds, int st, int64_t ks) {
#pragma unroll
  for (int p = 0; p < 4; ++p) read_part(f, lds, st, ks, p);
}

__device__ __forceinline__ void multiply2(const Frag& f, v16f acc[4][4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
      acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(f.b[j], f.a[i], acc[i][j], 0, 0,
                                                                 0, f.sb[j], 0, f.sa[i]);
}

// acc += A[a_row0 + r] . B[b_row0 + c] over K steps [ks_begin, ks_end) of 64 bytes; with
// `mask`, A's bytes of K outside [mlo, mhi) count as 0 (in the first and last steps).
//
// Step k: wait for this wave's loads of step k + 1 and pass the barrier (step k + 1's
// stage is then whole, and every wave has read step k's, whose stage step k + 4's
// loads take); then the 16 MFMAs of step k on `cur`, each after a slice of the memory
// work: one of step k + 4's loads and a part of step k + 1's LDS reads into `nxt`. A
// wave issues in order, so a load that waits for the memory pipe to take it waits while
// an MFMA runs, not while the matrix core idles; sched_barrier keeps that order.
__device__ __forceinline__ void mainloop2(const Operand& A, int64_t a_row0, const Operand& B,
                                          int64_t b_row0, int64_t ks_begin, int64_t ks_end,
                                          bool mask, int64_t mlo, int64_t mhi, Lds2& lds,
                                          v16f acc[4][4]) {
  const int64_t n = ks_end - ks_begin;
  if (n <= 0) return;
  const Loads la = loads_for(A, a_row0), lb = loads_for(B, b_row0);
  auto edge = [&](int64_t k) { return mask && (k == 0 || k == n - 1); };
  for (int64_t s = 0; s < STAGES && s < n; ++s) issue2(la, lb, ks_begin + s, lds, static_cast<int>(s));
  wait_loads(n - 1 < 3 ? n - 1 : 3);
  barrier_lds();
  if (edge(0)) {
    mask2(lds, 0, ks_begin, mlo, mhi);
    barrier_lds();
  }
  Frag cur, nxt;
  read_frag(cur, lds, 0, ks_begin);
  for (int64_t k = 0; k < n; ++k) {
    const bool more = k + 1 < n, load = k + 4 < n;
    if (more) {
      const int64_t later = n - 2 - k;
      wait_loads(later < 2 ? later : 2);
    }
    barrier_lds();
    if (more && edge(k + 1)) {
      mask2(lds, static_cast<int>((k + 1) % STAGES), ks_begin + k + 1, mlo, mhi);
      barrier_lds();
    }
    const int st_next = static_cast<int>((k + 1) % STAGES), st_load = static_cast<int>(k % STAGES);
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      const int i = q >> 2, j = q & 3;
      if (load && q < LOADS_A_STEP) issue_one(la, lb, ks_begin + k + 4, lds, st_load, q);
      if (more && j == 0) read_part(nxt, lds, st_next, ks_begin + k + 1, i);
      __builtin_amdgcn_sched_barrier(0);
      acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(cur.b[j], cur.a[i], acc[i][j], 0,
                                                                 0, 0, cur.sb[j], 0, cur.sa[i]);
      __builtin_amdgcn_sched_barrier(0);
    }
    cur = nxt;
  }
  // Every wave is done with every stage before the caller's LDS reuse.
  __syncthreads();
}

template <typename T>
__device__ __forceinline__ void store_run(T* at, const v16f& acc, int g);
template <>
__device__ __forceinline__ void store_run<uint16_t>(uint16_t* at, const v16f& acc, int g) {
  *reinterpret_cast<uint2*>(at) =
      make_uint2(pack_bf16x2(acc[4 * g], acc[4 * g + 1]), pack_bf16x2(acc[4 * g + 2], acc[4 * g + 3]));
}
template <>
__device__ __forceinline__ void store_run<float>(float* at, const v16f& acc, int g) {
  *reinterpret_cast<float4*>(at) = make_float4(acc[4 * g], acc[4 * g + 1], acc[4 * g + 2], acc[4 * g + 3]);
}

// Stores rows [row_lo, row_hi) and columns below n_cols (a multiple of 4) of the tile
// at (row0, col0): lane l holds row l % 32 of each 32-row block and, in register run g,
// columns 8 g + 4 (l / 32) .. + 3 of each 32-column block.
template <typename T>
__device__ __forceinline__ void store2(const v16f acc[4][4], T* out, int64_t ld, int64_t row0,
                                       int64_t col0, int64_t row_lo, int64_t row_hi,
                                       int64_t n_cols) {
  const int t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  const int wm = wave >> 1, wn = wave & 1;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t row = row0 + wm * 128 + i * 32 + (lane & 31);
    if (row < row_lo || row >= row_hi) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int64_t col = col0 + wn * 128 + j * 32 + 8 * g + 4 * (lane >> 5);
        if (col < n_cols) store_run<T>(out + row * ld + col, acc[i][j], g);
      }
  }
}

template <typename T>
__device__ void store_zeros2(T* out, int64_t ld, int64_t row_lo, int64_t row_hi, int64_t col0,
                             int64_t n_cols) {
  // 4 columns a lane-step: n_cols is a multiple of 4
  const int64_t width = ((col0 + BN2 < n_cols ? col0 + BN2 : n_cols) - col0) / 4;
  const v16f zero = {};
  for (int64_t i = threadIdx.x; i < (row_hi - row_lo) * width; i += THREADS)
    store_run<T>(out + (row_lo + i / width) * ld + col0 + 4 * (i % width), zero, 0);
}

// The workgroup's tile in a grid renumbered so that XCD x (workgroup id % 8) takes the
// contiguous tiles [x per, (x + 1) per); -1 past the tiles.
__device__ __forceinline__ int64_t xcd_tile(int64_t total) {
  const int64_t per = (total + 7) / 8;
  const int64_t logical = static_cast<int64_t>(blockIdx.x % 8) * per + blockIdx.x / 8;
  return logical < total ? logical : -1;
}

__device__ __forceinline__ void zero_acc(v16f acc[4][4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int q = 0; q < 16; ++q) acc[i][j][q] = 0.0f;
}

template <typename T>
__global__ __launch_bounds__(THREADS) __attribute__((amdgpu_waves_per_eu(1, 1))) void rows2_kernel(
    Operand A, Operand B, int32_t groups, int64_t n, int64_t height, const Tile* __restrict__ tiles,
    int64_t col_tiles, int64_t total, T* __restrict__ y) {
  extern __shared__ __align__(16) uint8_t smem[];
  Lds2& lds = *reinterpret_cast<Lds2*>(smem);
  const int64_t id = xcd_tile(total);
  if (id < 0) return;
  const int64_t col0 = (id % col_tiles) * BN2;
  Tile tile = tiles[id / col_tiles];
  if (tile.hi > height) tile.hi = static_cast<int32_t>(height);
  if (tile.lo >= tile.hi) return;
  if (tile.group >= groups) {  // rows past the groups
    store_zeros2(y, n, tile.lo, tile.hi, col0, n);
    return;
  }
  Operand b = B;
  b.values += static_cast<int64_t>(tile.group) * B.rows * B.ld;
  b.scales += static_cast<int64_t>(tile.group) * B.rows * (B.ld / 32);
  v16f acc[4][4];
  zero_acc(acc);
  mainloop2(A, tile.lo, b, col0, 0, A.ld / BK2, false, 0, 0, lds, acc);
  store2(acc, y, n, tile.lo, col0, tile.lo, tile.hi, n);
}

template <typename T>
__global__ __launch_bounds__(THREADS) __attribute__((amdgpu_waves_per_eu(1, 1))) void contract2_kernel(
    Operand A, Operand B, int32_t groups, const int32_t* __restrict__ starts, int64_t d_tiles,
    int64_t f_tiles, int64_t total, T* __restrict__ dw) {
  extern __shared__ __align__(16) uint8_t smem[];
  Lds2& lds = *reinterpret_cast<Lds2*>(smem);
  const int64_t id = xcd_tile(total);
  if (id < 0) return;
  const int64_t per_group = d_tiles * f_tiles;
  const int64_t g = id / per_group, rest = id % per_group;
  const int64_t row0 = (rest / f_tiles) * BM2, col0 = (rest % f_tiles) * BN2;
  const int64_t start = starts[g], end = starts[g + 1];
  v16f acc[4][4];
  zero_acc(acc);
  if (end > start) {
    const int64_t kt_begin = start / BK2, kt_end = (end + BK2 - 1) / BK2;
    const bool ragged = (start % BK2) != 0 || (end % BK2) != 0;
    mainloop2(A, row0, B, col0, kt_begin, kt_end, ragged, start, end, lds, acc);
  }
  store2(acc, dw + g * A.rows * B.rows, B.rows, row0, col0, row0, A.rows, B.rows);
}

// Lets a kernel take `bytes` (over 64 KiB) of dynamic LDS; gfx950 has 160 KiB a CU.
template <typename K>
int allow_lds(K kernel, size_t bytes, const char* name) {
  hipError_t err = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                       hipFuncAttributeMaxDynamicSharedMemorySize,
                                       static_cast<int>(bytes));
  if (err != hipSuccess) return fail(BUX_E_LAUNCH, "%s: %s", name, hipGetErrorString(err));
  return BUX_OK;
}

// Whether the v2 kernels take these shapes: K whole 128-byte steps, output columns a
// multiple of 4.
bool fits_v2(int64_t k, int64_t n) { return k % SCALE_K == 0 && n % 4 == 0; }

// Whether an operand's bytes fit the v2 kernels' 32-bit buffer offsets.
bool offsets_fit(int64_t rows, int64_t ld) { return rows * ld < (1LL << 31); }

int64_t row_slots(int32_t groups, int64_t m, int64_t height, int tile_rows) {
  const int64_t rows = m > height ? m : height;
  // tiles of rows, plus one a group (and one for the rows past them) at most
  return ceil_div(rows, tile_rows) + groups + 1;
}

template <typename T>
int launch_rows(const Operand& A, const Operand& B, int32_t groups, int64_t n, int64_t height,
                const Tile* tiles, int64_t slots, bool v2, void* y, hipStream_t s) {
  if (v2) {
    const int64_t col_tiles = ceil_div(n, BN2);
    const int64_t total = slots * col_tiles;
    const int64_t blocks = 8 * ceil_div(total, 8);
    if (blocks >= (1LL << 31)) return fail(BUX_E_ARGUMENT, "bux_mx_grouped_rows: too many tiles");
    if (int rc = allow_lds(rows2_kernel<T>, sizeof(Lds2), "rows2_kernel")) return rc;
    hipLaunchKernelGGL(rows2_kernel<T>, dim3(static_cast<unsigned>(blocks)), dim3(THREADS),
                       sizeof(Lds2), s, A, B, groups, n, height, tiles, col_tiles, total,
                       static_cast<T*>(y));
    return launched("rows2_kernel");
  }
  const int64_t col_tiles = ceil_div(n, BN);
  const int64_t blocks = slots * col_tiles;
  if (blocks >= (1LL << 31)) return fail(BUX_E_ARGUMENT, "bux_mx_grouped_rows: too many tiles");
  if (int rc = allow_lds(rows_kernel<T>, sizeof(Lds), "rows_kernel")) return rc;
  hipLaunchKernelGGL(rows_kernel<T>, dim3(static_cast<unsigned>(blocks)), dim3(THREADS),
                     sizeof(Lds), s, A, B, groups, n, height, tiles, col_tiles,
                     static_cast<T*>(y));
  return launched("rows_kernel");
}

template <typename T>
int launch_contract(const Operand& A, const Operand& B, int32_t groups, const int32_t* starts,
                    bool v2, void* dw, hipStream_t s) {
  if (v2) {
    const int64_t d_tiles = ceil_div(A.rows, BM2), f_tiles = ceil_div(B.rows, BN2);
    const int64_t total = static_cast<int64_t>(groups) * d_tiles * f_tiles;
    const int64_t blocks = 8 * ceil_div(total, 8);
    if (blocks >= (1LL << 31)) return fail(BUX_E_ARGUMENT, "bux_mx_grouped_contract: too many tiles");
    if (int rc = allow_lds(contract2_kernel<T>, sizeof(Lds2), "contract2_kernel")) return rc;
    hipLaunchKernelGGL(contract2_kernel<T>, dim3(static_cast<unsigned>(blocks)), dim3(THREADS),
                       sizeof(Lds2), s, A, B, groups, starts, d_tiles, f_tiles, total,
                       static_cast<T*>(dw));
    return launched("contract2_kernel");
  }
  const int64_t d_tiles = ceil_div(A.rows, BM), f_tiles = ceil_div(B.rows, BN);
  const int64_t blocks = static_cast<int64_t>(groups) * d_tiles * f_tiles;
  if (blocks >= (1LL << 31)) return fail(BUX_E_ARGUMENT, "bux_mx_grouped_contract: too many tiles");
  if (int rc = allow_lds(contract_kernel<T>, sizeof(Lds), "contract_kernel")) return rc;
  hipLaunchKernelGGL(contract_kernel<T>, dim3(static_cast<unsigned>(blocks)), dim3(THREADS),
                     sizeof(Lds), s, A, B, groups, starts, d_tiles, f_tiles, static_cast<T*>(dw));
  return launched("contract_kernel");
}

size_t align256(size_t v) { return (v + 255) & ~static_cast<size_t>(255); }

}  // namespace
}  // namespace bux

extern "C" size_t bux_mx_grouped_rows_workspace_size(int32_t groups, int64_t m, int64_t height) {
  using namespace bux;
  // room for the longer of the two kernels' tile lists (128-row tiles)
  return align256(static_cast<size_t>(groups + 1) * sizeof(int32_t)) +
         static_cast<size_t>(row_slots(groups, m, height, BM)) * sizeof(Tile);
}

extern "C" int bux_mx_grouped_rows(const uint8_t* a_values, const uint8_t* a_scales,
                                   const uint8_t* b_values, const uint8_t* b_scales,
                                   const int32_t* sizes, int32_t groups, int64_t m, int64_t n,
                                   int64_t k, int64_t height, int out_dtype, void* y,
                                   void* workspace, size_t workspace_bytes, void* stream) {
  using namespace bux;
  clear_error();
  BUX_CHECK(groups >= 1 && groups <= MAX_GROUPS, "bux_mx_grouped_rows: groups=%d outside [1, %d]",
            groups, MAX_GROUPS);
  BUX_CHECK(m >= 0 && n > 0 && k > 0 && height >= 0 && height < (1LL << 31) && m < (1LL << 31),
            "bux_mx_grouped_rows: bad shape m=%lld n=%lld k=%lld height=%lld", (long long)m,
            (long long)n, (long long)k, (long long)height);
  BUX_CHECK(k % 32 == 0, "bux_mx_grouped_rows: k=%lld is not a multiple of 32", (long long)k);
  BUX_CHECK(out_dtype == BUX_BF16 || out_dtype == BUX_F32, "bux_mx_grouped_rows: out_dtype=%d",
            out_dtype);
  BUX_CHECK(sizes && b_values && b_scales && y && (m == 0 || (a_values && a_scales)),
            "bux_mx_grouped_rows: NULL buffer");
  const size_t need = bux_mx_grouped_rows_workspace_size(groups, m, height);
  if (workspace == nullptr || workspace_bytes < need)
    return fail(BUX_E_WORKSPACE, "bux_mx_grouped_rows: workspace of %zu bytes, %zu needed",
                workspace_bytes, need);
  if (height == 0) return BUX_OK;
  hipStream_t s = as_stream(stream);
  int32_t* starts = static_cast<int32_t*>(workspace);
  Tile* tiles = reinterpret_cast<Tile*>(static_cast<uint8_t*>(workspace) +
                                        align256(static_cast<size_t>(groups + 1) * sizeof(int32_t)));
  const bool v2 = fits_v2(k, n) && m > 0 && offsets_fit(m, k) && offsets_fit(n, k);
  const int tile_rows = v2 ? BM2 : BM;
  const int64_t slots = row_slots(groups, m, height, tile_rows);
  hipLaunchKernelGGL(prologue_kernel, dim3(1), dim3(THREADS), 0, s, sizes, groups, height, slots,
                     tile_rows, v2, starts, tiles);
  if (int rc = launched("prologue_kernel")) return rc;
  const Operand A{a_values, a_scales, k, m};
  const Operand B{b_values, b_scales, k, n};
  return out_dtype == BUX_BF16
             ? launch_rows<uint16_t>(A, B, groups, n, height, tiles, slots, v2, y, s)
             : launch_rows<float>(A, B, groups, n, height, tiles, slots, v2, y, s);
}

extern "C" size_t bux_mx_grouped_contract_workspace_size(int32_t groups) {
  return static_cast<size_t>(groups + 1) * sizeof(int32_t);
}

extern "C" int bux_mx_grouped_contract(const uint8_t* a_values, const uint8_t* a_scales,
                                       const uint8_t* b_values, const uint8_t* b_scales,
                                       const int32_t* sizes, int32_t groups, int64_t d, int64_t f,
                                       int64_t m, int out_dtype, void* dw, void* workspace,
                                       size_t workspace_bytes, void* stream) {
  using namespace bux;
  clear_error();
  BUX_CHECK(groups >= 1 && groups <= MAX_GROUPS,
            "bux_mx_grouped_contract: groups=%d outside [1, %d]", groups, MAX_GROUPS);
  BUX_CHECK(d > 0 && f > 0 && m >= 0, "bux_mx_grouped_contract: bad shape d=%lld f=%lld m=%lld",
            (long long)d, (long long)f, (long long)m);
  BUX_CHECK(m % 32 == 0, "bux_mx_grouped_contract: m=%lld is not a multiple of 32", (long long)m);
  BUX_CHECK(out_dtype == BUX_BF16 || out_dtype == BUX_F32, "bux_mx_grouped_contract: out_dtype=%d",
            out_dtype);
  BUX_CHECK(sizes && dw && (m == 0 || (a_values && a_scales && b_values && b_scales)),
            "bux_mx_grouped_contract: NULL buffer");
  const size_t need = bux_mx_grouped_contract_workspace_size(groups);
  if (workspace == nullptr || workspace_bytes < need)
    return fail(BUX_E_WORKSPACE, "bux_mx_grouped_contract: workspace of %zu bytes, %zu needed",
                workspace_bytes, need);
  hipStream_t s = as_stream(stream);
  int32_t* starts = static_cast<int32_t*>(workspace);
  hipLaunchKernelGGL(prologue_kernel, dim3(1), dim3(THREADS), 0, s, sizes, groups, 0, 0, BM, false,
                     starts, nullptr);
  if (int rc = launched("prologue_kernel")) return rc;
  // The operands' K is m: each of a's d rows (b's f rows) is m bytes.
  const Operand A{a_values, a_scales, m, d};
  const Operand B{b_values, b_scales, m, f};
  const bool v2 = fits_v2(m, f) && m > 0 && offsets_fit(d, m) && offsets_fit(f, m);
  return out_dtype == BUX_BF16 ? launch_contract<uint16_t>(A, B, groups, starts, v2, dw, s)
                               : launch_contract<float>(A, B, groups, starts, v2, dw, s);
}
