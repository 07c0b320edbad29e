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
// row's eight 16-byte chunks sit at chunk ^ (row % 8), so that the 32 lanes reading one
// chunk of 32 consecutive rows spread over every bank.
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
__global__ __launch_bounds__(THREADS) void prologue_kernel(const int32_t* __restrict__ sizes,
                                                           int32_t groups, int64_t height,
                                                           int64_t slots,
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
  for (int g = t; g < all; g += THREADS) {
    const int64_t s = size_of(g), start = starts[g];
    before[g] = s > 0 ? static_cast<int32_t>((start + s + BM - 1) / BM - start / BM) : 0;
  }
  __syncthreads();
  const int32_t used = block_scan(before, all, partial);
  for (int g = t; g < all; g += THREADS) {
    const int64_t s = size_of(g), start = starts[g], end = start + s;
    if (s == 0) continue;
    const int64_t first = start / BM, count = (end + BM - 1) / BM - first;
    // Sizes summing past the rows there are would list more tiles than there are
    // slots: those are dropped, never written past the list.
    for (int64_t j = 0; j < count && before[g] + j < slots; ++j) {
      const int64_t tile = first + j;
      Tile out;
      out.group = g;
      out.lo = static_cast<int32_t>(start > tile * BM ? start : tile * BM);
      out.hi = static_cast<int32_t>(end < (tile + 1) * BM ? end : (tile + 1) * BM);
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
    const int at = r * BK + ((chunk ^ (r & 7)) << 4);
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
  const uint4 lo = *reinterpret_cast<const uint4*>(tile + row * BK + (((c0) ^ (row & 7)) << 4));
  const uint4 hi = *reinterpret_cast<const uint4*>(tile + row * BK + (((c0 + 2) ^ (row & 7)) << 4));
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

// Lets a kernel take sizeof(Lds) (over 64 KiB) of dynamic LDS; gfx950 has 160 KiB a CU.
template <typename K>
int allow_lds(K kernel, const char* name) {
  hipError_t err = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                       hipFuncAttributeMaxDynamicSharedMemorySize,
                                       static_cast<int>(sizeof(Lds)));
  if (err != hipSuccess) return fail(BUX_E_LAUNCH, "%s: %s", name, hipGetErrorString(err));
  return BUX_OK;
}

template <typename T>
int launch_rows(const Operand& A, const Operand& B, int32_t groups, int64_t n, int64_t height,
                const Tile* tiles, int64_t slots, void* y, hipStream_t s) {
  const int64_t col_tiles = ceil_div(n, BN);
  const int64_t blocks = slots * col_tiles;
  if (blocks >= (1LL << 31)) return fail(BUX_E_ARGUMENT, "bux_mx_grouped_rows: too many tiles");
  if (int rc = allow_lds(rows_kernel<T>, "rows_kernel")) return rc;
  hipLaunchKernelGGL(rows_kernel<T>, dim3(static_cast<unsigned>(blocks)), dim3(THREADS),
                     sizeof(Lds), s, A, B, groups, n, height, tiles, col_tiles,
                     static_cast<T*>(y));
  return launched("rows_kernel");
}

template <typename T>
int launch_contract(const Operand& A, const Operand& B, int32_t groups, const int32_t* starts,
                    void* dw, hipStream_t s) {
  const int64_t d_tiles = ceil_div(A.rows, BM), f_tiles = ceil_div(B.rows, BN);
  const int64_t blocks = static_cast<int64_t>(groups) * d_tiles * f_tiles;
  if (blocks >= (1LL << 31)) return fail(BUX_E_ARGUMENT, "bux_mx_grouped_contract: too many tiles");
  if (int rc = allow_lds(contract_kernel<T>, "contract_kernel")) return rc;
  hipLaunchKernelGGL(contract_kernel<T>, dim3(static_cast<unsigned>(blocks)), dim3(THREADS),
                     sizeof(Lds), s, A, B, groups, starts, d_tiles, f_tiles, static_cast<T*>(dw));
  return launched("contract_kernel");
}

int64_t row_slots(int32_t groups, int64_t m, int64_t height) {
  const int64_t rows = m > height ? m : height;
  return ceil_div(rows, BM) + groups;  // tiles of rows, plus one a group but the first
}

size_t align256(size_t v) { return (v + 255) & ~static_cast<size_t>(255); }

}  // namespace
}  // namespace bux

extern "C" size_t bux_mx_grouped_rows_workspace_size(int32_t groups, int64_t m, int64_t height) {
  using namespace bux;
  return align256(static_cast<size_t>(groups + 1) * sizeof(int32_t)) +
         static_cast<size_t>(row_slots(groups, m, height)) * sizeof(Tile);
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
  const int64_t slots = row_slots(groups, m, height);
  hipLaunchKernelGGL(prologue_kernel, dim3(1), dim3(THREADS), 0, s, sizes, groups, height, slots,
                     starts, tiles);
  if (int rc = launched("prologue_kernel")) return rc;
  const Operand A{a_values, a_scales, k, m};
  const Operand B{b_values, b_scales, k, n};
  return out_dtype == BUX_BF16
             ? launch_rows<uint16_t>(A, B, groups, n, height, tiles, slots, y, s)
             : launch_rows<float>(A, B, groups, n, height, tiles, slots, y, s);
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
  hipLaunchKernelGGL(prologue_kernel, dim3(1), dim3(THREADS), 0, s, sizes, groups, 0, 0, starts,
                     nullptr);
  if (int rc = launched("prologue_kernel")) return rc;
  // The operands' K is m: each of a's d rows (b's f rows) is m bytes.
  const Operand A{a_values, a_scales, m, d};
  const Operand B{b_values, b_scales, m, f};
  return out_dtype == BUX_BF16 ? launch_contract<uint16_t>(A, B, groups, starts, dw, s)
                               : launch_contract<float>(A, B, groups, starts, dw, s);
}
