// bfloat16 grouped GEMMs (the experts in "compute" precision) on CDNA4's
// v_mfma_f32_32x32x16_bf16, float32 accumulation, bfloat16 out.
//
//   rows      y[i] = x[i] w[g(i)]   (w [g, k, n]) or x[i] w[g(i)]^T (w [g, n, k])
//             grouped.dot / jax.lax.ragged_dot, src/bux/architecture/experts/
//             grouped.py:90-102: rows past sum(sizes) are 0.
//   contract  dw[g] = x[rows of g]^T dy[rows of g]   grouped.py:105-146.
//
// One mainloop computes C[r][c] = sum_k A(r, k) B(c, k) over a 128 x 128 tile, in steps
// of 32 of k through LDS ([row][k], rows padded to 80 bytes so that ds_read_b128 of 32
// consecutive rows spreads over the banks). An operand is "k-major" (A(r, k) at
// p[r ld + k]) or "mn-major" (p[k ld + r]); an mn-major operand is transposed on its
// way into LDS. Rows (or ks) outside a window read 0, which is how a tile that several
// groups share multiplies each group's rows by its own matrix into one accumulator.
// Not the MXFP8 hot path: it serves the experts' "compute" format (config 1).

#include "common.h"

namespace bux {
namespace {

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int BM = 128, BN = 128, BK = 32, THREADS = 256;
constexpr int PITCH = 40;  // bfloat16 a row of an LDS tile
constexpr int MAX_GROUPS = 4096;

struct Operand {
  const uint16_t* p;
  int64_t ld;
  bool k_major;
  int64_t rows;  // rows r there are
  int64_t ks;    // ks there are
};

struct Window {
  int64_t lo, hi;  // rows (k_major) or ks of A that read as themselves; others read 0
  bool on_k;
};

// Global -> LDS for K step k0 of an operand's 128 rows from row0.
__device__ __forceinline__ void load_tile(uint16_t* lds, const Operand& op, int64_t row0,
                                          int64_t k0, const Window* window) {
  const int t = threadIdx.x;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    if (op.k_major) {
      const int r = (t >> 2) + 64 * i, chunk = t & 3;
      const int64_t row = row0 + r, k = k0 + 8 * chunk;
      uint4 v = make_uint4(0, 0, 0, 0);
      bool ok = row < op.rows && k < op.ks;
      if (window && !window->on_k) ok = ok && row >= window->lo && row < window->hi;
      if (window && window->on_k) ok = ok && k >= window->lo && k + 8 <= window->hi;
      if (ok) v = *reinterpret_cast<const uint4*>(op.p + row * op.ld + k);
      if (window && window->on_k && row < op.rows && k < op.ks && !ok) {
        // a chunk across the window's edge: element by element
        uint16_t e[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int64_t kk = k + j;
          e[j] = (kk >= window->lo && kk < window->hi) ? op.p[row * op.ld + kk] : 0;
        }
        v = make_uint4(e[0] | (e[1] << 16), e[2] | (e[3] << 16), e[4] | (e[5] << 16),
                       e[6] | (e[7] << 16));
      }
      *reinterpret_cast<uint4*>(lds + r * PITCH + 8 * chunk) = v;
    } else {
      const int kk = (t >> 4) + 16 * i, chunk = t & 15;
      const int64_t k = k0 + kk, row = row0 + 8 * chunk;
      uint4 v = make_uint4(0, 0, 0, 0);
      bool ok = k < op.ks && row < op.rows;
      if (window && window->on_k) ok = ok && k >= window->lo && k < window->hi;
      if (ok) v = *reinterpret_cast<const uint4*>(op.p + k * op.ld + row);
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        uint16_t e = static_cast<uint16_t>(w[j >> 1] >> (16 * (j & 1)));
        if (window && !window->on_k && (row + j < window->lo || row + j >= window->hi)) e = 0;
        lds[(8 * chunk + j) * PITCH + kk] = e;
      }
    }
  }
}

__device__ __forceinline__ v8bf fragment(const uint16_t* lds, int row, int k) {
  const uint4 v = *reinterpret_cast<const uint4*>(lds + row * PITCH + k);
  return __builtin_bit_cast(v8bf, v);
}

__device__ void mainloop(const Operand& A, int64_t a_row0, const Operand& B, int64_t b_row0,
                         int64_t k_begin, int64_t k_end, const Window* window, uint16_t* lds_a,
                         uint16_t* lds_b, v16f acc[2][2]) {
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  for (int64_t k0 = k_begin; k0 < k_end; k0 += BK) {
    load_tile(lds_a, A, a_row0, k0, window);
    load_tile(lds_b, B, b_row0, k0, nullptr);
    __syncthreads();
#pragma unroll
    for (int sub = 0; sub < 2; ++sub) {
      const int k = 16 * sub + 8 * (lane >> 5);
      v8bf a[2], b[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        a[i] = fragment(lds_a, wm * 64 + 32 * i + (lane & 31), k);
        b[i] = fragment(lds_b, wn * 64 + 32 * i + (lane & 31), k);
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
    }
    __syncthreads();
  }
}

__device__ void store(const v16f acc[2][2], uint16_t* out, int64_t ld, int64_t row0, int64_t col0,
                      int64_t rows, int64_t cols) {
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int wm = wave >> 1, wn = wave & 1;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int64_t col = col0 + wn * 64 + 32 * j + (lane & 31);
      if (col >= cols) continue;
#pragma unroll
      for (int q = 0; q < 16; ++q) {
        const int64_t row = row0 + wm * 64 + 32 * i + 8 * (q >> 2) + 4 * (lane >> 5) + (q & 3);
        if (row < rows) out[row * ld + col] = f32_to_bf16(acc[i][j][q]);
      }
    }
}

// starts[0..groups] of the sizes, in LDS, by one workgroup.
__device__ void group_starts(const int32_t* sizes, int32_t groups, int32_t* starts,
                             int32_t* partial) {
  const int t = threadIdx.x;
  const int per = (groups + THREADS - 1) / THREADS;
  const int lo = t * per, hi = lo + per < groups ? lo + per : groups;
  int32_t sum = 0;
  for (int i = lo; i < hi; ++i) sum += sizes[i];
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
    starts[i] = run;
    run += sizes[i];
  }
  if (t == THREADS - 1) starts[groups] = partial[THREADS - 1];
  __syncthreads();
}

__global__ __launch_bounds__(THREADS) void rows_kernel(const uint16_t* __restrict__ x,
                                                       const uint16_t* __restrict__ w,
                                                       int w_transposed,
                                                       const int32_t* __restrict__ sizes,
                                                       int32_t groups, int64_t m, int64_t n,
                                                       int64_t k, int64_t col_tiles,
                                                       uint16_t* __restrict__ y) {
  __shared__ __align__(16) uint16_t lds_a[BM * PITCH];
  __shared__ __align__(16) uint16_t lds_b[BN * PITCH];
  __shared__ int32_t starts[MAX_GROUPS + 1];
  __shared__ int32_t partial[THREADS];
  const int64_t row0 = (blockIdx.x / col_tiles) * BM;
  const int64_t col0 = (blockIdx.x % col_tiles) * BN;
  group_starts(sizes, groups, starts, partial);
  v16f acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int q = 0; q < 16; ++q) acc[i][j][q] = 0.0f;
  const Operand A{x, k, true, m, k};
  for (int g = 0; g < groups; ++g) {
    const int64_t lo = starts[g], hi = starts[g + 1];
    if (hi <= row0 || lo >= row0 + BM || lo >= hi) continue;
    const uint16_t* wg = w + static_cast<int64_t>(g) * k * n;
    const Operand B = w_transposed ? Operand{wg, k, true, n, k} : Operand{wg, n, false, n, k};
    const Window window{lo, hi, false};
    mainloop(A, row0, B, col0, 0, k, &window, lds_a, lds_b, acc);
  }
  store(acc, y, n, row0, col0, m, n);
}

__global__ __launch_bounds__(THREADS) void contract_kernel(const uint16_t* __restrict__ x,
                                                           const uint16_t* __restrict__ dy,
                                                           const int32_t* __restrict__ sizes,
                                                           int32_t groups, int64_t m, int64_t k,
                                                           int64_t n, int64_t k_tiles,
                                                           int64_t n_tiles,
                                                           uint16_t* __restrict__ dw) {
  __shared__ __align__(16) uint16_t lds_a[BM * PITCH];
  __shared__ __align__(16) uint16_t lds_b[BN * PITCH];
  __shared__ int32_t starts[MAX_GROUPS + 1];
  __shared__ int32_t partial[THREADS];
  const int64_t per_group = k_tiles * n_tiles;
  const int64_t g = blockIdx.x / per_group, rest = blockIdx.x % per_group;
  const int64_t row0 = (rest / n_tiles) * BM, col0 = (rest % n_tiles) * BN;
  group_starts(sizes, groups, starts, partial);
  v16f acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int q = 0; q < 16; ++q) acc[i][j][q] = 0.0f;
  const int64_t lo = starts[g], hi = starts[g + 1];
  if (hi > lo) {
    // A(r, i) = x[i][r] and B(c, i) = dy[i][c]: both mn-major over the rows i.
    const Operand A{x, k, false, k, m};
    const Operand B{dy, n, false, n, m};
    const Window window{lo, hi, true};
    mainloop(A, row0, B, col0, lo / BK * BK, hi, &window, lds_a, lds_b, acc);
  }
  store(acc, dw + g * k * n, n, row0, col0, k, n);
}

}  // namespace
}  // namespace bux

extern "C" int bux_bf16_grouped_rows(const uint16_t* x, const uint16_t* w, int w_transposed,
                                     const int32_t* sizes, int32_t groups, int64_t m, int64_t n,
                                     int64_t k, uint16_t* y, void* stream) {
  using namespace bux;
  clear_error();
  BUX_CHECK(groups >= 1 && groups <= MAX_GROUPS, "bux_bf16_grouped_rows: groups=%d outside [1, %d]",
            groups, MAX_GROUPS);
  BUX_CHECK(m >= 0 && n > 0 && k > 0, "bux_bf16_grouped_rows: bad shape m=%lld n=%lld k=%lld",
            (long long)m, (long long)n, (long long)k);
  BUX_CHECK(n % 8 == 0 && k % 8 == 0, "bux_bf16_grouped_rows: n=%lld and k=%lld must be multiples of 8",
            (long long)n, (long long)k);
  if (m == 0) return BUX_OK;
  BUX_CHECK(x && w && sizes && y, "bux_bf16_grouped_rows: NULL buffer");
  const int64_t col_tiles = ceil_div(n, BN);
  const int64_t blocks = ceil_div(m, BM) * col_tiles;
  BUX_CHECK(blocks < (1LL << 31), "bux_bf16_grouped_rows: too many tiles");
  hipLaunchKernelGGL(rows_kernel, dim3(static_cast<unsigned>(blocks)), dim3(THREADS), 0,
                     as_stream(stream), x, w, w_transposed, sizes, groups, m, n, k, col_tiles, y);
  return launched("bf16 rows_kernel");
}

extern "C" int bux_bf16_grouped_contract(const uint16_t* x, const uint16_t* dy, const int32_t* sizes,
                                         int32_t groups, int64_t m, int64_t k, int64_t n,
                                         uint16_t* dw, void* stream) {
  using namespace bux;
  clear_error();
  BUX_CHECK(groups >= 1 && groups <= MAX_GROUPS,
            "bux_bf16_grouped_contract: groups=%d outside [1, %d]", groups, MAX_GROUPS);
  BUX_CHECK(m >= 0 && n > 0 && k > 0, "bux_bf16_grouped_contract: bad shape m=%lld k=%lld n=%lld",
            (long long)m, (long long)k, (long long)n);
  BUX_CHECK(n % 8 == 0 && k % 8 == 0,
            "bux_bf16_grouped_contract: k=%lld and n=%lld must be multiples of 8", (long long)k,
            (long long)n);
  BUX_CHECK(x && dy && sizes && dw, "bux_bf16_grouped_contract: NULL buffer");
  const int64_t k_tiles = ceil_div(k, BM), n_tiles = ceil_div(n, BN);
  const int64_t blocks = static_cast<int64_t>(groups) * k_tiles * n_tiles;
  BUX_CHECK(blocks < (1LL << 31), "bux_bf16_grouped_contract: too many tiles");
  hipLaunchKernelGGL(contract_kernel, dim3(static_cast<unsigned>(blocks)), dim3(THREADS), 0,
                     as_stream(stream), x, dy, sizes, groups, m, k, n, k_tiles, n_tiles, dw);
  return launched("bf16 contract_kernel");
}
