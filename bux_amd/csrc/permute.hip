// Sorting an MoE's picks by expert, stably: order, its inverse, each expert's size
// and the groups' offsets (src/bux/architecture/experts/moe.py:776-797: a stable
// argsort of the flat picks with those outside [0, E) as E, bincount, argsort of the
// order; the offsets cumsum(sizes) - sizes of grouped_mxfp8.py:142).
//
// A counting sort over segments of 256 picks (one wave a segment):
//   1. count:   each wave counts its segment's picks per bin (E bins and one for the
//               picks outside) in LDS; counts[bin][segment] goes to the workspace.
//   2. rows:    a workgroup a bin scans its row of counts exclusively, in place, and
//               leaves the bin's total.
//   3. bases:   one workgroup scans the bins' totals: where each bin starts in `order`
//               (the offsets; the totals are the sizes).
//   4. scatter: each wave walks its segment 64 picks at a time, in order, from its
//               bins' starts (base + row prefix). A pick's rank among the same bin's
//               picks of those 64 comes from ballots over its bin's bits (the lanes that
//               agree on every bit), and the lowest lane of each bin moves the bin's
//               running position on by the count: a stable order.
// All integer work: bit-exact by construction.

#include "common.h"

namespace bux {
namespace {

constexpr int SEGMENT = 256;  // picks a wave takes
constexpr int WAVES = 4;      // waves a workgroup
constexpr int MAX_BINS = 8192;  // experts + 1 (the LDS of count and scatter limits them further)

__device__ __forceinline__ int bin_of(int32_t expert, int32_t num_experts) {
  return (expert >= 0 && expert < num_experts) ? expert : num_experts;
}

__global__ __launch_bounds__(64 * WAVES) void count_kernel(const int32_t* __restrict__ idx,
                                                           int64_t n, int32_t num_experts,
                                                           int64_t segments,
                                                           int32_t* __restrict__ counts) {
  extern __shared__ int32_t lds[];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int bins = num_experts + 1;
  int32_t* mine = lds + wave * bins;
  for (int b = lane; b < bins; b += 64) mine[b] = 0;
  __syncthreads();
  const int64_t seg = static_cast<int64_t>(blockIdx.x) * WAVES + wave;
  if (seg < segments) {
    for (int i = lane; i < SEGMENT; i += 64) {
      const int64_t p = seg * SEGMENT + i;
      if (p < n) atomicAdd(&mine[bin_of(idx[p], num_experts)], 1);
    }
  }
  __syncthreads();
  if (seg < segments) {
    for (int b = lane; b < bins; b += 64) counts[static_cast<int64_t>(b) * segments + seg] = mine[b];
  }
}

constexpr int SCAN_THREADS = 256;

// Exclusive scan of one value a thread over the workgroup (SCAN_THREADS lanes), by
// wave prefix sums and one pass over the waves' totals; returns the workgroup's total.
__device__ __forceinline__ int32_t block_exclusive(int32_t v, int32_t& prefix, int32_t* wave_sums) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int32_t x = v;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int32_t y = __shfl_up(x, d);
    if (lane >= d) x += y;
  }
  if (lane == 63) wave_sums[wave] = x;
  __syncthreads();
  int32_t before = 0, total = 0;
#pragma unroll
  for (int w = 0; w < SCAN_THREADS / 64; ++w) {
    const int32_t t = wave_sums[w];
    if (w < wave) before += t;
    total += t;
  }
  __syncthreads();
  prefix = before + x - v;
  return total;
}

// Workgroup b scans counts[b][0 .. segments) exclusively in place; totals[b] = the sum.
__global__ __launch_bounds__(SCAN_THREADS) void rows_kernel(int32_t* __restrict__ counts,
                                                            int64_t segments,
                                                            int32_t* __restrict__ totals) {
  __shared__ int32_t wave_sums[SCAN_THREADS / 64];
  int32_t* row = counts + static_cast<int64_t>(blockIdx.x) * segments;
  int32_t carry = 0;
  for (int64_t base = 0; base < segments; base += SCAN_THREADS) {
    const int64_t i = base + threadIdx.x;
    const int32_t v = i < segments ? row[i] : 0;
    int32_t prefix;
    const int32_t total = block_exclusive(v, prefix, wave_sums);
    if (i < segments) row[i] = carry + prefix;
    carry += total;
  }
  if (threadIdx.x == 0) totals[blockIdx.x] = carry;
}

// One workgroup: bases[b] = the totals of the bins before b; sizes and offsets of the
// experts (offsets[E] = the picks of experts: `filled`).
__global__ __launch_bounds__(SCAN_THREADS) void bases_kernel(const int32_t* __restrict__ totals,
                                                             int32_t bins,
                                                             int32_t* __restrict__ bases,
                                                             int32_t* __restrict__ sizes,
                                                             int32_t* __restrict__ offsets) {
  __shared__ int32_t wave_sums[SCAN_THREADS / 64];
  int32_t carry = 0;
  for (int32_t base = 0; base < bins; base += SCAN_THREADS) {
    const int32_t b = base + threadIdx.x;
    const int32_t v = b < bins ? totals[b] : 0;
    int32_t prefix;
    const int32_t total = block_exclusive(v, prefix, wave_sums);
    if (b < bins) {
      bases[b] = carry + prefix;
      if (b < bins - 1) {
        sizes[b] = v;
        offsets[b] = carry + prefix;
      } else {
        offsets[b] = carry + prefix;  // past the last expert: the sum of their sizes
      }
    }
    carry += total;
  }
}

__global__ __launch_bounds__(64 * WAVES) void scatter_kernel(
    const int32_t* __restrict__ idx, int64_t n, int32_t num_experts, int32_t bits,
    int64_t segments, const int32_t* __restrict__ base, const int32_t* __restrict__ bases,
    int32_t* __restrict__ order, int32_t* __restrict__ inverse) {
  extern __shared__ int32_t lds[];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int bins = num_experts + 1;
  int32_t* running = lds + wave * bins;
  const int64_t seg = static_cast<int64_t>(blockIdx.x) * WAVES + wave;
  if (seg >= segments) return;  // whole waves leave; no workgroup barrier follows
  for (int b = lane; b < bins; b += 64)
    running[b] = bases[b] + base[static_cast<int64_t>(b) * segments + seg];
  __builtin_amdgcn_wave_barrier();
  const uint64_t below = (1ull << lane) - 1ull;
  for (int i = 0; i < SEGMENT; i += 64) {
    const int64_t p = seg * SEGMENT + i + lane;
    const bool valid = p < n;
    const int b = valid ? bin_of(idx[p], num_experts) : 0;
    uint64_t peers = __ballot(valid);
    for (int bit = 0; bit < bits; ++bit) {
      const bool set = (b >> bit) & 1;
      const uint64_t m = __ballot(set);
      peers &= set ? m : ~m;
    }
    const int rank = __popcll(peers & below);
    const int32_t start = valid ? running[b] : 0;
    __builtin_amdgcn_wave_barrier();
    if (valid) {
      const int32_t pos = start + rank;
      order[pos] = static_cast<int32_t>(p);
      inverse[p] = pos;
      if (rank == 0) running[b] = start + __popcll(peers);
    }
    __builtin_amdgcn_wave_barrier();
  }
}

}  // namespace
}  // namespace bux

extern "C" size_t bux_moe_permute_workspace_size(int64_t n_picks, int32_t num_experts) {
  // counts[bins][segments], then the bins' totals and bases
  const int64_t segments = (n_picks + bux::SEGMENT - 1) / bux::SEGMENT;
  return static_cast<size_t>(segments + 2) * static_cast<size_t>(num_experts + 1) * sizeof(int32_t);
}

extern "C" int bux_moe_permute(const int32_t* idx, int64_t n_picks, int32_t num_experts,
                               int32_t* order, int32_t* inverse, int32_t* sizes, int32_t* offsets,
                               void* workspace, size_t workspace_bytes, void* stream) {
  using namespace bux;
  clear_error();
  BUX_CHECK(n_picks >= 0 && n_picks <= 2147483647LL,
            "bux_moe_permute: n_picks=%lld outside [0, 2^31)", (long long)n_picks);
  BUX_CHECK(num_experts >= 1 && num_experts < MAX_BINS,
            "bux_moe_permute: num_experts=%d outside [1, %d)", num_experts, MAX_BINS);
  BUX_CHECK(sizes && offsets, "bux_moe_permute: sizes and offsets are needed");
  BUX_CHECK(n_picks == 0 || (idx && order && inverse),
            "bux_moe_permute: idx, order and inverse are needed");
  const size_t need = bux_moe_permute_workspace_size(n_picks, num_experts);
  if (workspace_bytes < need || workspace == nullptr)
    return fail(BUX_E_WORKSPACE, "bux_moe_permute: workspace of %zu bytes, %zu needed",
                workspace_bytes, need);
  const int64_t segments = ceil_div(n_picks, SEGMENT);
  const int bins = num_experts + 1;
  int bits = 0;
  while ((1 << bits) < bins) ++bits;
  int32_t* counts = static_cast<int32_t*>(workspace);
  const size_t lds = static_cast<size_t>(WAVES) * bins * sizeof(int32_t);
  BUX_CHECK(lds <= 64 * 1024, "bux_moe_permute: %d experts exceed the LDS a workgroup takes",
            num_experts);
  hipStream_t s = as_stream(stream);
  const unsigned blocks = static_cast<unsigned>(ceil_div(segments, WAVES));
  if (segments > 0) {
    hipLaunchKernelGGL(count_kernel, dim3(blocks), dim3(64 * WAVES), lds, s, idx, n_picks,
                       num_experts, segments, counts);
    if (int rc = launched("count_kernel")) return rc;
  }
  int32_t* totals = counts + segments * bins;
  int32_t* bases = totals + bins;
  hipLaunchKernelGGL(rows_kernel, dim3(bins), dim3(SCAN_THREADS), 0, s, counts, segments, totals);
  if (int rc = launched("rows_kernel")) return rc;
  hipLaunchKernelGGL(bases_kernel, dim3(1), dim3(SCAN_THREADS), 0, s, totals, bins, bases, sizes,
                     offsets);
  if (int rc = launched("bases_kernel")) return rc;
  if (segments > 0) {
    hipLaunchKernelGGL(scatter_kernel, dim3(blocks), dim3(64 * WAVES), lds, s, idx, n_picks,
                       num_experts, bits, segments, counts, bases, order, inverse);
    if (int rc = launched("scatter_kernel")) return rc;
  }
  return BUX_OK;
}
