// Sorting an MoE's picks by expert, stably: order, its inverse, each expert's size
// and the groups' offsets (src/bux/architecture/experts/moe.py:776-797: a stable
// argsort of the flat picks with those outside [0, E) as E, bincount, argsort of the
// order; the offsets cumsum(sizes) - sizes of grouped_mxfp8.py:142).
//
// A counting sort in three launches over segments of 256 picks (one wave a segment):
//   1. count:   each wave counts its segment's picks per bin (E bins and one for the
//               picks outside) in LDS; counts[bin][segment] goes to the workspace.
//   2. scan:    one workgroup scans counts bin-major, exclusively: entry (b, s) becomes
//               where bin b's picks of segment s start in `order`. The scan's values at
//               each bin's first segment are the offsets; their differences the sizes.
//   3. scatter: each wave walks its segment 64 picks at a time, in order. A pick's rank
//               among the same bin's picks of those 64 comes from ballots over its bin's
//               bits (the lanes that agree on every bit), and the lowest lane of each
//               bin moves the bin's running position on by the count: a stable order.
// All integer work: bit-exact by construction.

#include "common.h"

namespace bux {
namespace {

constexpr int SEGMENT = 256;  // picks a wave takes
constexpr int WAVES = 4;      // waves a workgroup
constexpr int MAX_BINS = 8192;  // experts + 1 the scan's LDS holds offsets for

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

constexpr int SCAN_THREADS = 1024;

__global__ __launch_bounds__(SCAN_THREADS) void scan_kernel(int32_t* __restrict__ counts,
                                                            int64_t segments, int32_t num_experts,
                                                            int64_t n, int32_t* __restrict__ sizes,
                                                            int32_t* __restrict__ offsets) {
  __shared__ int32_t partial[SCAN_THREADS];
  __shared__ int32_t starts[MAX_BINS + 1];
  const int t = threadIdx.x;
  const int bins = num_experts + 1;
  const int64_t total = static_cast<int64_t>(bins) * segments;
  const int64_t per = (total + SCAN_THREADS - 1) / SCAN_THREADS;
  const int64_t lo = t * per, hi = lo + per < total ? lo + per : total;
  int32_t sum = 0;
  for (int64_t i = lo; i < hi; ++i) sum += counts[i];
  partial[t] = sum;
  __syncthreads();
  // Inclusive Hillis-Steele scan of the 1024 partial sums.
  for (int step = 1; step < SCAN_THREADS; step <<= 1) {
    const int32_t add = t >= step ? partial[t - step] : 0;
    __syncthreads();
    partial[t] += add;
    __syncthreads();
  }
  int32_t run = t > 0 ? partial[t - 1] : 0;
  for (int64_t i = lo; i < hi; ++i) {
    const int32_t c = counts[i];
    counts[i] = run;
    if (i % segments == 0) starts[i / segments] = run;
    run += c;
  }
  if (segments == 0) {
    for (int b = t; b < bins; b += SCAN_THREADS) starts[b] = 0;
  }
  if (t == 0) starts[bins] = static_cast<int32_t>(n);
  __syncthreads();
  for (int b = t; b < num_experts; b += SCAN_THREADS) {
    sizes[b] = starts[b + 1] - starts[b];
    offsets[b] = starts[b];
  }
  if (t == 0) offsets[num_experts] = starts[num_experts];  // the picks of experts: filled
}

__global__ __launch_bounds__(64 * WAVES) void scatter_kernel(
    const int32_t* __restrict__ idx, int64_t n, int32_t num_experts, int32_t bits,
    int64_t segments, const int32_t* __restrict__ base, int32_t* __restrict__ order,
    int32_t* __restrict__ inverse) {
  extern __shared__ int32_t lds[];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int bins = num_experts + 1;
  int32_t* running = lds + wave * bins;
  const int64_t seg = static_cast<int64_t>(blockIdx.x) * WAVES + wave;
  if (seg >= segments) return;  // whole waves leave; no workgroup barrier follows
  for (int b = lane; b < bins; b += 64) running[b] = base[static_cast<int64_t>(b) * segments + seg];
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
  const int64_t segments = (n_picks + bux::SEGMENT - 1) / bux::SEGMENT;
  return static_cast<size_t>(segments) * static_cast<size_t>(num_experts + 1) * sizeof(int32_t);
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
  if (workspace_bytes < need || (need > 0 && workspace == nullptr))
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
  hipLaunchKernelGGL(scan_kernel, dim3(1), dim3(SCAN_THREADS), 0, s, counts, segments,
                     num_experts, n_picks, sizes, offsets);
  if (int rc = launched("scan_kernel")) return rc;
  if (segments > 0) {
    hipLaunchKernelGGL(scatter_kernel, dim3(blocks), dim3(64 * WAVES), lds, s, idx, n_picks,
                       num_experts, bits, segments, counts, order, inverse);
    if (int rc = launched("scatter_kernel")) return rc;
  }
  return BUX_OK;
}
