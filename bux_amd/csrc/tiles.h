// The grouped GEMMs' shared schedule, whatever their operands' format:
//
// - the ragged tile list, built on the device from the groups' sizes by a one-workgroup
//   prologue (the reference's tiles_of, grouped_mxfp8.py:157-182), so the host never
//   synchronises; a list opens with a header that names the dimensions it was made for;
// - the persistent grid: one workgroup a CU, each XCD (workgroup id % 8) taking a
//   contiguous run of tiles, which share A's rows and a group's B in its L2;
// - run_tiles, the pipeline over a workgroup's tiles: a ring of STAGES LDS stages filled
//   by direct loads STAGES steps ahead of their MFMAs, across tiles.
//
// A format supplies the operand type, the stage layout, the loads, the fragment reads
// and the MFMA step as the static members of a policy struct P (the MXFP8 GEMMs' Mx and
// the bfloat16 GEMMs' Bf16); the output, a functor with store(acc, job, stage).
#pragma once

#include <type_traits>

#include "common.h"

namespace bux {
namespace {

constexpr int BM = 256;  // rows of a tile (A's)
constexpr int BN = 256;  // columns of a tile (B's rows)
constexpr int STAGES = 4;
constexpr int THREADS = 256;
constexpr int MAX_GROUPS = 4096;

typedef float v16f __attribute__((ext_vector_type(16)));

struct Tile {
  int32_t group, lo, hi;
};

// --- the device-side prologue: group starts and the ragged tile list ----------------

// Exclusive scan of data[0, n) (each >= 0) in LDS by one workgroup of THREADS lanes,
// in 64 bits, each prefix sum capped at `cap`; returns the capped total. `partial` is
// THREADS int64s of LDS.
__device__ int32_t block_scan(int32_t* data, int n, int64_t* partial, int32_t cap) {
  const int t = threadIdx.x;
  const int per = (n + THREADS - 1) / THREADS;
  const int lo = t * per, hi = lo + per < n ? lo + per : n;
  int64_t sum = 0;
  for (int i = lo; i < hi; ++i) sum += data[i];
  partial[t] = sum;
  __syncthreads();
  for (int step = 1; step < THREADS; step <<= 1) {
    const int64_t add = t >= step ? partial[t - step] : 0;
    __syncthreads();
    partial[t] += add;
    __syncthreads();
  }
  int64_t run = t > 0 ? partial[t - 1] : 0;
  for (int i = lo; i < hi; ++i) {
    const int32_t c = data[i];
    data[i] = static_cast<int32_t>(run < cap ? run : cap);
    run += c;
  }
  const int64_t total = partial[THREADS - 1];
  __syncthreads();
  return static_cast<int32_t>(total < cap ? total : cap);
}

// A tile list opens with a header of LIST_HEADER bytes: LIST_MAGIC, the groups, m and
// height it was made for, and a status word (LIST_REFUSED once a listed GEMM was called
// with other dimensions); its group starts follow.
constexpr int LIST_HEADER = 64;
constexpr int32_t LIST_MAGIC = BUX_LIST_MAGIC;  // "BUXT"
constexpr int32_t LIST_REFUSED = BUX_LIST_REFUSED;

// starts[g] for g <= groups (starts[groups] = sum of sizes; a negative size counts as
// 0, and the sums stop at max(m, height) where that is positive), then, if `tiles`, the
// tile list of `slots` entries: each group's rows in tiles of BM from its first row
// rounded down to a multiple of `align` (a power of two; the last tile partial), then
// the rows from the sum of sizes to `height` as group `groups`, then empty tiles
// (0, 0, 0); and the number of tiles listed in starts[groups + 1]. A tile (g, lo, hi)
// computes rows [lo, lo + BM) and holds rows [max(lo, starts[g]), hi) of group g.
//
// With `header` (a tile list's, LIST_HEADER bytes before its starts), the list's
// dimensions go there too: LIST_MAGIC, groups, m, height, and a 0 status word. With
// `a_starts`, the tiles lie where the groups' rows lie in a (a_starts[g] on), not packed
// (starts_out stays packed: where their rows lie in y).
__global__ __launch_bounds__(THREADS) void prologue_kernel(const int32_t* __restrict__ sizes,
                                                           int32_t groups, int64_t height,
                                                           int64_t slots, int32_t align,
                                                           int32_t* __restrict__ starts_out,
                                                           Tile* __restrict__ tiles,
                                                           int32_t* __restrict__ header,
                                                           int64_t m,
                                                           const int32_t* __restrict__ a_starts) {
  if (header != nullptr && threadIdx.x < LIST_HEADER / 4) {
    const int32_t i = threadIdx.x;
    header[i] = i == 0 ? LIST_MAGIC : i == 1 ? groups : i == 2 ? static_cast<int32_t>(m)
              : i == 3 ? static_cast<int32_t>(height) : 0;
  }
  __shared__ int32_t starts[MAX_GROUPS + 2];
  __shared__ int32_t before[MAX_GROUPS + 2];
  __shared__ int64_t partial[THREADS];
  const int t = threadIdx.x;
  // The sizes as the tiles take them: a negative one as 0, and the starts capped at the
  // rows there are (m or height, whichever is more: the rows GEMM's rows, the contract's
  // K; unbounded where neither is given), so that sizes past them give the last groups
  // fewer rows, the same in the rows GEMM and the contract, never a tile outside the
  // rows or a count that overflows.
  const int64_t rows = m > height ? m : height;
  const int32_t cap = rows > 0 && rows < INT32_MAX ? static_cast<int32_t>(rows) : INT32_MAX;
  for (int g = t; g < groups; g += THREADS) starts[g] = sizes[g] > 0 ? sizes[g] : 0;
  __syncthreads();
  const int32_t filled = block_scan(starts, groups, partial, cap);
  if (t == 0) starts[groups] = filled;
  __syncthreads();
  for (int g = t; g <= groups; g += THREADS) starts_out[g] = starts[g];
  if (tiles == nullptr) return;
  const int all = groups + 1;
  auto size_of = [&](int g) -> int64_t {
    if (g < groups) return starts[g + 1] - starts[g];
    return height > filled ? height - filled : 0;
  };
  // where group g's rows lie in a: `a_starts` (given), else packed; the rows past the
  // groups where they lie in y
  auto first = [&](int g) -> int64_t {
    return a_starts != nullptr && g < groups ? static_cast<int64_t>(a_starts[g]) : starts[g];
  };
  // tiles of group g: from its first row rounded down to `align`
  auto count_of = [&](int g) -> int64_t {
    const int64_t s = size_of(g);
    if (s <= 0) return 0;
    const int64_t start = first(g), base = start & ~static_cast<int64_t>(align - 1);
    return (start + s - base + BM - 1) / BM;
  };
  for (int g = t; g < all; g += THREADS) before[g] = static_cast<int32_t>(count_of(g));
  __syncthreads();
  const int32_t used = block_scan(before, all, partial, INT32_MAX);
  for (int g = t; g < all; g += THREADS) {
    const int64_t s = size_of(g), start = first(g), end = start + s;
    const int64_t base = start & ~static_cast<int64_t>(align - 1), count = count_of(g);
    // The capped starts keep the counts within the slots; a tile past them would be
    // dropped, never written past the list.
    for (int64_t j = 0; j < count && before[g] + j < slots; ++j) {
      const int64_t lo = base + j * BM;
      tiles[before[g] + j] = Tile{g, static_cast<int32_t>(lo),
                                  static_cast<int32_t>(end < lo + BM ? end : lo + BM)};
    }
  }
  for (int64_t i = used + t; i < slots; i += THREADS) tiles[i] = Tile{0, 0, 0};
  if (t == 0) starts_out[groups + 1] = used < slots ? used : static_cast<int32_t>(slots);
}

// Whether the list whose starts are `starts` (its header LIST_HEADER bytes before them)
// was made for these groups (and, m >= 0, this m and height); if not, workgroup 0 sets
// its status word to LIST_REFUSED and the caller computes nothing from it.
__device__ __forceinline__ bool list_fits(const int32_t* starts, int32_t groups, int32_t m,
                                          int32_t height) {
  const int32_t* header = starts - LIST_HEADER / 4;
  const bool fits = header[0] == LIST_MAGIC && header[1] == groups &&
                    (m < 0 || (header[2] == m && header[3] == height));
  if (!fits && blockIdx.x == 0 && threadIdx.x == 0)
    const_cast<int32_t*>(header)[4] = LIST_REFUSED;
  return fits;
}

// --- the persistent tile loop ----------------------------------------------------------

// The tiles a workgroup of a persistent grid takes, of `count`: XCD x (workgroup id % 8)
// takes the contiguous tiles [x per, (x + 1) per), its workgroups one after another, so
// that the XCD's CUs work on neighbouring tiles at any time (they share A's rows and a
// group's B in the XCD's L2).
struct Turns {
  int32_t first, end, stride;
};
__device__ __forceinline__ Turns turns(int32_t count) {
  const int32_t per = (count + 7) / 8, xcd = blockIdx.x % 8;
  const int32_t lo = xcd * per, hi = lo + per < count ? lo + per : count;
  return Turns{lo + static_cast<int32_t>(blockIdx.x / 8), hi, static_cast<int32_t>(gridDim.x / 8)};
}

__device__ __forceinline__ int32_t smaller(int32_t a, int32_t b) { return a < b ? a : b; }

// One output tile's work: C[r][c] = sum over K steps [ks_begin, ks_begin + n) of
// A[a_row0 + r] . B[b_row0 + c] (B of `group`), the K positions outside [mlo, mhi)
// counting 0 where `mask` (in the first and last steps); its rows [0, rows) and columns
// [0, cols) stored at `corner`. A `half` tile holds at most BM / 2 rows: only its first
// BM / 2 rows of A are loaded and computed (a format that has half tiles, P::HALVES).
struct Job {
  int32_t a_row0, b_row0, group;
  int32_t ks_begin, n;
  int32_t mlo, mhi;
  bool mask, half;
  int64_t corner;
  int32_t rows, cols;
  int32_t row_lo;  // the first of the tile's rows it stores (the fused epilogue's)
};

// The rows GEMM's tiles: the tile list's row tiles by 256-column tiles of y. K is k_end
// positions in k_steps steps; with TAIL the last step reaches past k_end and is masked
// there. With HALVES a tile of at most BM / 2 rows (a group's last, or a small group's
// only one) is a half tile.
template <bool TAIL = false, bool HALVES_ = false>
struct RowsTiles {
  static constexpr bool HALVES = HALVES_;
  const Tile* tiles;
  int32_t groups, n, height, col_tiles, k_steps, k_end;
  __device__ bool job(int32_t id, Job& j) const {
    const Tile t = tiles[id / col_tiles];
    const int32_t col0 = (id % col_tiles) * BN;
    // Rows of y stop at height whatever the sizes say.
    j.rows = smaller(t.hi, height) - t.lo;
    if (j.rows <= 0) return false;
    j.cols = smaller(n - col0, BN);
    j.a_row0 = t.lo;
    j.b_row0 = col0;
    j.group = t.group < groups ? t.group : 0;
    j.ks_begin = 0;
    j.n = t.group < groups ? k_steps : 0;  // rows past the groups: zeros
    j.mask = TAIL;
    j.half = HALVES && j.rows <= BM / 2;
    j.mlo = 0;
    j.mhi = k_end;
    j.corner = static_cast<int64_t>(t.lo) * n + col0;
    return true;
  }
};

// The rows GEMM's tiles where each group's rows lie in a from a_starts[g] (tiles from
// the prologue given those starts) while y's rows stay packed (starts, the prologue's):
// a tile's rows of a map to y's by the group's shift, packed start less a's. HALVES as
// RowsTiles's.
template <bool HALVES_ = false>
struct StartedTiles {
  static constexpr bool HALVES = HALVES_;
  const Tile* tiles;
  const int32_t* starts;    // packed: where each group's rows lie in y
  const int32_t* a_starts;  // where they lie in a
  int32_t groups, n, height, col_tiles, k_steps;
  __device__ bool job(int32_t id, Job& j) const {
    const Tile t = tiles[id / col_tiles];
    const int32_t col0 = (id % col_tiles) * BN;
    const int32_t shift = t.group < groups ? starts[t.group] - a_starts[t.group] : 0;
    const int32_t lo = t.lo + shift;  // the tile's first row of y
    j.rows = smaller(t.hi + shift, height) - lo;
    if (j.rows <= 0) return false;
    j.cols = smaller(n - col0, BN);
    j.a_row0 = t.lo;
    j.b_row0 = col0;
    j.group = t.group < groups ? t.group : 0;
    j.ks_begin = 0;
    j.n = t.group < groups ? k_steps : 0;  // rows past the groups: zeros
    j.mask = false;
    j.half = HALVES && j.rows <= BM / 2;
    j.mlo = j.mhi = 0;
    j.corner = static_cast<int64_t>(lo) * n + col0;
    return true;
  }
};

// The contract GEMM's tiles: each group's d x f output in 256 x 256 tiles; K is the
// rows of the operands, `step` of them a K step, and a group's sum takes its own rows
// [starts[g], starts[g + 1]) only.
struct ContractTiles {
  static constexpr bool HALVES = false;
  const int32_t* starts;
  int32_t d, f, d_tiles, f_tiles, step;
  __device__ bool job(int32_t id, Job& j) const {
    const int32_t per_group = d_tiles * f_tiles;
    const int32_t g = id / per_group, rest = id % per_group;
    const int32_t row0 = (rest / f_tiles) * BM, col0 = (rest % f_tiles) * BN;
    const int32_t start = starts[g], end = starts[g + 1];
    j.a_row0 = row0;
    j.b_row0 = col0;
    j.group = 0;
    j.ks_begin = start / step;
    j.n = end > start ? (end + step - 1) / step - j.ks_begin : 0;
    j.mask = (start % step) != 0 || (end % step) != 0;
    j.half = false;
    j.mlo = start;
    j.mhi = end;
    j.corner = (static_cast<int64_t>(g) * d + row0) * f + col0;
    j.rows = smaller(d - row0, BM);
    j.cols = smaller(f - col0, BN);
    return true;
  }
};

template <typename Tiles>
__device__ __forceinline__ bool next_job(const Tiles& tiles, const Turns& mine, int32_t& id, Job& j) {
  for (; id < mine.end; id += mine.stride) {
    if (tiles.job(id, j)) {
      id += mine.stride;
      return true;
    }
  }
  return false;
}

__device__ __forceinline__ void zero_acc(v16f acc[4][4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int q = 0; q < 16; ++q) acc[i][j][q] = 0.0f;
}

// The workgroup barrier of the pipeline: this wave's LDS reads and writes are done,
// then s_barrier. Unlike __syncthreads it does not wait for vector memory in flight
// (a fence would: vmcnt(0)).
__device__ __forceinline__ void barrier_lds() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// A workgroup's tiles, one after another through one ring of STAGES (4) stages. The K
// steps of all its tiles form one stream: step g sits in stage g % 4, and the loads of
// step g + 4 go out during step g, also across tiles, so that a tile's first steps land
// while the tile before it finishes. The one exception: the last step of a tile leaves
// its stage to the epilogue, which stages the outputs there; the next tile's step 3 is
// issued after it.
//
// A wave keeps two sets of operand registers: while the MFMAs of step k run on one, its
// LDS reads of step k + 1 fill the other. The workgroup's one barrier a step comes first
// (after it step k + 1's stage is whole and every wave has read step k's), then the
// step's MFMAs, each followed by a slice of the memory work (P::step).
//
// Stores and loads share a wave's vmcnt, and a wait counts only the loads issued after
// the step it waits for: a store still in flight makes it wait longer, never too little.
// The epilogue's stores go out while the next tile's first steps are still loading
// (waiting for those loads first, as an earlier version did, measured 2% slower over
// the six GEMMs at config 3, with the same outputs).
//
// Half tiles (P::HALVES, and a tile list with them, Tiles::HALVES): the same stream and the same number of loads a step and wave
// (P::issue stands in cheap ones for the A loads a half tile skips), so every wait
// counts as for a whole tile; their steps run P::step's half form.
template <typename P, typename Out, typename Tiles>
__device__ __forceinline__ void run_tiles(const Tiles& tiles, int32_t count,
                                          const typename P::Operand& A,
                                          const typename P::Operand& B, typename P::Lds& lds,
                                          const Out& out) {
  using Loads = typename P::Loads;
  using Frag = typename P::Frag;
  const Turns mine = turns(count);
  int32_t id = mine.first;
  Job job{}, next{};
  if (!next_job(tiles, mine, id, job)) return;
  const uint32_t lds0 = lds_at(&lds);
  int32_t base = 0;  // the stage of this tile's step 0
  {
    const Loads la = P::loads_a(A, job.a_row0), lb = P::loads_b(B, job.group, job.b_row0);
    for (int32_t s = 0; s < STAGES && s < job.n; ++s)
      P::issue(la, lb, job.ks_begin + s, lds0, s, Tiles::HALVES && job.half);
  }
  for (;;) {
    const bool more = next_job(tiles, mine, id, next);
    const int32_t n = job.n, nn = more ? next.n : 0;
    auto stage = [&](int32_t k) { return (base + k) & (STAGES - 1); };
    const Loads la = P::loads_a(A, job.a_row0), lb = P::loads_b(B, job.group, job.b_row0);
    const Loads na = P::loads_a(A, next.a_row0), nb = P::loads_b(B, next.group, next.b_row0);
    // The next tile's steps issued so far; those whose stages this tile does not use go
    // now.
    int32_t ahead = 0;
    for (; ahead < 3 && ahead < nn && n + ahead < STAGES; ++ahead)
      P::issue(na, nb, next.ks_begin + ahead, lds0, stage(n + ahead), Tiles::HALVES && next.half);
    v16f acc[4][4];
    zero_acc(acc);
    // The K loop of a whole (H false) or a half tile.
    auto loop = [&](auto half) {
      constexpr bool H = decltype(half)::value;
      const typename P::Lanes ln = P::template lanes_of<H>();
      auto edge = [&](int32_t k) { return job.mask && (k == 0 || k == n - 1); };
      P::wait_loads(smaller(n, STAGES) - 1 + ahead);
      barrier_lds();
      Frag cur, nxt;
      P::template read_frag<H>(cur, lds, ln, stage(0), job.ks_begin);
      if (edge(0)) P::mask_frag(cur, job.ks_begin, job.mlo, job.mhi);
      int32_t k = 0;
      // Steps with this tile's load 4 ahead, two a turn so that the operand sets swap
      // roles without a copy; step k + 1 < n - 1 is never an edge here.
      for (; k + 5 < n; k += 2) {
        P::wait_loads(2);
        // Step k + 1's stage is whole; every wave has read step k's, which step k + 4's
        // loads take.
        barrier_lds();
        P::template step<true, true, H>(cur, nxt, la, lb, lds, lds0, ln, job.ks_begin + k + 4,
                                        stage(k), job.ks_begin + k + 1, stage(k + 1), acc);
        P::wait_loads(2);
        barrier_lds();
        P::template step<true, true, H>(nxt, cur, la, lb, lds, lds0, ln, job.ks_begin + k + 5,
                                        stage(k + 1), job.ks_begin + k + 2, stage(k + 2), acc);
      }
      for (; k + 4 < n; ++k) {
        P::wait_loads(2);
        barrier_lds();
        P::template step<true, true, H>(cur, nxt, la, lb, lds, lds0, ln, job.ks_begin + k + 4,
                                        stage(k), job.ks_begin + k + 1, stage(k + 1), acc);
        cur = nxt;
      }
      // The last steps: the freed stages take the next tile's first steps.
      for (; k + 1 < n; ++k) {
        P::wait_loads(smaller(n - 2 - k + ahead, 3));
        barrier_lds();
        if (ahead < 3 && ahead < nn && k + STAGES == n + ahead) {
          P::issue(na, nb, next.ks_begin + ahead, lds0, stage(k), Tiles::HALVES && next.half);
          ++ahead;
        }
        P::template step<false, true, H>(cur, nxt, la, lb, lds, lds0, ln, 0, 0,
                                         job.ks_begin + k + 1, stage(k + 1), acc);
        cur = nxt;
      }
      // the last step's operands (read during the step before): its edge, if it has one
      if (n > 1 && edge(n - 1)) P::mask_frag(cur, job.ks_begin + n - 1, job.mlo, job.mhi);
      P::template step<false, false, H>(cur, nxt, la, lb, lds, lds0, ln, 0, 0, 0, 0, acc);
    };
    if (n > 0) {
      if constexpr (P::HALVES && Tiles::HALVES) {
        if (job.half) loop(std::true_type{});
        else loop(std::false_type{});
      } else {
        loop(std::false_type{});
      }
    }
    // Every wave is done with this tile's stages; its last step's (stage n + 3) stages the
    // outputs.
    barrier_lds();
    out.store(acc, job, lds.st[stage(n + 3)]);
    barrier_lds();
    if (!more) break;
    if (nn > 3) P::issue(na, nb, next.ks_begin + 3, lds0, stage(n + 3), Tiles::HALVES && next.half);
    base = stage(n);
    job = next;
  }
}

// --- host side -------------------------------------------------------------------------

// Lets a kernel take `bytes` (over 64 KiB) of dynamic LDS; gfx950 has 160 KiB a CU.
template <typename K>
int allow_lds(K kernel, size_t bytes, const char* name) {
  hipError_t err = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                       hipFuncAttributeMaxDynamicSharedMemorySize,
                                       static_cast<int>(bytes));
  if (err != hipSuccess) return fail(BUX_E_LAUNCH, "%s: %s", name, hipGetErrorString(err));
  return BUX_OK;
}

int64_t row_slots(int32_t groups, int64_t m, int64_t height) {
  const int64_t rows = m > height ? m : height;
  // tiles of rows, plus one a group (and one for the rows past them) at most
  return ceil_div(rows, BM) + groups + 1;
}

// The persistent grid: one workgroup a CU of the current device (a multiple of 8, one
// share a XCD), or fewer for fewer tiles.
int grid_for(int64_t tiles, unsigned* blocks) {
  int device = 0, cus = 0;
  hipError_t err = hipGetDevice(&device);
  if (err == hipSuccess) err = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device);
  if (err != hipSuccess) return fail(BUX_E_DEVICE, "the device's compute units: %s", hipGetErrorString(err));
  const int64_t most = cus >= 8 ? cus / 8 * 8 : 8;
  const int64_t want = 8 * ceil_div(tiles > 0 ? tiles : 1, 8);
  *blocks = static_cast<unsigned>(want < most ? want : most);
  return BUX_OK;
}

size_t align256(size_t v) { return (v + 255) & ~static_cast<size_t>(255); }

// A tile list's buffer: the header (LIST_HEADER bytes), the group starts (groups + 2
// ints; header and starts 256-byte aligned together), then the tile records.
int32_t* header_in(const void* list) { return static_cast<int32_t*>(const_cast<void*>(list)); }
int32_t* starts_in(const void* list) {
  return reinterpret_cast<int32_t*>(static_cast<uint8_t*>(const_cast<void*>(list)) + LIST_HEADER);
}
size_t starts_bytes(int32_t groups) {
  return align256(LIST_HEADER + static_cast<size_t>(groups + 2) * sizeof(int32_t));
}
Tile* tiles_in(const void* list, int32_t groups) {
  return reinterpret_cast<Tile*>(static_cast<uint8_t*>(const_cast<void*>(list)) +
                                 starts_bytes(groups));
}

}  // namespace
}  // namespace bux
