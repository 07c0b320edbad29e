// The MoE router: each token's logits over the experts, their scores, the top-k picks
// and the picks' weights, in one kernel (after a transpose of the router's kernel).
//
//   logits  (x @ kernel + bias) * logit_scale         moe.py:249, 275-284
//           bfloat16 operands, float32 sums (MFMA v_mfma_f32_32x32x16_bf16)
//   scores  softmax over every logit | sigmoid | sqrt(softplus), float32   moe.py:251-257
//   choice  scores[:scored] + choice_bias, at -inf outside the `keep` best of `groups`
//           groups (a group's score: the sum of its best two)   moe.py:258-261, 474-483
//   picks   the k largest choices, the largest first, ties to the lower index
//           (jax.lax.top_k)                            moe.py:262
//   weights the picked scores, divided by their sum plus the sinks' (scores past
//           `scored`) if normalize; both to bfloat16, then times the bfloat16-rounded
//           scaling factor in bfloat16                  moe.py:265-270
//
// A workgroup takes 32 tokens. Its 4 waves split the logits' 32-column blocks (wave w
// the blocks w, w + 4, ...) and run the K loop on registers: each lane loads 16 bytes of
// its token's row and of its expert's row of the transposed kernel a step, both
// straight from global memory (the kernel, 2 d bytes an expert, stays in L2). The
// logits go to LDS, a row a token (its pitch one float past a multiple of 32, so that
// 32 lanes reading 32 rows at one column hit 32 banks); then a lane a token computes
// the scores in place, the group limit, the top-k and the weights, and the workgroup
// writes the rows of scores and logits asked for. HBM-bound: x is read once.

#include <math.h>

#include "common.h"

namespace bux {
namespace {

constexpr int THREADS = 256;   // 4 waves
constexpr int MAX_LOGITS = 1024;
constexpr int MAX_PICKS = 16;  // k, and the groups kept
constexpr int MAX_GROUPS = 64;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));

// kernel (d, n) row-major -> kt (npad, d): kt[e][j] = kernel[j][e], rows n.. npad 0.
// A 32 x 32 tile through LDS a workgroup.
__global__ __launch_bounds__(THREADS) void transpose_kernel(const uint16_t* __restrict__ kernel,
                                                            int64_t d, int32_t n, int32_t npad,
                                                            uint16_t* __restrict__ kt) {
  __shared__ uint16_t tile[32][33];
  const int64_t j0 = static_cast<int64_t>(blockIdx.x) * 32;  // rows of kernel (d)
  const int32_t e0 = blockIdx.y * 32;                         // columns of kernel (n)
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;     // 8 rows at a time
#pragma unroll
  for (int r = ty; r < 32; r += 8) {
    const int64_t j = j0 + r;
    const int32_t e = e0 + tx;
    tile[r][tx] = (j < d && e < n) ? kernel[j * n + e] : 0;
  }
  __syncthreads();
#pragma unroll
  for (int r = ty; r < 32; r += 8) {
    const int32_t e = e0 + r;
    const int64_t j = j0 + tx;
    if (e < npad && j < d) kt[static_cast<int64_t>(e) * d + j] = tile[tx][r];
  }
}

__device__ __forceinline__ bf16x8 load8(const uint16_t* p) {
  return __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(p));
}

struct Params {
  const uint16_t* x;
  const uint16_t* kt;
  const float* bias;
  const float* choice_bias;
  int64_t t, d;
  int32_t n, npad, scored, k, groups, keep, router;
  float logit_scale, scaling;
  bool normalize;
  int32_t* idx;
  uint16_t* weights;
  uint16_t* sinks;
  float* scores;
  float* logits;
};

// The k (at most CAP) largest of a stream of values in arrival order, the largest first,
// a value equal to one held going after it (so ties go to the earlier index). Registers
// only: every index into the arrays is a constant after unrolling.
template <int CAP>
struct Best {
  float val[CAP];
  int32_t at[CAP];
  int32_t held;   // values held, at most k
  float last;     // the k-th value held (once k are)

  __device__ __forceinline__ void clear() {
#pragma unroll
    for (int j = 0; j < CAP; ++j) {
      val[j] = -INFINITY;
      at[j] = -1;
    }
    held = 0;
    last = -INFINITY;
  }
  __device__ __forceinline__ void offer(float v, int32_t i, int32_t k) {
    if (held == k && !(v > last)) return;
    int32_t p = 0;  // the held values >= v stay ahead of it
#pragma unroll
    for (int j = 0; j < CAP; ++j) p += (j < held && val[j] >= v) ? 1 : 0;
#pragma unroll
    for (int j = CAP - 1; j > 0; --j) {
      if (j < k && j > p) {
        val[j] = val[j - 1];
        at[j] = at[j - 1];
      }
    }
#pragma unroll
    for (int j = 0; j < CAP; ++j) {
      if (j == p) {
        val[j] = v;
        at[j] = i;
      }
    }
    if (held < k) ++held;
#pragma unroll
    for (int j = 0; j < CAP; ++j)
      if (j == k - 1) last = val[j];
  }
  // Drops the largest.
  __device__ __forceinline__ void pop() {
#pragma unroll
    for (int j = 0; j + 1 < CAP; ++j) {
      val[j] = val[j + 1];
      at[j] = at[j + 1];
    }
    --held;
  }
};

__device__ __forceinline__ float softplus(float v) {
  // log(1 + e^v) = max(v, 0) + log1p(e^-|v|)
  return fmaxf(v, 0.0f) + log1pf(expf(-fabsf(v)));
}

// bfloat16 bits of bf16(w) * bf16(factor), the product rounded to bfloat16.
__device__ __forceinline__ uint16_t scaled_bf16(float w, float factor_bf16) {
  const uint16_t b = f32_to_bf16(w);
  return factor_bf16 == 1.0f ? b : f32_to_bf16(bf16_to_f32(b) * factor_bf16);
}

// Reductions over the LANES lanes of a token (lanes LANES q .. LANES q + LANES - 1).
template <int LANES>
__device__ __forceinline__ float lanes_max(float v) {
#pragma unroll
  for (int o = 1; o < LANES; o <<= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}
template <int LANES>
__device__ __forceinline__ float lanes_sum(float v) {
#pragma unroll
  for (int o = 1; o < LANES; o <<= 1) v += __shfl_xor(v, o);
  return v;
}

// The logits' row pitch in floats: 8 past a multiple of 32, so that the 64 lanes of a
// wave, 8 tokens x 8 lanes (or 16 x 4) reading neighbouring columns of their rows, hit
// 64 banks (32 at worst); and the MFMA results' two lane halves, rows 4 apart, land 32
// banks apart.
__device__ __host__ __forceinline__ int pitch_of(int npad) { return npad + 8; }

// Once the logits sit in `tile` (TOKS rows of `pitch` floats from token t0): the
// scores, the group limit, the picks and the weights, LANES lanes a token.
template <int TOKS, int CAP>
__device__ __forceinline__ void select(const Params& p, float* tile, int pitch, int64_t t0,
                                       uint64_t* kept_groups) {
  constexpr int LANES = THREADS / TOKS;
  // lane s of token q takes the columns s, s + LANES, ...
  const int q = threadIdx.x / LANES, s = threadIdx.x % LANES;
  float* row = tile + q * pitch;
  const int n = p.n, scored = p.scored;
  if (p.router == BUX_ROUTER_SOFTMAX) {
    float m = -INFINITY;
    for (int i = s; i < n; i += LANES) m = fmaxf(m, row[i]);
    m = lanes_max<LANES>(m);
    float sum = 0.0f;
    for (int i = s; i < n; i += LANES) {
      const float e = __expf(row[i] - m);
      row[i] = e;
      sum += e;
    }
    const float inv = 1.0f / lanes_sum<LANES>(sum);
    for (int i = s; i < n; i += LANES) row[i] *= inv;
  } else if (p.router == BUX_ROUTER_SIGMOID) {
    for (int i = s; i < n; i += LANES) row[i] = 1.0f / (1.0f + __expf(-row[i]));
  } else {
    for (int i = s; i < n; i += LANES) row[i] = sqrtf(softplus(row[i]));
  }
  __syncthreads();
  auto choice = [&](int i) { return p.choice_bias ? row[i] + p.choice_bias[i] : row[i]; };
  const int per = scored / p.groups;
  uint64_t kept = ~0ull;  // the groups kept, a bit each
  if (p.groups > 1) {
    if (s == 0) {
      Best<MAX_PICKS> g;
      g.clear();
      for (int grp = 0; grp < p.groups; ++grp) {
        float b1 = -INFINITY, b2 = -INFINITY;
        for (int i = grp * per; i < (grp + 1) * per; ++i) {
          const float v = choice(i);
          if (v > b1) {
            b2 = b1;
            b1 = v;
          } else if (v > b2) {
            b2 = v;
          }
        }
        g.offer(per >= 2 ? b1 + b2 : b1, grp, p.keep);
      }
      uint64_t bits = 0;
#pragma unroll
      for (int j = 0; j < MAX_PICKS; ++j)
        if (j < p.keep) bits |= 1ull << g.at[j];
      kept_groups[q] = bits;
    }
    __syncthreads();
    kept = kept_groups[q];
  }
  // Each lane's k best of its columns, then k rounds of the lanes' best of the best.
  Best<CAP> mine;
  mine.clear();
  for (int i = s; i < scored; i += LANES)
    mine.offer(((kept >> (i / per)) & 1ull) ? choice(i) : -INFINITY, i, p.k);
  int32_t pick[CAP];
#pragma unroll
  for (int j = 0; j < CAP; ++j) {
    pick[j] = 0;
    if (j < p.k) {
      int has = mine.held > 0;
      float v = mine.val[0];
      int32_t i = has ? mine.at[0] : 0x7fffffff;
#pragma unroll
      for (int o = 1; o < LANES; o <<= 1) {
        const float ov = __shfl_xor(v, o);
        const int32_t oi = __shfl_xor(i, o);
        const int oh = __shfl_xor(has, o);
        if (oh && (!has || ov > v || (ov == v && oi < i))) {
          v = ov;
          i = oi;
          has = oh;
        }
      }
      pick[j] = i;
      if (mine.held > 0 && mine.at[0] == i) mine.pop();
    }
  }
  if (s == 0 && t0 + q < p.t) {
    const int64_t tok = t0 + q;
    float total = 0.0f;
#pragma unroll
    for (int j = 0; j < CAP; ++j)
      if (j < p.k) total = j == 0 ? row[pick[j]] : total + row[pick[j]];
    if (n > scored) {
      float sinks = row[scored];
      for (int i = scored + 1; i < n; ++i) sinks += row[i];
      total += sinks;
    }
    const float factor = bf16_to_f32(f32_to_bf16(p.scaling));
#pragma unroll
    for (int j = 0; j < CAP; ++j) {
      if (j < p.k) {
        const float w = row[pick[j]];
        p.idx[tok * p.k + j] = pick[j];
        p.weights[tok * p.k + j] = scaled_bf16(p.normalize ? w / total : w, factor);
      }
    }
    for (int i = scored; i < n; ++i)
      p.sinks[tok * (n - scored) + (i - scored)] =
          scaled_bf16(p.normalize ? row[i] / total : row[i], factor);
  }

  if (p.scores) {
    __syncthreads();
    for (int i = threadIdx.x; i < TOKS * p.scored; i += THREADS) {
      const int rr = i / p.scored, col = i % p.scored;
      if (t0 + rr < p.t) p.scores[(t0 + rr) * p.scored + col] = tile[rr * pitch + col];
    }
  }
}

// SPLIT = 4 (at most 256 logits): wave w sums a quarter of K over every 32-column
//   block, and the four partial sums meet in LDS, added in wave order.
// SPLIT = 1 (wider): wave w sums all of K over the column blocks w, w + 4, ...
// BLOCKS: the column blocks a wave holds. TOKS: tokens a workgroup, 32 or (at most 128
// logits) 64, each row block of 32 taking the same kernel operands: the kernel's
// bytes a token halve. CAP: the picks a list holds (k at most).
template <int SPLIT, int BLOCKS, int TOKS, int CAP>
__global__ __launch_bounds__(THREADS) void route_kernel(Params p) {
  constexpr int RB = TOKS / 32;
  extern __shared__ __align__(16) float lds[];  // SPLIT tiles of TOKS rows
  __shared__ uint64_t kept_groups[TOKS];
  const int pitch = pitch_of(p.npad);
  float* tile = lds;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int r = lane & 31, h = lane >> 5;
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * TOKS;
  const int nb = p.npad / 32;

  // --- logits: rows past t load the last row (not stored)
  {
    constexpr int U = BLOCKS * RB <= 4 ? 4 : 2;  // K chunks of 16 a turn
    const int64_t chunks = p.d / 16;
    const int64_t c_lo = SPLIT == 4 ? chunks * wave / 4 : 0;
    const int64_t c_hi = SPLIT == 4 ? chunks * (wave + 1) / 4 : chunks;
    const uint16_t* xa[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      const int64_t tok = t0 + rb * 32 + r < p.t ? t0 + rb * 32 + r : p.t - 1;
      xa[rb] = p.x + tok * p.d + 8 * h;
    }
    const uint16_t* kb[BLOCKS];
    bool live[BLOCKS];
#pragma unroll
    for (int j = 0; j < BLOCKS; ++j) {
      const int c = SPLIT == 4 ? j : wave + 4 * j;
      live[j] = c < nb;
      kb[j] = p.kt + static_cast<int64_t>((live[j] ? c : 0) * 32 + r) * p.d + 8 * h;
    }
    v16f acc[RB][BLOCKS];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int j = 0; j < BLOCKS; ++j) acc[rb][j] = v16f{};
    int64_t c = c_lo;
    for (; c + U <= c_hi; c += U) {
      bf16x8 a[RB][U], b[BLOCKS][U];
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int u = 0; u < U; ++u) a[rb][u] = load8(xa[rb] + (c + u) * 16);
#pragma unroll
      for (int j = 0; j < BLOCKS; ++j)
#pragma unroll
        for (int u = 0; u < U; ++u) b[j][u] = live[j] ? load8(kb[j] + (c + u) * 16) : bf16x8{};
#pragma unroll
      for (int j = 0; j < BLOCKS; ++j)
        if (live[j])
#pragma unroll
          for (int u = 0; u < U; ++u)
#pragma unroll
            for (int rb = 0; rb < RB; ++rb)
              acc[rb][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[rb][u], b[j][u], acc[rb][j],
                                                                   0, 0, 0);
    }
    for (; c < c_hi; ++c) {
#pragma unroll
      for (int j = 0; j < BLOCKS; ++j) {
        if (!live[j]) continue;
        const bf16x8 b = load8(kb[j] + c * 16);
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
          acc[rb][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(load8(xa[rb] + c * 16), b,
                                                               acc[rb][j], 0, 0, 0);
      }
    }
    // Lane l holds column l % 32 of a block, token rows 8 (q / 4) + 4 h + q % 4.
    float* dst = SPLIT == 4 ? lds + wave * TOKS * pitch : tile;
#pragma unroll
    for (int j = 0; j < BLOCKS; ++j) {
      const int col = (SPLIT == 4 ? j : wave + 4 * j) * 32 + r;
      if (!live[j] || col >= p.n) continue;
      const float bias = SPLIT == 1 && p.bias ? p.bias[col] : 0.0f;
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int q = 0; q < 16; ++q) {
          const int row = rb * 32 + 8 * (q >> 2) + 4 * h + (q & 3);
          dst[row * pitch + col] =
              SPLIT == 4 ? acc[rb][j][q] : (acc[rb][j][q] + bias) * p.logit_scale;
        }
    }
  }
  __syncthreads();
  if (SPLIT == 4) {
    for (int i = threadIdx.x; i < TOKS * p.n; i += THREADS) {
      const int at = (i / p.n) * pitch + i % p.n;
      const float v = ((lds[at] + lds[at + TOKS * pitch]) + lds[at + 2 * TOKS * pitch]) +
                      lds[at + 3 * TOKS * pitch];
      tile[at] = (v + (p.bias ? p.bias[i % p.n] : 0.0f)) * p.logit_scale;
    }
    __syncthreads();
  }
  if (p.logits) {
    for (int i = threadIdx.x; i < TOKS * p.n; i += THREADS) {
      const int row = i / p.n, col = i % p.n;
      if (t0 + row < p.t) p.logits[(t0 + row) * p.n + col] = tile[row * pitch + col];
    }
    __syncthreads();  // copied before the scores overwrite them
  }

  select<TOKS, CAP>(p, tile, pitch, t0, kept_groups);
}

// s_waitcnt vmcnt(N) alone (gfx9's encoding: vmcnt's low bits at 3:0 and high bits at
// 15:14, expcnt and lgkmcnt at their maxima).
template <int N>
__device__ __forceinline__ void wait_vm() {
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// The K loop staged through LDS (at most 256 logits, d a multiple of 64). A workgroup
// takes TOKS tokens (32 or 64); per step of 64 columns of K, the tokens' 128-byte row
// pieces (TOKS / 8 KiB) and the transposed kernel's (128 CB rows, 16 CB KiB) go straight
// from global memory into a stage of LDS (buffer_load ... lds, 1 KiB an instruction),
// STAGES - 1 steps ahead, one barrier a step; wave w multiplies the tokens by its CB
// blocks of 32 experts from LDS. A stage's rows are 128 bytes, their 16-byte chunk c at
// c ^ ((row / 2) % 8), so the 16 lanes that read one chunk of 16 rows hit 16 different
// bank groups; a load's lane i takes the chunk that belongs at its place. After the loop
// the stages hold the logits tile.
template <int TOKS>
constexpr int staged_stages(int cb) { return TOKS == 32 ? 3 : (cb == 1 ? 4 : 3); }
template <int CB, int CAP, int TOKS>
__global__ __launch_bounds__(THREADS) void route_staged_kernel(Params p) {
  constexpr int RB = TOKS / 32;  // row blocks of 32 tokens, and a wave's loads of x a step
  constexpr int NPAD = 128 * CB;
  constexpr int X_BYTES = TOKS * 128;
  constexpr int STAGE = X_BYTES + NPAD * 128;
  constexpr int STAGES = staged_stages<TOKS>(CB);
  constexpr int LPS = RB + NPAD / 32;  // a wave's loads a step: RB of x, 4 CB of kernel
  extern __shared__ __align__(16) float lds[];
  __shared__ uint64_t kept_groups[TOKS];
  const int pitch = pitch_of(p.npad);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int r = lane & 31, h = lane >> 5;
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * TOKS;
  const uint32_t lds0 = lds_at(lds);
  const int64_t row_bytes = p.d * 2;
  // x from the workgroup's first token (past t reads 0), the kernel's padded rows
  // (past npad read 0).
  const i32x4 xr = resource(p.x + t0 * p.d, (p.t - t0) * row_bytes);
  const i32x4 kr = resource(p.kt, static_cast<int64_t>(p.npad) * row_bytes);
  // This lane's place in a 1 KiB slice of 8 rows, and the chunk that belongs there.
  const int srow = lane >> 3, place = lane & 7;
  auto voff = [&](int row) { return row * static_cast<int>(row_bytes) + 16 * (place ^ ((row >> 1) & 7)); };
  int xoff[RB], koff[4 * CB];
#pragma unroll
  for (int j = 0; j < RB; ++j) xoff[j] = voff((RB * wave + j) * 8 + srow);
#pragma unroll
  for (int j = 0; j < 4 * CB; ++j) koff[j] = voff((wave * 4 * CB + j) * 8 + srow);
  const int steps = static_cast<int>(p.d / 64);
  auto issue = [&](int ks, int st) {
    const uint32_t at = lds0 + st * STAGE;
#pragma unroll
    for (int j = 0; j < RB; ++j)
      load_lds16_uniform(xr, at + (RB * wave + j) * 1024, xoff[j], ks * 128);
#pragma unroll
    for (int j = 0; j < 4 * CB; ++j)
      load_lds16_uniform(kr, at + X_BYTES + (wave * 4 * CB + j) * 1024, koff[j], ks * 128);
  };
  // Lane offsets of the fragments: row block rb of x, expert block cb of the wave; the
  // chunk of K sub-step u is 2 u + h.
  auto frag_at = [&](int row, int u) { return row * 128 + 16 * ((2 * u + h) ^ ((row >> 1) & 7)); };
  v16f acc[RB][CB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) acc[rb][cb] = v16f{};
  for (int s0 = 0; s0 < STAGES - 1 && s0 < steps; ++s0) issue(s0, s0);
  const uint8_t* base = reinterpret_cast<const uint8_t*>(lds);
  for (int ks = 0; ks < steps; ++ks) {
    const int later = steps - 1 - ks;  // steps issued after this one, at most STAGES - 2
    if (later >= 2 && STAGES > 3) wait_vm<2 * LPS>();
    else if (later >= 1) wait_vm<LPS>();
    else wait_vm<0>();
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    if (ks + STAGES - 1 < steps) issue(ks + STAGES - 1, (ks + STAGES - 1) % STAGES);
    const uint8_t* st = base + (ks % STAGES) * STAGE;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      bf16x8 a[RB], b[CB];
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
        a[rb] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(st + frag_at(rb * 32 + r, u)));
#pragma unroll
      for (int cb = 0; cb < CB; ++cb)
        b[cb] = __builtin_bit_cast(
            bf16x8, *reinterpret_cast<const uint4*>(st + X_BYTES + frag_at((wave * CB + cb) * 32 + r, u)));
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int cb = 0; cb < CB; ++cb)
          acc[rb][cb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[rb], b[cb], acc[rb][cb], 0, 0, 0);
    }
  }
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");  // every stage read
  float* tile = lds;
#pragma unroll
  for (int cb = 0; cb < CB; ++cb) {
    const int col = (wave * CB + cb) * 32 + r;
    if (col >= p.n) continue;
    const float bias = p.bias ? p.bias[col] : 0.0f;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int q = 0; q < 16; ++q) {
        const int row = rb * 32 + 8 * (q >> 2) + 4 * h + (q & 3);
        tile[row * pitch + col] = (acc[rb][cb][q] + bias) * p.logit_scale;
      }
  }
  __syncthreads();
  if (p.logits) {
    for (int i = threadIdx.x; i < TOKS * p.n; i += THREADS) {
      const int row = i / p.n, col = i % p.n;
      if (t0 + row < p.t) p.logits[(t0 + row) * p.n + col] = tile[row * pitch + col];
    }
    __syncthreads();  // copied before the scores overwrite them
  }
  select<TOKS, CAP>(p, tile, pitch, t0, kept_groups);
}

template <int CB, int CAP, int TOKS>
int launch_staged_of(const Params& p, hipStream_t s) {
  constexpr int STAGE = (TOKS + 128 * CB) * 128, STAGES = staged_stages<TOKS>(CB);
  const size_t tile = static_cast<size_t>(TOKS) * pitch_of(p.npad) * sizeof(float);
  const size_t lds = tile > static_cast<size_t>(STAGES * STAGE) ? tile : STAGES * STAGE;
  const void* kernel = reinterpret_cast<const void*>(route_staged_kernel<CB, CAP, TOKS>);
  hipError_t err = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                       static_cast<int>(lds));
  if (err != hipSuccess) return fail(BUX_E_LAUNCH, "route_staged_kernel: %s", hipGetErrorString(err));
  hipLaunchKernelGGL((route_staged_kernel<CB, CAP, TOKS>), dim3(static_cast<unsigned>(ceil_div(p.t, TOKS))),
                     dim3(THREADS), lds, s, p);
  return launched("route_staged_kernel");
}

// 32 tokens a workgroup for up to 128 logits (two workgroups a CU in LDS, one's
// selection beside the other's K loop); 64 for more.
template <int CB, int CAP>
int launch_staged(const Params& p, hipStream_t s) {
  if constexpr (CB == 1) return launch_staged_of<CB, CAP, 32>(p, s);
  else return launch_staged_of<CB, CAP, 64>(p, s);
}

template <int SPLIT, int BLOCKS, int TOKS, int CAP>
int launch(const Params& p, hipStream_t s) {
  const size_t lds = static_cast<size_t>(SPLIT) * TOKS * pitch_of(p.npad) * sizeof(float);
  const void* kernel = reinterpret_cast<const void*>(route_kernel<SPLIT, BLOCKS, TOKS, CAP>);
  hipError_t err = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                       static_cast<int>(lds));
  if (err != hipSuccess) return fail(BUX_E_LAUNCH, "route_kernel: %s", hipGetErrorString(err));
  hipLaunchKernelGGL((route_kernel<SPLIT, BLOCKS, TOKS, CAP>),
                     dim3(static_cast<unsigned>(ceil_div(p.t, TOKS))), dim3(THREADS), lds, s, p);
  return launched("route_kernel");
}

template <int CAP>
int launch_for(const Params& p, hipStream_t s) {
  const int nb = p.npad / 32;
  if (p.d % 64 == 0 && nb <= 4) return launch_staged<1, CAP>(p, s);
  if (p.d % 64 == 0 && nb <= 8) return launch_staged<2, CAP>(p, s);
  if (nb <= 1) return launch<4, 1, 64, CAP>(p, s);
  if (nb <= 2) return launch<4, 2, 64, CAP>(p, s);
  if (nb <= 4) return launch<4, 4, 64, CAP>(p, s);
  if (nb <= 8) return launch<4, 8, 32, CAP>(p, s);
  if (nb <= 16) return launch<1, 4, 32, CAP>(p, s);
  return launch<1, 8, 32, CAP>(p, s);
}

int32_t padded(int32_t n) { return static_cast<int32_t>(ceil_div(n, 32) * 32); }

}  // namespace
}  // namespace bux

extern "C" size_t bux_route_workspace_size(int64_t d, int32_t n_logits) {
  using namespace bux;
  if (d <= 0 || n_logits <= 0) return 0;
  return static_cast<size_t>(padded(n_logits)) * static_cast<size_t>(d) * sizeof(uint16_t);
}

extern "C" int bux_route(const uint16_t* x, const uint16_t* kernel, const float* bias, int64_t t,
                         int64_t d, int32_t n_logits, float logit_scale, int router,
                         int32_t scored, const float* choice_bias, int32_t groups, int32_t keep,
                         int32_t k, int normalize, float scaling, int32_t* idx, uint16_t* weights,
                         uint16_t* sinks, float* scores, float* logits, void* workspace,
                         size_t workspace_bytes, void* stream) {
  using namespace bux;
  clear_error();
  BUX_CHECK(t >= 0 && t < (1LL << 31) && d > 0 && d % 16 == 0 && d < (1LL << 31),
            "bux_route: t=%lld d=%lld (d a positive multiple of 16)", (long long)t, (long long)d);
  BUX_CHECK(n_logits >= 1 && n_logits <= MAX_LOGITS, "bux_route: n_logits=%d outside [1, %d]",
            n_logits, MAX_LOGITS);
  BUX_CHECK(scored >= 1 && scored <= n_logits, "bux_route: scored=%d outside [1, %d]", scored,
            n_logits);
  BUX_CHECK(router == BUX_ROUTER_SOFTMAX || router == BUX_ROUTER_SIGMOID ||
                router == BUX_ROUTER_SQRTSOFTPLUS,
            "bux_route: router=%d", router);
  BUX_CHECK(k >= 1 && k <= MAX_PICKS && k <= scored, "bux_route: k=%d outside [1, min(%d, %d)]",
            k, MAX_PICKS, scored);
  BUX_CHECK(groups >= 1 && groups <= MAX_GROUPS && scored % groups == 0,
            "bux_route: groups=%d (at most %d, dividing scored=%d)", groups, MAX_GROUPS, scored);
  BUX_CHECK(keep >= 1 && keep <= groups && keep <= MAX_PICKS,
            "bux_route: keep=%d outside [1, min(groups=%d, %d)]", keep, groups, MAX_PICKS);
  BUX_CHECK(groups == 1 || keep * (scored / groups) >= k,
            "bux_route: %d kept groups of %d experts hold fewer than k=%d", keep,
            scored / groups, k);
  BUX_CHECK(kernel && (t == 0 || (x && idx && weights && (n_logits == scored || sinks))),
            "bux_route: NULL buffer");
  const size_t need = bux_route_workspace_size(d, n_logits);
  if (workspace == nullptr || workspace_bytes < need)
    return fail(BUX_E_WORKSPACE, "bux_route: workspace of %zu bytes, %zu needed",
                workspace_bytes, need);
  if (t == 0) return BUX_OK;
  hipStream_t s = as_stream(stream);
  Params p{};
  p.x = x;
  p.kt = static_cast<const uint16_t*>(workspace);
  p.bias = bias;
  p.choice_bias = choice_bias;
  p.t = t;
  p.d = d;
  p.n = n_logits;
  p.npad = padded(n_logits);
  p.scored = scored;
  p.k = k;
  p.groups = groups;
  p.keep = keep;
  p.router = router;
  p.logit_scale = logit_scale;
  p.scaling = scaling;
  p.normalize = normalize != 0;
  p.idx = idx;
  p.weights = weights;
  p.sinks = sinks;
  p.scores = scores;
  p.logits = logits;
  hipLaunchKernelGGL(transpose_kernel, dim3(static_cast<unsigned>(ceil_div(d, 32)), p.npad / 32),
                     dim3(THREADS), 0, s, kernel, d, n_logits, p.npad,
                     static_cast<uint16_t*>(workspace));
  if (int rc = launched("transpose_kernel")) return rc;
  return k <= 8 ? launch_for<8>(p, s) : launch_for<16>(p, s);
}
