// bfloat16 grouped GEMMs (the experts in "compute" precision) on CDNA4's
// v_mfma_f32_32x32x16_bf16: float32 sums, bfloat16 out.
//
//   rows      y[i] = x[i] w[g(i)]   (w [g, k, n]) or x[i] w[g(i)]^T (w [g, n, k], the
//             dgrad): grouped.dot / jax.lax.ragged_dot, src/bux/architecture/experts/
//             grouped.py:90-102; rows past sum(sizes) are 0.
//   contract  dw[g] = x[rows of g]^T dy[rows of g]   grouped.py:105-146.
//
// The schedule is the MXFP8 GEMMs' (tiles.h): a tile list built on the device, a
// persistent grid split by XCD, 256 x 256 output tiles of 4 waves (each 128 x 128 as
// 4 x 4 MFMAs of 32 x 32: 256 accumulator registers, one wave a SIMD) and a ring of 4
// LDS stages that direct loads (buffer_load ... lds) fill 4 steps ahead. A step is 32 of
// K, 64 bytes of an operand's row: 32 MFMAs a wave, the same MFMA time for the bytes
// loaded as an MXFP8 step's 16 MFMAs at twice the rate.
//
// Operands arrive as the reference holds them, in two layouts, and either sits in a
// stage as it lies in memory:
//  - K-major, A(r, k) at p[r ld + k] (x; w of the dgrad): a stage holds 256 rows of 64
//    bytes, 16-byte chunk c of row r at place c ^ ((r / 4) % 4) (16 lanes of a
//    ds_read_b128 read one chunk of 16 rows, every bank once); a lane's MFMA operand (row
//    l % 32, K 8 (l / 32) .. + 7) is one ds_read_b128.
//  - MN-major, A(r, k) at p[k ld + r] (w of the fprop; x and dy of the wgrad): a stage
//    holds 32 rows of K of 512 bytes (the tile's 256 r), chunk c of K row k at place
//    c ^ 4 (k % 4). gfx950's ds_read_b64_tr_b16 transposes on the way out of LDS:
//    measured on the MI355X, within each 16 lanes, lane j's 16-bit element e is element
//    j % 4 of the 8 bytes that lane 4 e + j / 4 read. So lane s of a 16 reads K row s / 4
//    at r = 4 (s % 4) .. + 3 (16 more in the odd 16), and lane j ends up with column
//    j of 4 consecutive K rows: two such reads make the MFMA's operand. The 32 lanes of
//    one read touch 4 K rows x 64 bytes, the swizzle putting each row's 64 bytes on
//    banks of their own.
//
// Edges: rows and K rows past an operand read 0 (the buffer resource ends there); a
// K step that holds K positions that are not the tile's (the wgrad's group boundaries;
// K past the rows GEMM's k) has both operands' registers of those positions zeroed
// before its MFMAs, so that nothing past them, NaN included, reaches a sum.

#include "tiles.h"

namespace bux {
namespace {

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef short v4s __attribute__((ext_vector_type(4)));
typedef short v8s __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) v4s lds_v4s;
typedef __attribute__((address_space(3))) uint4 lds_u4;

constexpr int BK = 32;     // K a step
constexpr int LOADS = 8;   // direct loads a wave issues a step: 4 of A, 4 of B

// A matrix: `p` (a group's matrix of B: p + group `stride`), `ld` elements from one row
// (K-major) or one K row (MN-major) to the next, `bytes` of it readable from there.
struct Operand {
  const uint16_t* p;
  int32_t ld;
  int32_t bytes;
  int64_t stride;
};

struct Stage {
  uint16_t a[BM * BK];
  uint16_t b[BN * BK];
};
struct Lds {
  Stage st[STAGES];
};
constexpr uint32_t B_AT = offsetof(Stage, b);

// A wave's direct loads of one operand's tile: its lane's offset, and the scalar bytes
// from one of its 4 loads of a step to the next and from one K step to the next.
//  K-major: wave w's load i holds rows 64 w + 16 i .. + 15 (1 KiB of LDS), lane l row
//    l / 4, the chunk that belongs in place l % 4.
//  MN-major: wave w's load i holds K rows 8 i + 2 w and + 1, lane l K row l / 32 and
//    the chunk that belongs in place l % 32. (Place ^ chunk depends on the K row mod 4,
//    the same for every i.)
struct Loads {
  i32x4 rsrc;
  int32_t voff, slice, step;
};

template <bool KM>
__device__ __forceinline__ Loads loads_for(const uint16_t* p, int32_t ld, int32_t bytes, int32_t row0) {
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  Loads o;
  o.rsrc = resource(p, bytes);
  if (KM) {
    o.voff = (row0 + w * 64 + (l >> 2)) * ld * 2 + 16 * ((l & 3) ^ ((l >> 4) & 3));
    o.slice = 16 * ld * 2;
    o.step = BK * 2;
  } else {
    const int k = 2 * w + (l >> 5);
    o.voff = k * ld * 2 + row0 * 2 + 16 * ((l & 31) ^ (4 * (k & 3)));
    o.slice = 8 * ld * 2;
    o.step = BK * ld * 2;
  }
  return o;
}

// Where in its operand's part of a stage wave w's load i lands.
template <bool KM>
__device__ __forceinline__ uint32_t slice_at(uint32_t w, int i) {
  return KM ? w * 4096 + i * 1024 : (8 * i + 2 * w) * 512;
}

// This lane's byte offsets of its MFMA operands in an operand's part of a stage:
//  K-major: of 32-row block 0, K 0 .. 15 (off[0]) and 16 .. 31 (off[1]); block p 2048
//    bytes further.
//  MN-major: of the first of the two reads of block p (off[p]), K 0 .. 15; the second
//    read 4 K rows (2048 bytes) further, K 16 .. 31 16 K rows (8192 bytes) further.
template <bool KM>
__device__ __forceinline__ void lane_offsets(int32_t off[4], int wbase) {
  const int l = threadIdx.x & 63;
  if (KM) {
    const int row = wbase + (l & 31), sw = ((l & 31) >> 2) & 3;
    off[0] = row * 64 + 16 * ((l >> 5) ^ sw);
    off[1] = row * 64 + 16 * ((2 + (l >> 5)) ^ sw);
    off[2] = off[3] = 0;
  } else {
    const int s = l & 15, kq = s >> 2;
    const int k = 8 * (l >> 5) + kq;
    const int col = 16 * ((l >> 4) & 1) + 4 * (s & 3);
#pragma unroll
    for (int p = 0; p < 4; ++p)
      off[p] = k * 512 + 16 * (wbase / 8 + 4 * (p ^ kq) + (col >> 3)) + 8 * ((col >> 2) & 1);
  }
}

__device__ __forceinline__ v8bf read16(uint32_t at) {
  return __builtin_bit_cast(v8bf, *reinterpret_cast<const lds_u4*>(at));
}
__device__ __forceinline__ v8bf read_tr(uint32_t at) {
  const v4s x = __builtin_amdgcn_ds_read_tr16_b64_v4i16(reinterpret_cast<lds_v4s*>(at));
  const v4s y = __builtin_amdgcn_ds_read_tr16_b64_v4i16(reinterpret_cast<lds_v4s*>(at + 2048));
  return __builtin_bit_cast(v8bf, __builtin_shufflevector(x, y, 0, 1, 2, 3, 4, 5, 6, 7));
}

// Block p's operand registers of K half s (K 16 s .. 16 s + 15 of the step) from an
// operand's part of a stage at LDS address `at`.
template <bool KM>
__device__ __forceinline__ v8bf read_block(uint32_t at, const int32_t off[4], int p, int s) {
  return KM ? read16(at + p * 2048 + off[s]) : read_tr(at + off[p] + s * 8192);
}

// Zeroes the 16-bit elements of v whose K (k0 + e for element e) lies outside [lo, hi).
__device__ __forceinline__ v8bf masked(v8bf v, int32_t k0, int32_t lo, int32_t hi) {
  u32x4 u = __builtin_bit_cast(u32x4, v);
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    const int32_t k = k0 + 2 * d;
    const uint32_t keep = (k >= lo && k < hi ? 0xffffu : 0u) | (k + 1 >= lo && k + 1 < hi ? 0xffff0000u : 0u);
    u[d] &= keep;
  }
  return __builtin_bit_cast(v8bf, u);
}

// The bfloat16 format's part of the shared pipeline (run_tiles): A K-major or not (AK),
// B likewise (BKM).
template <bool AK, bool BKM>
struct Bf16 {
  using Operand = bux::Operand;
  using Lds = bux::Lds;
  using Loads = bux::Loads;
  static constexpr bool HALVES = false;  // whole tiles only
  struct Lanes {
    int32_t a[4], b[4];
  };
  // A wave's operands of one step: 4 blocks of 32 rows of A and of B, each in two K
  // halves of 16.
  struct Frag {
    v8bf a[4][2], b[4][2];
  };

  __device__ static __forceinline__ Loads loads_a(const Operand& a, int32_t row0) {
    return loads_for<AK>(a.p, a.ld, a.bytes, row0);
  }
  __device__ static __forceinline__ Loads loads_b(const Operand& b, int32_t group, int32_t row0) {
    return loads_for<BKM>(b.p + group * b.stride, b.ld, b.bytes, row0);
  }

  // Direct load Q (0..7) of K step ks into stage `st`: even Q A's load Q / 2, odd B's.
  template <int Q>
  __device__ static __forceinline__ void issue_one(const Loads& la, const Loads& lb, int32_t ks,
                                                   uint32_t lds0, int st) {
    const uint32_t w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t at = lds0 + static_cast<uint32_t>(st * sizeof(Stage));
    constexpr int i = Q >> 1;
    if ((Q & 1) == 0)
      load_lds16(la.rsrc, at + slice_at<AK>(w, i), la.voff, ks * la.step + i * la.slice);
    else
      load_lds16(lb.rsrc, at + B_AT + slice_at<BKM>(w, i), lb.voff, ks * lb.step + i * lb.slice);
  }
  template <int Q>
  __device__ static __forceinline__ void issue_from(const Loads& la, const Loads& lb, int32_t ks,
                                                    uint32_t lds0, int st) {
    issue_one<Q>(la, lb, ks, lds0, st);
    if constexpr (Q + 1 < LOADS) issue_from<Q + 1>(la, lb, ks, lds0, st);
  }
  __device__ static __forceinline__ void issue(const Loads& la, const Loads& lb, int32_t ks,
                                               uint32_t lds0, int st, bool) {
    issue_from<0>(la, lb, ks, lds0, st);
  }

  // Waits until at most `steps` steps' loads of this wave are in flight (a wave's loads
  // complete in the order they were issued).
  __device__ static __forceinline__ void wait_loads(int32_t steps) {
    if (steps >= 3) asm volatile("s_waitcnt vmcnt(24)" ::: "memory");
    else if (steps == 2) asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
    else if (steps == 1) asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
    else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  }

  template <bool H>
  __device__ static __forceinline__ Lanes lanes_of() {
    static_assert(!H, "no half tiles");
    const int wave = threadIdx.x >> 6;
    Lanes ln;
    lane_offsets<AK>(ln.a, (wave >> 1) * 128);
    lane_offsets<BKM>(ln.b, (wave & 1) * 128);
    return ln;
  }

  // Read item x (0..15) of a step's operands, in the order its MFMAs take them: K half
  // x / 8, then A's block 0, B's blocks 0-3, A's blocks 1-3.
  __device__ static __forceinline__ void read_item(Frag& f, uint32_t at, const Lanes& ln, int x) {
    const int s = x >> 3, y = x & 7;
    if (y == 0) f.a[0][s] = read_block<AK>(at, ln.a, 0, s);
    else if (y <= 4) f.b[y - 1][s] = read_block<BKM>(at + B_AT, ln.b, y - 1, s);
    else f.a[y - 4][s] = read_block<AK>(at, ln.a, y - 4, s);
  }

  // All of a step's operands from stage `st`.
  template <bool H>
  __device__ static __forceinline__ void read_frag(Frag& f, const Lds& lds, const Lanes& ln, int st,
                                                   int32_t) {
    const uint32_t at = lds_at(&lds) + static_cast<uint32_t>(st * sizeof(Stage));
#pragma unroll
    for (int x = 0; x < 16; ++x) read_item(f, at, ln, x);
  }

  // Zeroes the K positions of step ks outside [lo, hi) in both operands: lane half h
  // holds K 16 s + 8 h .. + 7 of the step in its registers of half s.
  __device__ static __forceinline__ void mask_frag(Frag& f, int32_t ks, int32_t lo, int32_t hi) {
    const int h = (threadIdx.x & 63) >> 5;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int32_t k0 = ks * BK + 16 * s + 8 * h;
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        f.a[p][s] = masked(f.a[p][s], k0, lo, hi);
        f.b[p][s] = masked(f.b[p][s], k0, lo, hi);
      }
    }
  }

  // The 32 MFMAs of one step on `cur` (K half q / 16, A's block (q / 4) % 4, B's block
  // q % 4), each followed by a slice of the memory work: with LOAD, the next loads (step
  // ks_load into stage st_load) after MFMAs 1, 5, .. 29; with READ, the next step's
  // operands into `nxt` after the even MFMAs, in the order its MFMAs take them.
  template <bool LOAD, bool READ, bool H>
  __device__ static __forceinline__ void step(const Frag& cur, Frag& nxt, const Loads& la,
                                              const Loads& lb, const Lds&, uint32_t lds0,
                                              const Lanes& ln, int32_t ks_load, int st_load,
                                              int32_t, int st_next, v16f acc[4][4]) {
    const uint32_t next_at = lds0 + static_cast<uint32_t>(st_next * sizeof(Stage));
#pragma unroll
    for (int q = 0; q < 32; ++q) {
      const int s = q >> 4, i = (q >> 2) & 3, j = q & 3;
      acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(cur.b[j][s], cur.a[i][s], acc[i][j], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
      if (LOAD && (q & 3) == 1) {
        switch (q >> 2) {
          case 0: issue_one<0>(la, lb, ks_load, lds0, st_load); break;
          case 1: issue_one<1>(la, lb, ks_load, lds0, st_load); break;
          case 2: issue_one<2>(la, lb, ks_load, lds0, st_load); break;
          case 3: issue_one<3>(la, lb, ks_load, lds0, st_load); break;
          case 4: issue_one<4>(la, lb, ks_load, lds0, st_load); break;
          case 5: issue_one<5>(la, lb, ks_load, lds0, st_load); break;
          case 6: issue_one<6>(la, lb, ks_load, lds0, st_load); break;
          default: issue_one<7>(la, lb, ks_load, lds0, st_load); break;
        }
      }
      if (READ && (q & 1) == 0) read_item(nxt, next_at, ln, q >> 1);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
};

// --- the epilogue ------------------------------------------------------------------------

// Output stores are non-temporal: the tile is written once and read by another kernel,
// and a round of tiles' outputs passing through the XCD's L2 would evict the operands
// the other CUs are about to reuse.
constexpr int NT = 2;  // a buffer store's cache policy: non-temporal

// The tile's rows [0, rows) and columns [0, cols) (cols a multiple of 8) at row pitch
// ld from its corner, bfloat16 (v_cvt_pk_bf16_f32: nearest even), through the stage the
// tile's last step left: in 4 rounds of 32 rows, each wave puts its 32 x 128 outputs in
// a region of its own (8 KiB: 256 bytes a row, 16-byte chunk c of row r at place
// c ^ (r % 16) and its two 8-byte halves swapped in rows 16 .. 31, so that the 64 lanes
// of a write fill every bank twice and the 16 lanes that read a row back read it once
// each), reads it back 16 bytes a lane, 16 lanes a row, and stores 4 runs of 256 bytes an
// instruction. No other wave touches the region: no workgroup barrier.
__device__ void store_tile(const v16f acc[4][4], uint16_t* tile, int32_t ld, int32_t rows,
                           int32_t cols, Stage& stage) {
  static_assert(4 * 32 * 256 == sizeof(Stage), "the epilogue's regions fill a stage");
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  uint8_t* region = reinterpret_cast<uint8_t*>(&stage) + wave * 32 * 256;
  // Lane l writes row l % 32 of the block, its 4 columns of each 8 at half l / 32.
  const int r = lane & 31;
  uint8_t* mine = region + r * 256 + 8 * ((lane >> 5) ^ (r >> 4));
  const int sw = r & 15;
  // ... and reads back chunk l % 16 (8 columns) of rows l / 16 + 4 it.
  const int cc = lane & 15;
  const int32_t col = wn * 128 + 8 * cc;
  const bool whole = rows >= BM && cols >= BN;
  const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(tile, 0, 0x7fffffff, 0x00020000);
  const int32_t lane_off = ((wm * 128 + (lane >> 4)) * ld + col) * 2;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const v16f& a = acc[i][j];
        const bf16x2 lo = __builtin_convertvector((f32x2{a[4 * g], a[4 * g + 1]}), bf16x2);
        const bf16x2 hi = __builtin_convertvector((f32x2{a[4 * g + 2], a[4 * g + 3]}), bf16x2);
        *reinterpret_cast<uint2*>(mine + 16 * ((4 * j + g) ^ sw)) =
            make_uint2(__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi));
      }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_wave_barrier();
    // All 8 reads of the round go out before its first store.
    uint4 v[8];
#pragma unroll
    for (int it = 0; it < 8; ++it) {
      const int row = (lane >> 4) + 4 * it;
      const uint4 t = *reinterpret_cast<const uint4*>(region + row * 256 + 16 * (cc ^ (row & 15)));
      v[it] = it < 4 ? t : make_uint4(t.z, t.w, t.x, t.y);
    }
    if (whole) {
#pragma unroll
      for (int it = 0; it < 8; ++it)
        __builtin_amdgcn_raw_buffer_store_b128(u32x4{v[it].x, v[it].y, v[it].z, v[it].w}, rsrc,
                                               lane_off, (i * 32 + it * 4) * ld * 2, NT);
    } else if (col < cols) {
      uint16_t* out = tile + (wm * 128 + (lane >> 4)) * ld + col;
#pragma unroll
      for (int it = 0; it < 8; ++it) {
        const int32_t row = wm * 128 + i * 32 + it * 4 + (lane >> 4);
        if (row < rows)
          __builtin_nontemporal_store(u32x4{v[it].x, v[it].y, v[it].z, v[it].w},
                                      reinterpret_cast<u32x4*>(out + (i * 32 + it * 4) * ld));
      }
    }
    // The reads are done before the next round's writes.
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_wave_barrier();
  }
}

struct Out {
  uint16_t* out;
  int32_t ld;
  __device__ __forceinline__ void store(const v16f acc[4][4], const Job& j, Stage& stage) const {
    store_tile(acc, out + j.corner, ld, j.rows, j.cols, stage);
  }
};

// --- the kernels: one workgroup a CU -------------------------------------------------------

// rows: A = x (K-major), B = w (K-major when transposed); TAIL: k is not a whole number
// of steps.
template <bool BKM, bool TAIL>
__global__ __launch_bounds__(THREADS) __attribute__((amdgpu_waves_per_eu(1, 1))) void rows_kernel(
    Operand A, Operand B, int32_t groups, int32_t m, int32_t n, int32_t k,
    const int32_t* __restrict__ starts, const Tile* __restrict__ tiles, int32_t col_tiles,
    uint16_t* __restrict__ y) {
  extern __shared__ __align__(16) uint8_t smem[];
  if (!list_fits(starts, groups, m, m)) return;
  Lds& lds = *reinterpret_cast<Lds*>(smem);
  const RowsTiles<TAIL> list{tiles, groups, n, m, col_tiles, (k + BK - 1) / BK, k};
  const int32_t count = starts[groups + 1] * col_tiles;
  run_tiles<Bf16<true, BKM>>(list, count, A, B, lds, Out{y, n});
}

// contract: A = x, B = dy, both MN-major over the rows (K).
__global__ __launch_bounds__(THREADS) __attribute__((amdgpu_waves_per_eu(1, 1))) void contract_kernel(
    Operand A, Operand B, int32_t groups, int32_t d, int32_t f, const int32_t* __restrict__ starts,
    int32_t d_tiles, int32_t f_tiles, uint16_t* __restrict__ dw) {
  extern __shared__ __align__(16) uint8_t smem[];
  if (!list_fits(starts, groups, -1, 0)) return;
  Lds& lds = *reinterpret_cast<Lds*>(smem);
  const ContractTiles list{starts, d, f, d_tiles, f_tiles, BK};
  const int32_t count = groups * d_tiles * f_tiles;
  run_tiles<Bf16<false, false>>(list, count, A, B, lds, Out{dw, f});
}

// --- any shape ----------------------------------------------------------------------------
//
// A matrix whose rows are not a whole number of 16-byte chunks (n or k not a multiple
// of 8) has rows that start off the chunks, which the direct loads above cannot take;
// one past 2 GiB has offsets past the buffer loads' 32 bits. These kernels read their
// operands an element at a time (2-byte loads at 64-bit addresses, each checked against
// the matrix and the group) into LDS and otherwise multiply as the kernels above do:
// the same tile list, v_mfma_f32_32x32x16_bf16, float32 sums, one rounding to
// bfloat16. A workgroup of 4 waves takes 256 rows by 64 columns of the output, wave w
// its rows 64 w .. 64 w + 63 as 2 x 2 MFMA blocks of 32 x 32; K goes 16 a step. Both
// operands sit in LDS K-contiguous, 16 elements (32 bytes) a row, so that a lane's
// MFMA operand (row l % 32, K 8 (l / 32) .. + 7) is one 16-byte read.

constexpr int ANY_BN = 64;
constexpr int ANY_BK = 16;

struct AnyStage {
  uint16_t a[BM][ANY_BK];
  uint16_t b[ANY_BN][ANY_BK];
};

// The 4 MFMAs of a step: wave w's A blocks 2 w, 2 w + 1 (rows 64 w + 32 p) by B's 2.
__device__ __forceinline__ void any_step(const AnyStage& st, v16f acc[2][2]) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 31, h = lane >> 5;
  v8bf a[2], b[2];
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    a[p] = *reinterpret_cast<const v8bf*>(&st.a[wave * 64 + p * 32 + r][8 * h]);
    b[p] = *reinterpret_cast<const v8bf*>(&st.b[p * 32 + r][8 * h]);
  }
#pragma unroll
  for (int p = 0; p < 2; ++p)
#pragma unroll
    for (int q = 0; q < 2; ++q)
      acc[p][q] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[p], b[q], acc[p][q], 0, 0, 0);
}

// The block's outputs: lane l holds column 32 q + l % 32 of rows 64 w + 32 p + 8 (j / 4)
// + 4 (l / 32) + j % 4, stored where row < rows and column < cols (2-byte stores).
__device__ __forceinline__ void any_store(const v16f acc[2][2], uint16_t* tile, int64_t ld,
                                          int32_t rows, int32_t cols) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int p = 0; p < 2; ++p)
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int32_t col = q * 32 + (lane & 31);
      if (col >= cols) continue;
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int32_t row = wave * 64 + p * 32 + 8 * (j >> 2) + 4 * (lane >> 5) + (j & 3);
        if (row < rows) tile[row * ld + col] = f32_to_bf16(acc[p][q][j]);
      }
    }
}

__device__ __forceinline__ uint16_t any_at(const uint16_t* p, bool inside) { return inside ? *p : 0; }

// rows, any shape: y[i] = x[i] w[g(i)] (w [g, k, n]; BKM: w [g, n, k] and x[i] w[g(i)]^T).
// Block b: tile b / col_tiles of the list, columns 64 (b % col_tiles) on.
template <bool BKM>
__global__ __launch_bounds__(THREADS) void rows_any_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w, int32_t groups, int64_t m,
    int64_t n, int64_t k, const int32_t* __restrict__ starts, const Tile* __restrict__ tiles,
    int64_t col_tiles, uint16_t* __restrict__ y) {
  __shared__ __align__(16) AnyStage st;
  if (!list_fits(starts, groups, static_cast<int32_t>(m), static_cast<int32_t>(m))) return;
  const int64_t id = blockIdx.x / col_tiles;
  if (id >= starts[groups + 1]) return;
  const Tile t = tiles[id];
  const int64_t col0 = (blockIdx.x % col_tiles) * ANY_BN;
  const int64_t hi = t.hi < m ? t.hi : m;
  const int32_t rows = static_cast<int32_t>(hi - t.lo);
  if (rows <= 0) return;
  const int32_t cols = static_cast<int32_t>(n - col0 < ANY_BN ? n - col0 : ANY_BN);
  v16f acc[2][2];
#pragma unroll
  for (int p = 0; p < 2; ++p)
#pragma unroll
    for (int q = 0; q < 2; ++q)
#pragma unroll
      for (int j = 0; j < 16; ++j) acc[p][q][j] = 0.0f;
  if (t.group < groups) {  // the rows past the groups: zeros
    const uint16_t* wg = w + static_cast<int64_t>(t.group) * n * k;
    const int tid = threadIdx.x, kk = tid & 15;
    for (int64_t k0 = 0; k0 < k; k0 += ANY_BK) {
      const bool kin = k0 + kk < k;
      uint16_t av[16], bv[4];
      // A: 16 rows an instruction, 16 consecutive K of each
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int32_t r = (tid >> 4) + 16 * i;
        av[i] = any_at(x + (t.lo + r) * k + k0 + kk, kin && r < rows);
      }
      if constexpr (BKM) {  // w [g, n, k]: 16 columns an instruction, 16 consecutive K
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int32_t c = (tid >> 4) + 16 * i;
          bv[i] = any_at(wg + (col0 + c) * k + k0 + kk, kin && c < cols);
        }
      } else {  // w [g, k, n]: K row tid / 16, 4 consecutive columns
        const int64_t kr = k0 + (tid >> 4);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int32_t c = 4 * (tid & 15) + i;
          bv[i] = any_at(wg + kr * n + col0 + c, kr < k && c < cols);
        }
      }
      __syncthreads();  // the last step's reads are done
#pragma unroll
      for (int i = 0; i < 16; ++i) st.a[(tid >> 4) + 16 * i][kk] = av[i];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if constexpr (BKM) st.b[(tid >> 4) + 16 * i][kk] = bv[i];
        else st.b[4 * (tid & 15) + i][tid >> 4] = bv[i];
      }
      __syncthreads();
      any_step(st, acc);
    }
  }
  any_store(acc, y + t.lo * n + col0, n, rows, cols);
}

// contract, any shape: dw[g] = x[rows of g]^T dy[rows of g], x [m, k], dy [m, n], dw
// [g, k, n]; K is the group's rows. Block b: group b / (k_tiles col_tiles), its rows of
// dw 256 (b / col_tiles % k_tiles) on, columns 64 (b % col_tiles) on.
__global__ __launch_bounds__(THREADS) void contract_any_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ dy, int32_t groups, int64_t m,
    int64_t k, int64_t n, const int32_t* __restrict__ starts, int64_t k_tiles, int64_t col_tiles,
    uint16_t* __restrict__ dw) {
  __shared__ __align__(16) AnyStage st;
  if (!list_fits(starts, groups, -1, 0)) return;
  const int64_t per = k_tiles * col_tiles;
  const int32_t g = static_cast<int32_t>(blockIdx.x / per);
  const int64_t row0 = (blockIdx.x / col_tiles % k_tiles) * BM, col0 = (blockIdx.x % col_tiles) * ANY_BN;
  const int32_t rows = static_cast<int32_t>(k - row0 < BM ? k - row0 : BM);
  const int32_t cols = static_cast<int32_t>(n - col0 < ANY_BN ? n - col0 : ANY_BN);
  v16f acc[2][2];
#pragma unroll
  for (int p = 0; p < 2; ++p)
#pragma unroll
    for (int q = 0; q < 2; ++q)
#pragma unroll
      for (int j = 0; j < 16; ++j) acc[p][q][j] = 0.0f;
  const int64_t start = starts[g], end = starts[g + 1] < m ? starts[g + 1] : m;
  const int tid = threadIdx.x;
  for (int64_t i0 = start; i0 < end; i0 += ANY_BK) {
    uint16_t av[16], bv[4];
    // A(r, i) = x[i][r]: thread tid takes r = tid of the 16 rows i
#pragma unroll
    for (int i = 0; i < 16; ++i) av[i] = any_at(x + (i0 + i) * k + row0 + tid, i0 + i < end && tid < rows);
    // B(c, i) = dy[i][c]: row i0 + tid / 16, 4 consecutive columns
    const int64_t ir = i0 + (tid >> 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int32_t c = 4 * (tid & 15) + i;
      bv[i] = any_at(dy + ir * n + col0 + c, ir < end && c < cols);
    }
    __syncthreads();
    uint32_t packed[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) packed[i] = av[2 * i] | (static_cast<uint32_t>(av[2 * i + 1]) << 16);
    *reinterpret_cast<uint4*>(&st.a[tid][0]) = make_uint4(packed[0], packed[1], packed[2], packed[3]);
    *reinterpret_cast<uint4*>(&st.a[tid][8]) = make_uint4(packed[4], packed[5], packed[6], packed[7]);
#pragma unroll
    for (int i = 0; i < 4; ++i) st.b[4 * (tid & 15) + i][tid >> 4] = bv[i];
    __syncthreads();
    any_step(st, acc);
  }
  any_store(acc, dw + (static_cast<int64_t>(g) * k + row0) * n + col0, n, rows, cols);
}

// --- float32 --------------------------------------------------------------------------
//
// The compute format's GEMMs for a layer in float32 (the reference's ragged_dot and its
// transpose on float32 operands, float32 sums and outputs, grouped.py:90-146): the
// any-shape kernels' tiles and element loads, 4 bytes each, with v_mfma_f32_32x32x2_f32
// (float32 products, float32 sums). K goes 16 a step; in MFMA kk of a step, lane half h
// takes K 8 h + kk, so that a lane's 8 operands of a step are one 32-byte LDS row
// segment. Rows are 20 floats apart in LDS (16 and a pad).

constexpr int F32_PITCH = ANY_BK + 4;

struct F32Stage {
  float a[BM][F32_PITCH];
  float b[ANY_BN][F32_PITCH];
};

__device__ __forceinline__ void f32_step(const F32Stage& st, v16f acc[2][2]) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 31, h = lane >> 5;
  float a[2][8], b[2][8];
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const float4* ar = reinterpret_cast<const float4*>(&st.a[wave * 64 + p * 32 + r][8 * h]);
    const float4* br = reinterpret_cast<const float4*>(&st.b[p * 32 + r][8 * h]);
    const float4 a0 = ar[0], a1 = ar[1], b0 = br[0], b1 = br[1];
    a[p][0] = a0.x; a[p][1] = a0.y; a[p][2] = a0.z; a[p][3] = a0.w;
    a[p][4] = a1.x; a[p][5] = a1.y; a[p][6] = a1.z; a[p][7] = a1.w;
    b[p][0] = b0.x; b[p][1] = b0.y; b[p][2] = b0.z; b[p][3] = b0.w;
    b[p][4] = b1.x; b[p][5] = b1.y; b[p][6] = b1.z; b[p][7] = b1.w;
  }
#pragma unroll
  for (int kk = 0; kk < 8; ++kk)
#pragma unroll
    for (int p = 0; p < 2; ++p)
#pragma unroll
      for (int q = 0; q < 2; ++q)
        acc[p][q] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[p][kk], b[q][kk], acc[p][q], 0, 0, 0);
}

__device__ __forceinline__ void f32_store(const v16f acc[2][2], float* tile, int64_t ld,
                                          int32_t rows, int32_t cols) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int p = 0; p < 2; ++p)
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int32_t col = q * 32 + (lane & 31);
      if (col >= cols) continue;
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int32_t row = wave * 64 + p * 32 + 8 * (j >> 2) + 4 * (lane >> 5) + (j & 3);
        if (row < rows) tile[row * ld + col] = acc[p][q][j];
      }
    }
}

__device__ __forceinline__ float f32_at(const float* p, bool inside) { return inside ? *p : 0.0f; }

__device__ __forceinline__ void zero_acc2(v16f acc[2][2]) {
#pragma unroll
  for (int p = 0; p < 2; ++p)
#pragma unroll
    for (int q = 0; q < 2; ++q)
#pragma unroll
      for (int j = 0; j < 16; ++j) acc[p][q][j] = 0.0f;
}

// rows in float32: y[i] = x[i] w[g(i)] (w [g, k, n]; BKM: w [g, n, k] and x[i] w[g(i)]^T),
// as rows_any_kernel.
template <bool BKM>
__global__ __launch_bounds__(THREADS) void rows_f32_kernel(
    const float* __restrict__ x, const float* __restrict__ w, int32_t groups, int64_t m,
    int64_t n, int64_t k, const int32_t* __restrict__ starts, const Tile* __restrict__ tiles,
    int64_t col_tiles, float* __restrict__ y) {
  __shared__ __align__(16) F32Stage st;
  if (!list_fits(starts, groups, static_cast<int32_t>(m), static_cast<int32_t>(m))) return;
  const int64_t id = blockIdx.x / col_tiles;
  if (id >= starts[groups + 1]) return;
  const Tile t = tiles[id];
  const int64_t col0 = (blockIdx.x % col_tiles) * ANY_BN;
  const int64_t hi = t.hi < m ? t.hi : m;
  const int32_t rows = static_cast<int32_t>(hi - t.lo);
  if (rows <= 0) return;
  const int32_t cols = static_cast<int32_t>(n - col0 < ANY_BN ? n - col0 : ANY_BN);
  v16f acc[2][2];
  zero_acc2(acc);
  if (t.group < groups) {  // the rows past the groups: zeros
    const float* wg = w + static_cast<int64_t>(t.group) * n * k;
    const int tid = threadIdx.x, kk = tid & 15;
    for (int64_t k0 = 0; k0 < k; k0 += ANY_BK) {
      const bool kin = k0 + kk < k;
      float av[16], bv[4];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int32_t r = (tid >> 4) + 16 * i;
        av[i] = f32_at(x + (t.lo + r) * k + k0 + kk, kin && r < rows);
      }
      if constexpr (BKM) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int32_t c = (tid >> 4) + 16 * i;
          bv[i] = f32_at(wg + (col0 + c) * k + k0 + kk, kin && c < cols);
        }
      } else {
        const int64_t kr = k0 + (tid >> 4);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int32_t c = 4 * (tid & 15) + i;
          bv[i] = f32_at(wg + kr * n + col0 + c, kr < k && c < cols);
        }
      }
      __syncthreads();  // the last step's reads are done
#pragma unroll
      for (int i = 0; i < 16; ++i) st.a[(tid >> 4) + 16 * i][kk] = av[i];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if constexpr (BKM) st.b[(tid >> 4) + 16 * i][kk] = bv[i];
        else st.b[4 * (tid & 15) + i][tid >> 4] = bv[i];
      }
      __syncthreads();
      f32_step(st, acc);
    }
  }
  f32_store(acc, y + t.lo * n + col0, n, rows, cols);
}

// contract in float32: dw[g] = x[rows of g]^T dy[rows of g], as contract_any_kernel.
__global__ __launch_bounds__(THREADS) void contract_f32_kernel(
    const float* __restrict__ x, const float* __restrict__ dy, int32_t groups, int64_t m,
    int64_t k, int64_t n, const int32_t* __restrict__ starts, int64_t k_tiles, int64_t col_tiles,
    float* __restrict__ dw) {
  __shared__ __align__(16) F32Stage st;
  if (!list_fits(starts, groups, -1, 0)) return;
  const int64_t per = k_tiles * col_tiles;
  const int32_t g = static_cast<int32_t>(blockIdx.x / per);
  const int64_t row0 = (blockIdx.x / col_tiles % k_tiles) * BM, col0 = (blockIdx.x % col_tiles) * ANY_BN;
  const int32_t rows = static_cast<int32_t>(k - row0 < BM ? k - row0 : BM);
  const int32_t cols = static_cast<int32_t>(n - col0 < ANY_BN ? n - col0 : ANY_BN);
  v16f acc[2][2];
  zero_acc2(acc);
  const int64_t start = starts[g], end = starts[g + 1] < m ? starts[g + 1] : m;
  const int tid = threadIdx.x;
  for (int64_t i0 = start; i0 < end; i0 += ANY_BK) {
    float av[16], bv[4];
    // A(r, i) = x[i][r]: thread tid takes r = tid of the 16 rows i
#pragma unroll
    for (int i = 0; i < 16; ++i) av[i] = f32_at(x + (i0 + i) * k + row0 + tid, i0 + i < end && tid < rows);
    // B(c, i) = dy[i][c]: row i0 + tid / 16, 4 consecutive columns
    const int64_t ir = i0 + (tid >> 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int32_t c = 4 * (tid & 15) + i;
      bv[i] = f32_at(dy + ir * n + col0 + c, ir < end && c < cols);
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4; ++i)
      *reinterpret_cast<float4*>(&st.a[tid][4 * i]) =
          make_float4(av[4 * i], av[4 * i + 1], av[4 * i + 2], av[4 * i + 3]);
#pragma unroll
    for (int i = 0; i < 4; ++i) st.b[4 * (tid & 15) + i][tid >> 4] = bv[i];
    __syncthreads();
    f32_step(st, acc);
  }
  f32_store(acc, dw + (static_cast<int64_t>(g) * k + row0) * n + col0, n, rows, cols);
}

// Whether every offset a kernel forms into an operand of `rows` rows of `cols` elements
// (a tile's reads past it included) fits the 32-bit buffer offsets.
bool fits(int64_t rows, int64_t cols) { return (rows + BM) * (cols + BM) * 2 < (1LL << 31); }

template <bool BKM, bool TAIL>
int launch_rows(const Operand& A, const Operand& B, int32_t groups, int64_t m, int64_t n,
                int64_t k, const void* list, hipStream_t s, uint16_t* y) {
  const int64_t col_tiles = ceil_div(n, BN), slots = row_slots(groups, m, m);
  if (slots * col_tiles >= (1LL << 31)) return fail(BUX_E_ARGUMENT, "bux_bf16_grouped_rows: too many tiles");
  unsigned blocks = 0;
  if (int rc = grid_for(slots * col_tiles, &blocks)) return rc;
  if (int rc = allow_lds(rows_kernel<BKM, TAIL>, sizeof(Lds), "bf16 rows_kernel")) return rc;
  hipLaunchKernelGGL((rows_kernel<BKM, TAIL>), dim3(blocks), dim3(THREADS), sizeof(Lds), s, A, B,
                     groups, static_cast<int32_t>(m), static_cast<int32_t>(n),
                     static_cast<int32_t>(k), starts_in(list), tiles_in(list, groups),
                     static_cast<int32_t>(col_tiles), y);
  return launched("bf16 rows_kernel");
}

}  // namespace
}  // namespace bux

extern "C" size_t bux_bf16_grouped_rows_workspace_size(int32_t groups, int64_t m) {
  using namespace bux;
  return starts_bytes(groups) + static_cast<size_t>(row_slots(groups, m, m)) * sizeof(Tile);
}

extern "C" int bux_bf16_grouped_rows(const uint16_t* x, const uint16_t* w, int w_transposed,
                                     const int32_t* sizes, int32_t groups, int64_t m, int64_t n,
                                     int64_t k, uint16_t* y, void* workspace,
                                     size_t workspace_bytes, void* stream) {
  using namespace bux;
  clear_error();
  BUX_CHECK(groups >= 1 && groups <= MAX_GROUPS, "bux_bf16_grouped_rows: groups=%d outside [1, %d]",
            groups, MAX_GROUPS);
  BUX_CHECK(m >= 0 && n > 0 && k > 0, "bux_bf16_grouped_rows: bad shape m=%lld n=%lld k=%lld",
            (long long)m, (long long)n, (long long)k);
  BUX_CHECK(m < INT32_MAX, "bux_bf16_grouped_rows: m=%lld rows", (long long)m);
  BUX_CHECK(sizes && w && y && (m == 0 || x), "bux_bf16_grouped_rows: NULL buffer");
  const size_t need = bux_bf16_grouped_rows_workspace_size(groups, m);
  if (workspace == nullptr || workspace_bytes < need)
    return fail(BUX_E_WORKSPACE, "bux_bf16_grouped_rows: workspace of %zu bytes, %zu needed",
                workspace_bytes, need);
  if (m == 0) return BUX_OK;
  hipStream_t s = as_stream(stream);
  hipLaunchKernelGGL(prologue_kernel, dim3(1), dim3(THREADS), 0, s, sizes, groups, m,
                     row_slots(groups, m, m), 1, starts_in(workspace), tiles_in(workspace, groups),
                     header_in(workspace), m, nullptr);
  if (int rc = launched("prologue_kernel")) return rc;
  // n or k off 16-byte rows, or an operand past 32-bit offsets: the any-shape kernel
  if (n % 8 != 0 || k % 8 != 0 || !fits(m, k) || !(w_transposed ? fits(n, k) : fits(k, n))) {
    const int64_t col_tiles = ceil_div(n, ANY_BN), slots = row_slots(groups, m, m);
    const int64_t blocks = slots * col_tiles;
    BUX_CHECK(blocks < (1LL << 31), "bux_bf16_grouped_rows: too many tiles");
    if (w_transposed)
      hipLaunchKernelGGL(rows_any_kernel<true>, dim3(static_cast<unsigned>(blocks)), dim3(THREADS), 0, s,
                         x, w, groups, m, n, k, starts_in(workspace), tiles_in(workspace, groups),
                         col_tiles, y);
    else
      hipLaunchKernelGGL(rows_any_kernel<false>, dim3(static_cast<unsigned>(blocks)), dim3(THREADS), 0, s,
                         x, w, groups, m, n, k, starts_in(workspace), tiles_in(workspace, groups),
                         col_tiles, y);
    return launched("bf16 rows_any_kernel");
  }
  const Operand A{x, static_cast<int32_t>(k), static_cast<int32_t>(m * k * 2), 0};
  const Operand B{w, static_cast<int32_t>(w_transposed ? k : n), static_cast<int32_t>(n * k * 2), n * k};
  const bool tail = k % BK != 0;
  if (w_transposed)
    return tail ? launch_rows<true, true>(A, B, groups, m, n, k, workspace, s, y)
                : launch_rows<true, false>(A, B, groups, m, n, k, workspace, s, y);
  return tail ? launch_rows<false, true>(A, B, groups, m, n, k, workspace, s, y)
              : launch_rows<false, false>(A, B, groups, m, n, k, workspace, s, y);
}

extern "C" size_t bux_bf16_grouped_contract_workspace_size(int32_t groups) {
  using namespace bux;
  return starts_bytes(groups);  // the group starts alone: header, starts
}

extern "C" int bux_bf16_grouped_contract(const uint16_t* x, const uint16_t* dy, const int32_t* sizes,
                                         int32_t groups, int64_t m, int64_t k, int64_t n,
                                         uint16_t* dw, void* workspace, size_t workspace_bytes,
                                         void* stream) {
  using namespace bux;
  clear_error();
  BUX_CHECK(groups >= 1 && groups <= MAX_GROUPS,
            "bux_bf16_grouped_contract: groups=%d outside [1, %d]", groups, MAX_GROUPS);
  BUX_CHECK(m >= 0 && n > 0 && k > 0, "bux_bf16_grouped_contract: bad shape m=%lld k=%lld n=%lld",
            (long long)m, (long long)k, (long long)n);
  BUX_CHECK(m < INT32_MAX, "bux_bf16_grouped_contract: m=%lld rows", (long long)m);
  BUX_CHECK(sizes && dw && (m == 0 || (x && dy)), "bux_bf16_grouped_contract: NULL buffer");
  const size_t need = bux_bf16_grouped_contract_workspace_size(groups);
  if (workspace == nullptr || workspace_bytes < need)
    return fail(BUX_E_WORKSPACE, "bux_bf16_grouped_contract: workspace of %zu bytes, %zu needed",
                workspace_bytes, need);
  hipStream_t s = as_stream(stream);
  // the starts capped at the contract's K (m rows), as the rows GEMM caps them at its rows
  hipLaunchKernelGGL(prologue_kernel, dim3(1), dim3(THREADS), 0, s, sizes, groups, 0, 0, 1,
                     starts_in(workspace), nullptr, header_in(workspace), m, nullptr);
  if (int rc = launched("prologue_kernel")) return rc;
  if (n % 8 != 0 || k % 8 != 0 || !fits(m, k) || !fits(m, n)) {  // the any-shape kernel
    const int64_t k_tiles = ceil_div(k, BM), col_tiles = ceil_div(n, ANY_BN);
    const int64_t blocks = static_cast<int64_t>(groups) * k_tiles * col_tiles;
    BUX_CHECK(blocks < (1LL << 31), "bux_bf16_grouped_contract: too many tiles");
    hipLaunchKernelGGL(contract_any_kernel, dim3(static_cast<unsigned>(blocks)), dim3(THREADS), 0, s, x,
                       dy, groups, m, k, n, starts_in(workspace), k_tiles, col_tiles, dw);
    return launched("bf16 contract_any_kernel");
  }
  const int64_t d_tiles = ceil_div(k, BM), f_tiles = ceil_div(n, BN);
  const int64_t tiles = static_cast<int64_t>(groups) * d_tiles * f_tiles;
  BUX_CHECK(tiles < (1LL << 31), "bux_bf16_grouped_contract: too many tiles");
  // K is the rows: A(r, i) = x[i][r] and B(c, i) = dy[i][c], both MN-major.
  const Operand A{x, static_cast<int32_t>(k), static_cast<int32_t>(m * k * 2), 0};
  const Operand B{dy, static_cast<int32_t>(n), static_cast<int32_t>(m * n * 2), 0};
  unsigned blocks = 0;
  if (int rc = grid_for(tiles, &blocks)) return rc;
  if (int rc = allow_lds(contract_kernel, sizeof(Lds), "bf16 contract_kernel")) return rc;
  hipLaunchKernelGGL(contract_kernel, dim3(blocks), dim3(THREADS), sizeof(Lds), s, A, B, groups,
                     static_cast<int32_t>(k), static_cast<int32_t>(n), starts_in(workspace),
                     static_cast<int32_t>(d_tiles), static_cast<int32_t>(f_tiles), dw);
  return launched("bf16 contract_kernel");
}

extern "C" int bux_bf16_grouped_rows_f32(const float* x, const float* w, int w_transposed,
                                         const int32_t* sizes, int32_t groups, int64_t m,
                                         int64_t n, int64_t k, float* y, void* workspace,
                                         size_t workspace_bytes, void* stream) {
  using namespace bux;
  clear_error();
  BUX_CHECK(groups >= 1 && groups <= MAX_GROUPS,
            "bux_bf16_grouped_rows_f32: groups=%d outside [1, %d]", groups, MAX_GROUPS);
  BUX_CHECK(m >= 0 && n > 0 && k > 0, "bux_bf16_grouped_rows_f32: bad shape m=%lld n=%lld k=%lld",
            (long long)m, (long long)n, (long long)k);
  BUX_CHECK(m < INT32_MAX, "bux_bf16_grouped_rows_f32: m=%lld rows", (long long)m);
  BUX_CHECK(sizes && w && y && (m == 0 || x), "bux_bf16_grouped_rows_f32: NULL buffer");
  const size_t need = bux_bf16_grouped_rows_workspace_size(groups, m);
  if (workspace == nullptr || workspace_bytes < need)
    return fail(BUX_E_WORKSPACE, "bux_bf16_grouped_rows_f32: workspace of %zu bytes, %zu needed",
                workspace_bytes, need);
  if (m == 0) return BUX_OK;
  hipStream_t s = as_stream(stream);
  hipLaunchKernelGGL(prologue_kernel, dim3(1), dim3(THREADS), 0, s, sizes, groups, m,
                     row_slots(groups, m, m), 1, starts_in(workspace), tiles_in(workspace, groups),
                     header_in(workspace), m, nullptr);
  if (int rc = launched("prologue_kernel")) return rc;
  const int64_t col_tiles = ceil_div(n, ANY_BN), slots = row_slots(groups, m, m);
  const int64_t blocks = slots * col_tiles;
  BUX_CHECK(blocks < (1LL << 31), "bux_bf16_grouped_rows_f32: too many tiles");
  if (w_transposed)
    hipLaunchKernelGGL(rows_f32_kernel<true>, dim3(static_cast<unsigned>(blocks)), dim3(THREADS), 0,
                       s, x, w, groups, m, n, k, starts_in(workspace), tiles_in(workspace, groups),
                       col_tiles, y);
  else
    hipLaunchKernelGGL(rows_f32_kernel<false>, dim3(static_cast<unsigned>(blocks)), dim3(THREADS),
                       0, s, x, w, groups, m, n, k, starts_in(workspace),
                       tiles_in(workspace, groups), col_tiles, y);
  return launched("rows_f32_kernel");
}

extern "C" int bux_bf16_grouped_contract_f32(const float* x, const float* dy, const int32_t* sizes,
                                             int32_t groups, int64_t m, int64_t k, int64_t n,
                                             float* dw, void* workspace, size_t workspace_bytes,
                                             void* stream) {
  using namespace bux;
  clear_error();
  BUX_CHECK(groups >= 1 && groups <= MAX_GROUPS,
            "bux_bf16_grouped_contract_f32: groups=%d outside [1, %d]", groups, MAX_GROUPS);
  BUX_CHECK(m >= 0 && n > 0 && k > 0,
            "bux_bf16_grouped_contract_f32: bad shape m=%lld k=%lld n=%lld", (long long)m,
            (long long)k, (long long)n);
  BUX_CHECK(m < INT32_MAX, "bux_bf16_grouped_contract_f32: m=%lld rows", (long long)m);
  BUX_CHECK(sizes && dw && (m == 0 || (x && dy)), "bux_bf16_grouped_contract_f32: NULL buffer");
  const size_t need = bux_bf16_grouped_contract_workspace_size(groups);
  if (workspace == nullptr || workspace_bytes < need)
    return fail(BUX_E_WORKSPACE,
                "bux_bf16_grouped_contract_f32: workspace of %zu bytes, %zu needed",
                workspace_bytes, need);
  hipStream_t s = as_stream(stream);
  hipLaunchKernelGGL(prologue_kernel, dim3(1), dim3(THREADS), 0, s, sizes, groups, 0, 0, 1,
                     starts_in(workspace), nullptr, header_in(workspace), m, nullptr);
  if (int rc = launched("prologue_kernel")) return rc;
  const int64_t k_tiles = ceil_div(k, BM), col_tiles = ceil_div(n, ANY_BN);
  const int64_t blocks = static_cast<int64_t>(groups) * k_tiles * col_tiles;
  BUX_CHECK(blocks < (1LL << 31), "bux_bf16_grouped_contract_f32: too many tiles");
  hipLaunchKernelGGL(contract_f32_kernel, dim3(static_cast<unsigned>(blocks)), dim3(THREADS), 0, s,
                     x, dy, groups, m, k, n, starts_in(workspace), k_tiles, col_tiles, dw);
  return launched("contract_f32_kernel");
}
