// Grouped MXFP8 GEMMs on CDNA4's block-scaled MFMA (v_mfma_scale_f32_32x32x64_f8f6f4):
// E4M3 x E4M3 with an E8M0 scale per 32 of what they contract, float32 accumulation.
//
//   rows      y[i] = a[i] b[g(i)]^T for each group g's rows i      grouped_mxfp8.py:116-154
//             (fprop x W and dgrad dy W^T); rows past sum(sizes) are 0.
//   contract  dw[g] = a[:, rows of g] b[:, rows of g]^T           grouped_mxfp8.py:185-210
//             (wgrad); a's bytes outside the group's rows count as 0 (the reference's
//             _edges, grouped_mxfp8.py:240-256).
//
// Operands arrive in the tiled MXFP8 layout that the quantizer writes: for a matrix of
// R rows and K bytes a row (K a whole number of 128s), codes [K/64][R][64] and scale
// bytes [K/128][R][4]. One step of 64 bytes of K of 256 consecutive rows is then 16 KiB
// in one run and its scales 1 KiB in one run: the loads that feed the MFMAs move whole
// cache lines. (From row-major operands, measured on the MI355X, the same direct loads
// of 16 rows x 64 bytes reach half that bandwidth, and scale words of 4 bytes a row
// under 1 byte a clock a CU.) One mainloop serves both GEMMs:
// C[r][c] = sum_k A[r][k] B[c][k] over a tile of 256 x 256 outputs.
//
// Workgroup: 4 waves (2 x 2), each 128 x 128 outputs as 4 x 4 MFMAs of 32 x 32: 256
// accumulator registers, one wave a SIMD. K goes in steps of 64 bytes (one MFMA deep).
// Each step's A and B tiles (16 KiB each) and scale words go from global memory straight
// into LDS (buffer_load ... lds, no registers on the way) in a ring of 4 stages, issued
// 4 steps ahead of their MFMAs. A wave keeps two sets of operand registers: while the
// MFMAs of step k run on one, its LDS reads of step k + 1 fill the other. The
// workgroup's one barrier a step comes first (after it step k + 1's stage is whole and
// every wave has read step k's), then the 16 MFMAs, each followed by a slice of the
// memory work (one of step k + 4's loads, a part of step k + 1's reads): a wave issues in
// order, so a load that waits for the memory pipe waits while the MFMA before it runs.
//
// MFMA lane layout (32 x 32 x 64), measured on the MI355X: lane l holds row l % 32 of
// its first operand (column l % 32 of its second); lane half h = l / 32 holds 16 bytes
// of each of the two blocks of 32 in K, block 0 in register bytes 0..15 and block 1 in
// bytes 16..31, and its scale operand (the register's low byte) scales block h of its
// row. A and B load alike, so the order of K inside a block is immaterial. The 16
// accumulator registers of lane l are rows 8 (j / 4) + 4 (l / 32) + j % 4 of the first
// operand, column l % 32 of the second: with B's rows first and A's second, a lane
// holds 4 runs of 4 consecutive output columns of one output row.
//
// Ragged rows: a tile list like the reference's tiles_of (grouped_mxfp8.py:157-182),
// built on the device from `sizes` so the host never synchronises; but a group's tiles
// start at its first row, so no tile computes two groups (a tile's rows past its group
// are computed from whatever rows follow and not stored). The rows past the groups are
// a group of their own that stores 0. Workgroups are renumbered so that each XCD (a
// workgroup's id modulo 8) takes a contiguous run of tiles, which share A's rows and a
// group's B in its L2.

#include <mutex>

#include "glu.h"
#include "tiles.h"

namespace bux {
namespace {

typedef int v8i __attribute__((ext_vector_type(8)));

constexpr int BK = 64;   // bytes of K a step
constexpr int LOADS_A_STEP = 10;  // direct loads a wave issues a step

// --- the pipeline --------------------------------------------------------------------

// An operand in the tiled layout: row r's byte k at values[((k / 64) rows + r) 64 +
// k % 64], the scale byte of its block b (of 32) at scales[((b / 4) rows + r) 4 + b % 4].
// Its bytes may pass 4 GiB: the loads address one K chunk at a time (chunk_at), so only
// a chunk's rows x 64 bytes must fit 32 bits (the host checks the rows).
struct Operand {
  const uint8_t* values;
  const uint8_t* scales;
  int32_t k;     // bytes of K a row: whole 128s
  int32_t rows;  // rows there are
};

// One K step's operands in LDS: 256 rows of A and of B, 64 bytes each, and their rows'
// scale words of the 128 bytes of K the step is in.
struct Stage {
  uint8_t a[BM * BK];
  uint8_t b[BN * BK];
  uint32_t as[BM];
  uint32_t bs[BN];
};
struct Lds {
  Stage st[STAGES];
};

// Where a 64-byte LDS row's 16-byte chunk c sits: c ^ swizzle(row). gfx950's LDS serves
// ds_read_b128 16 lanes at a time over 64 banks of 4 bytes; those 16 lanes read one
// chunk of 16 consecutive rows. Rows r .. r + 3 lie 64 bytes apart and (r / 4) % 4
// spreads each such four over the 4 chunk places: 16 places of 16 bytes in 256, every
// bank once. Rows 16 apart share a swizzle, so blocks of 16 or 32 rows are copies of
// one another at fixed offsets.
__device__ __forceinline__ int swizzle(int row) { return (row >> 2) & 3; }

// What a wave w loads of one operand's 256 rows from `row0` on: rows [64 w, 64 w + 64)
// of the tile, as 4 slices of 16 rows x 64 bytes (each 1 KiB in one run; a lane takes
// the 16-byte chunk that belongs in its swizzled place) and the scale words of those
// rows. Slices are 1 KiB apart in memory and in LDS alike (rows 16 apart share a
// swizzle), so one lane offset serves them all, the scalar offset adding 1 KiB a slice.
// Rows past the operand read 0 (or, in a narrow operand's chunk, the next chunk's rows);
// their outputs are never stored.
struct Loads {
  const uint8_t* values;              // the operand's codes and scale words
  const uint8_t* scales;
  i32x4 rv, rs;                       // resources over the whole operand (narrow)
  int32_t voff, soff;                 // this lane's
  int32_t chunk_stride, word_stride;  // a K chunk's bytes (64 / 128 bytes of K): rows x 64, rows x 4
};

// The buffer resource of K chunk c of an operand and the scalar offset into it: a wide
// operand's (W) base moves a chunk at a time in 64 bits and the resource holds that
// chunk's rows alone, so that no offset passes 32 bits whatever the operand's size (a
// resource over the whole operand holds at most 4 GiB, and a scalar offset of c x
// stride 2 GiB); a narrow one (under 2 GiB with a tile's reads past its rows) takes
// its one resource and the offset c x stride, which costs the K loop no scalar
// arithmetic (wide: 3% slower at c3).
template <bool W>
__device__ __forceinline__ i32x4 chunk_at(const uint8_t* base, const i32x4& whole, int32_t c,
                                          int32_t stride, int32_t& soff) {
  if constexpr (W) {
    soff = 0;
    return resource(base + static_cast<int64_t>(c) * stride, stride);
  } else {
    soff = c * stride;
    return whole;
  }
}

__device__ __forceinline__ Loads loads_for(const Operand& op, int32_t row0) {
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  Loads ld;
  ld.values = op.values;
  ld.scales = op.scales;
  ld.rv = resource(op.values, static_cast<int64_t>(op.k) * op.rows);
  ld.rs = resource(op.scales, static_cast<int64_t>(op.k / 32) * op.rows);
  const int r = w * 64 + (l >> 2);
  ld.voff = (row0 + r) * 64 + 16 * ((l & 3) ^ swizzle(r));
  ld.soff = (row0 + w * 64 + l) * 4;
  ld.chunk_stride = op.rows * 64;
  ld.word_stride = op.rows * 4;
  return ld;
}

// Direct load Q (0..9) of K step ks into stage `st`: Q < 8 a 16-row slice of A's (even
// Q) or B's (odd Q) rows of this wave; 8 and 9 the scale words of its A and B rows. In a
// half tile (H) the A rows of waves 2 and 3 (128 .. 255) are not loaded: each of those
// waves loads its A scale words again in their place (4 bytes a lane, the same bytes to
// the same place as load 8), so that every wave issues 10 loads a step whatever the
// tile, and the waits count them alike.
template <int Q, bool H, bool W>
__device__ __forceinline__ void issue_one(const Loads& la, const Loads& lb, int32_t ks,
                                          uint32_t lds0, int st) {
  const uint32_t w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t at = lds0 + static_cast<uint32_t>(st * sizeof(Stage));
  if (Q < 8) {
    constexpr int i = Q >> 1;
    const uint32_t slice = w * 4096 + i * 1024;
    int32_t so;
    if ((Q & 1) == 0 && H && w >= 2) {
      const i32x4 r = chunk_at<W>(la.scales, la.rs, ks >> 1, la.word_stride, so);
      load_lds4(r, at + offsetof(Stage, as) + w * 256, la.soff, so);
    } else if ((Q & 1) == 0) {
      const i32x4 r = chunk_at<W>(la.values, la.rv, ks, la.chunk_stride, so);
      load_lds16(r, at + offsetof(Stage, a) + slice, la.voff, so + i * 1024);
    } else {
      const i32x4 r = chunk_at<W>(lb.values, lb.rv, ks, lb.chunk_stride, so);
      load_lds16(r, at + offsetof(Stage, b) + slice, lb.voff, so + i * 1024);
    }
  } else if (Q == 8) {
    int32_t so;
    const i32x4 r = chunk_at<W>(la.scales, la.rs, ks >> 1, la.word_stride, so);
    load_lds4(r, at + offsetof(Stage, as) + w * 256, la.soff, so);
  } else {
    int32_t so;
    const i32x4 r = chunk_at<W>(lb.scales, lb.rs, ks >> 1, lb.word_stride, so);
    load_lds4(r, at + offsetof(Stage, bs) + w * 256, lb.soff, so);
  }
}

template <int Q, bool H, bool W>
__device__ __forceinline__ void issue_from(const Loads& la, const Loads& lb, int32_t ks,
                                           uint32_t lds0, int st) {
  issue_one<Q, H, W>(la, lb, ks, lds0, st);
  if constexpr (Q + 1 < LOADS_A_STEP) issue_from<Q + 1, H, W>(la, lb, ks, lds0, st);
}

// All of a wave's direct loads of K step ks into stage `st`, of a whole or a half tile.
template <bool W>
__device__ __forceinline__ void issue(const Loads& la, const Loads& lb, int32_t ks, uint32_t lds0,
                                      int st, bool half) {
  if (half) issue_from<0, true, W>(la, lb, ks, lds0, st);
  else issue_from<0, false, W>(la, lb, ks, lds0, st);
}

// Waits until at most `steps` steps' loads of this wave are in flight. A wave's loads
// complete in the order they were issued, so a step is complete once no more than the
// loads issued after it are outstanding; stores of its own in flight only make the
// count stricter (the epilogue keeps them out of the way: see run_tiles).
__device__ __forceinline__ void wait_loads(int32_t steps) {
  if (steps >= 3) asm volatile("s_waitcnt vmcnt(30)" ::: "memory");
  else if (steps == 2) asm volatile("s_waitcnt vmcnt(20)" ::: "memory");
  else if (steps == 1) asm volatile("s_waitcnt vmcnt(10)" ::: "memory");
  else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// A wave's operands of one step: 4 blocks of 32 rows of A and of B, and their scales.
struct Frag {
  v8i a[4], b[4];
  int sa[4], sb[4];
};

// Zeroes the bytes of A's operand registers of K step ks whose K lies outside [lo, hi)
// (a wgrad's edge steps): lane half h holds K bytes 16 h .. 16 h + 15 of the step in
// dwords 0-3 and 32 + 16 h .. in dwords 4-7, the same for every row it holds.
__device__ __forceinline__ void mask_frag(Frag& f, int32_t ks, int32_t lo, int32_t hi) {
  const int h = (threadIdx.x & 63) >> 5;
  uint32_t keep[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int32_t k0 = ks * BK + (j < 4 ? 16 * h + 4 * j : 32 + 16 * h + 4 * (j - 4));
    uint32_t m = 0;
#pragma unroll
    for (int b = 0; b < 4; ++b)
      if (k0 + b >= lo && k0 + b < hi) m |= 0xffu << (8 * b);
    keep[j] = m;
  }
#pragma unroll
  for (int p = 0; p < 4; ++p)
#pragma unroll
    for (int j = 0; j < 8; ++j) f.a[p][j] &= keep[j];
}

// This lane's byte offsets in a stage, computed once: its two 16-byte chunks of A's
// (B's) 32-row block 0 (K chunks h and 2 + h of the step for lane half h, the MFMA's two
// blocks of 32), and its scale byte of block 0 in an even step. Block p is 2048 bytes
// further (128 for the scale), an odd step's scale 2 bytes.
// A whole tile's waves are 2 x 2 (each 128 rows of A, 128 of B); a half tile's 1 x 4
// (each the tile's 128 rows of A, 64 of B).
struct Lanes {
  int32_t a_lo, a_hi, b_lo, b_hi, sa, sb;
};
template <bool H>
__device__ __forceinline__ Lanes lanes_of() {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int half = lane >> 5, row = lane & 31, sw = swizzle(row);
  const int ra = (H ? 0 : (wave >> 1) * 128) + row;
  const int rb = (H ? wave * 64 : (wave & 1) * 128) + row;
  const int lo = (half ^ sw) << 4, hi = ((2 + half) ^ sw) << 4;
  return Lanes{ra * BK + lo, ra * BK + hi, rb * BK + lo, rb * BK + hi, ra * 4 + half, rb * 4 + half};
}

__device__ __forceinline__ v8i chunks(const uint8_t* lo, const uint8_t* hi) {
  const uint4 x = *reinterpret_cast<const uint4*>(lo);
  const uint4 y = *reinterpret_cast<const uint4*>(hi);
  v8i v;
  v[0] = x.x; v[1] = x.y; v[2] = x.z; v[3] = x.w;
  v[4] = y.x; v[5] = y.y; v[6] = y.z; v[7] = y.w;
  return v;
}

// Block p (0..3) of 32 rows of A's (B's) part of a wave's operands of step ks from
// stage `st`, and its scales. The scale bytes are read one byte each (ds_read_u8), so
// no instruction touches them before the MFMAs that take them: a read whose value is
// used at once exposes the LDS latency to the whole wave.
__device__ __forceinline__ void read_a(Frag& f, const Lds& lds, const Lanes& ln, int st,
                                       int32_t ks, int p) {
  const uint8_t* t = lds.st[st].a + p * 2048;
  f.a[p] = chunks(t + ln.a_lo, t + ln.a_hi);
  f.sa[p] = (reinterpret_cast<const uint8_t*>(lds.st[st].as) + ((ks & 1) << 1) + p * 128)[ln.sa];
}
__device__ __forceinline__ void read_b(Frag& f, const Lds& lds, const Lanes& ln, int st,
                                       int32_t ks, int p) {
  const uint8_t* t = lds.st[st].b + p * 2048;
  f.b[p] = chunks(t + ln.b_lo, t + ln.b_hi);
  f.sb[p] = (reinterpret_cast<const uint8_t*>(lds.st[st].bs) + ((ks & 1) << 1) + p * 128)[ln.sb];
}

// A step's operands: A's 4 blocks and B's 4 (a half tile's wave: B's 2).
template <bool H>
__device__ __forceinline__ void read_frag(Frag& f, const Lds& lds, const Lanes& ln, int st,
                                          int32_t ks) {
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    read_a(f, lds, ln, st, ks, p);
    if (!H || p < 2) read_b(f, lds, ln, st, ks, p);
  }
}

// The 16 MFMAs of one step on `cur`, MFMA q taking A's block q / 4 and B's block q % 4,
// each followed by a slice of the memory work: with LOAD, the next loads (step ks_load
// into stage st_load), one after each of the first 10; with READ, the next step's blocks
// into `nxt` in the order its MFMAs take them (a0 b0, b1, b2, b3, then a1, a2, a3 four
// MFMAs apart), so that each lands a dozen MFMAs before its first use. The MFMA goes
// first: a load that waits to issue (the memory pipe full) then waits while the MFMA
// runs, rather than holding the MFMA back.
template <bool LOAD, bool READ, bool W>
__device__ __forceinline__ void step(const Frag& cur, Frag& nxt, const Loads& la, const Loads& lb,
                                     const Lds& lds, uint32_t lds0, const Lanes& ln,
                                     int32_t ks_load, int st_load, int32_t ks_next, int st_next,
                                     v16f acc[4][4]) {
#pragma unroll
  for (int q = 0; q < 16; ++q) {
    const int i = q >> 2, j = q & 3;
    acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(cur.b[j], cur.a[i], acc[i][j], 0,
                                                               0, 0, cur.sb[j], 0, cur.sa[i]);
    __builtin_amdgcn_sched_barrier(0);
    if (LOAD) {
      switch (q) {
        case 0: issue_one<0, false, W>(la, lb, ks_load, lds0, st_load); break;
        case 1: issue_one<1, false, W>(la, lb, ks_load, lds0, st_load); break;
        case 2: issue_one<2, false, W>(la, lb, ks_load, lds0, st_load); break;
        case 3: issue_one<3, false, W>(la, lb, ks_load, lds0, st_load); break;
        case 4: issue_one<4, false, W>(la, lb, ks_load, lds0, st_load); break;
        case 5: issue_one<5, false, W>(la, lb, ks_load, lds0, st_load); break;
        case 6: issue_one<6, false, W>(la, lb, ks_load, lds0, st_load); break;
        case 7: issue_one<7, false, W>(la, lb, ks_load, lds0, st_load); break;
        case 8: issue_one<8, false, W>(la, lb, ks_load, lds0, st_load); break;
        case 9: issue_one<9, false, W>(la, lb, ks_load, lds0, st_load); break;
        default: break;
      }
    }
    if (READ) {
      if (q == 0) read_a(nxt, lds, ln, st_next, ks_next, 0);
      if (q < 4) read_b(nxt, lds, ln, st_next, ks_next, q);
      if (q == 4 || q == 8 || q == 12) read_a(nxt, lds, ln, st_next, ks_next, q >> 2);
    }
    __builtin_amdgcn_sched_barrier(0);
  }
}

// A half tile's step: each wave's 128 x 64 outputs, 8 MFMAs (MFMA q taking A's block
// q / 2 and B's block q % 2), with the same 10 loads (one after each of the first 7
// MFMAs, three after the last) and the next step's 6 blocks read in the order its
// MFMAs take them (a0 b0, b1, a1, a2, a3).
template <bool LOAD, bool READ, bool W>
__device__ __forceinline__ void step_half(const Frag& cur, Frag& nxt, const Loads& la,
                                          const Loads& lb, const Lds& lds, uint32_t lds0,
                                          const Lanes& ln, int32_t ks_load, int st_load,
                                          int32_t ks_next, int st_next, v16f acc[4][4]) {
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const int i = q >> 1, j = q & 1;
    acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(cur.b[j], cur.a[i], acc[i][j], 0,
                                                               0, 0, cur.sb[j], 0, cur.sa[i]);
    __builtin_amdgcn_sched_barrier(0);
    if (LOAD) {
      switch (q) {
        case 0: issue_one<0, true, W>(la, lb, ks_load, lds0, st_load); break;
        case 1: issue_one<1, true, W>(la, lb, ks_load, lds0, st_load); break;
        case 2: issue_one<2, true, W>(la, lb, ks_load, lds0, st_load); break;
        case 3: issue_one<3, true, W>(la, lb, ks_load, lds0, st_load); break;
        case 4: issue_one<4, true, W>(la, lb, ks_load, lds0, st_load); break;
        case 5: issue_one<5, true, W>(la, lb, ks_load, lds0, st_load); break;
        case 6: issue_one<6, true, W>(la, lb, ks_load, lds0, st_load); break;
        default:
          issue_one<7, true, W>(la, lb, ks_load, lds0, st_load);
          issue_one<8, true, W>(la, lb, ks_load, lds0, st_load);
          issue_one<9, true, W>(la, lb, ks_load, lds0, st_load);
          break;
      }
    }
    if (READ) {
      if (q == 0) read_a(nxt, lds, ln, st_next, ks_next, 0);
      if (q < 2) read_b(nxt, lds, ln, st_next, ks_next, q);
      if (q == 2 || q == 4 || q == 6) read_a(nxt, lds, ln, st_next, ks_next, q >> 1);
    }
    __builtin_amdgcn_sched_barrier(0);
  }
}

// --- the epilogue ----------------------------------------------------------------------

// Output stores are non-temporal: the tile is written once and read by another kernel,
// and a whole round of tiles' outputs (4 MiB an XCD in bfloat16) passing through the
// XCD's 4 MiB L2 would evict the operands the other CUs are about to reuse.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
constexpr int NT = 2;  // a buffer store's cache policy: non-temporal
__device__ __forceinline__ void stream16(void* at, uint4 v) {
  __builtin_nontemporal_store(u32x4{v.x, v.y, v.z, v.w}, reinterpret_cast<u32x4*>(at));
}
__device__ __forceinline__ void stream8(void* at, uint32_t x, uint32_t y) {
  __builtin_nontemporal_store(u32x2{x, y}, reinterpret_cast<u32x2*>(at));
}

// float32 (for tests), by every wave, straight from the accumulators: lane l holds row
// l % 32 of each 32-row block and, in register run g, columns 8 g + 4 (l / 32) .. + 3 of
// each 32-column block. The tile's rows [0, rows) and columns [0, cols) are stored (cols
// a multiple of 4), at row pitch ld, from its corner.
__device__ void store_f32(const v16f acc[4][4], float* tile, int32_t ld, int32_t rows, int32_t cols) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int32_t row = wm * 128 + i * 32 + (lane & 31);
    if (row >= rows) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int32_t col = wn * 128 + j * 32 + 8 * g + 4 * (lane >> 5);
        const v16f& a = acc[i][j];
        if (col < cols)
          stream16(tile + row * ld + col,
                   make_uint4(__float_as_uint(a[4 * g]), __float_as_uint(a[4 * g + 1]),
                              __float_as_uint(a[4 * g + 2]), __float_as_uint(a[4 * g + 3])));
      }
  }
}

// bfloat16 through one stage of LDS, in 4 rounds of 32 rows: each wave puts its block of
// 32 x 128 outputs in a region of its own (rows 272 bytes apart, 256 and a pad, so that
// the 16 lanes that read a row and rows 4 apart use different banks; the four regions
// fill the stage), reads it back 16 bytes a lane, 16 lanes a row, and stores 4 runs of
// 256 bytes an instruction. No other wave touches the region: no workgroup barrier.
// Every LDS address is a lane's base plus a constant.
constexpr int PITCH = 272;
static_assert(4 * 32 * PITCH == sizeof(Stage), "the epilogue's regions fill a stage");

// With LO, only the rows from row_lo on are stored.
// The accumulators of a 32 x 32 block as bfloat16 pairs: run g's columns 0-1 and 2-3
// (v_cvt_pk_bf16_f32: two floats to two bfloat16, nearest even).
struct FromAcc {
  const v16f (*acc)[4];
  __device__ __forceinline__ uint2 operator()(int i, int j, int g) const {
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    const v16f& a = acc[i][j];
    const bf16x2 lo = __builtin_convertvector((f32x2{a[4 * g], a[4 * g + 1]}), bf16x2);
    const bf16x2 hi = __builtin_convertvector((f32x2{a[4 * g + 2], a[4 * g + 3]}), bf16x2);
    return make_uint2(__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi));
  }
};

// `pairs(i, j, g)`: the bfloat16 pairs of block (i, j), register run g. With LO, only
// the rows from row_lo on are stored.
template <bool LO = false, typename Pairs>
__device__ void store_bf16(const Pairs& pairs, uint16_t* tile, int32_t ld, int32_t rows,
                           int32_t cols, Stage& stage, int32_t row_lo = 0) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  uint8_t* region = reinterpret_cast<uint8_t*>(&stage) + wave * 32 * PITCH;
  // Lane l writes row l % 32 of the block, its 4 columns of each 8 at byte 8 (l / 32).
  uint8_t* mine = region + (lane & 31) * PITCH + 8 * (lane >> 5);
  // ... and reads back chunk l % 16 (8 columns) of row l / 16 (of 4).
  const int cc = lane & 15;
  const uint8_t* from = region + (lane >> 4) * PITCH + cc * 16;
  const int32_t col = wn * 128 + 8 * cc;
  uint16_t* out = tile + (wm * 128 + (lane >> 4)) * ld + col;
  // A whole tile (the common case) stores without bounds checks, through a buffer
  // resource from its corner: the lane's offset, a scalar one a row of stores.
  const bool whole = rows >= BM && cols >= BN && (!LO || row_lo <= 0);
  const __amdgpu_buffer_rsrc_t rsrc =
      __builtin_amdgcn_make_buffer_rsrc(tile, 0, 0x7fffffff, 0x00020000);
  const int32_t lane_off = ((wm * 128 + (lane >> 4)) * ld + col) * 2;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g) *reinterpret_cast<uint2*>(mine + (j * 4 + g) * 16) = pairs(i, j, g);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_wave_barrier();
    // All 8 reads of the round go out before its first store.
    uint4 v[8];
#pragma unroll
    for (int it = 0; it < 8; ++it) v[it] = *reinterpret_cast<const uint4*>(from + it * 4 * PITCH);
    if (whole) {
#pragma unroll
      for (int it = 0; it < 8; ++it)
        __builtin_amdgcn_raw_buffer_store_b128(u32x4{v[it].x, v[it].y, v[it].z, v[it].w}, rsrc,
                                               lane_off, (i * 32 + it * 4) * ld * 2, NT);
    } else if (col < cols) {
#pragma unroll
      for (int it = 0; it < 8; ++it) {
        const int32_t row = wm * 128 + i * 32 + it * 4 + (lane >> 4);
        if (row < rows && (!LO || row >= row_lo)) {
          uint16_t* at = out + (i * 32 + it * 4) * ld;
          if (col + 8 <= cols) stream16(at, v[it]);
          else stream8(at, v[it].x, v[it].y);  // cols % 4 == 0
        }
      }
    }
    // The reads are done before the next round's writes.
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_wave_barrier();
  }
}

__device__ __forceinline__ void store_tile(const v16f acc[4][4], uint16_t* tile, int32_t ld,
                                           int32_t rows, int32_t cols, Stage& stage) {
  store_bf16(FromAcc{acc}, tile, ld, rows, cols, stage);
}
__device__ __forceinline__ void store_tile(const v16f acc[4][4], float* tile, int32_t ld,
                                           int32_t rows, int32_t cols, Stage&) {
  store_f32(acc, tile, ld, rows, cols);
}

// A half tile's outputs, each wave's 128 rows x 64 columns (columns 64 w on; accumulator
// blocks [i][0..1]). bfloat16 through the wave's region of the stage as store_bf16 does,
// read back 16 bytes a lane, 8 lanes a row, in 4 rounds of 32 rows.
__device__ void store_tile_half(const v16f acc[4][4], uint16_t* tile, int32_t ld, int32_t rows,
                                int32_t cols, Stage& stage) {
  const FromAcc pairs{acc};
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  uint8_t* region = reinterpret_cast<uint8_t*>(&stage) + wave * 32 * PITCH;
  uint8_t* mine = region + (lane & 31) * PITCH + 8 * (lane >> 5);
  const int cc = lane & 7;
  const uint8_t* from = region + (lane >> 3) * PITCH + cc * 16;
  const int32_t col = wave * 64 + 8 * cc;
  uint16_t* out = tile + (lane >> 3) * ld + col;
  const bool whole = rows >= BM / 2 && cols >= BN;
  const __amdgpu_buffer_rsrc_t rsrc =
      __builtin_amdgcn_make_buffer_rsrc(tile, 0, 0x7fffffff, 0x00020000);
  const int32_t lane_off = ((lane >> 3) * ld + col) * 2;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g) *reinterpret_cast<uint2*>(mine + (j * 4 + g) * 16) = pairs(i, j, g);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_wave_barrier();
    uint4 v[4];
#pragma unroll
    for (int it = 0; it < 4; ++it) v[it] = *reinterpret_cast<const uint4*>(from + it * 8 * PITCH);
    if (whole) {
#pragma unroll
      for (int it = 0; it < 4; ++it)
        __builtin_amdgcn_raw_buffer_store_b128(u32x4{v[it].x, v[it].y, v[it].z, v[it].w}, rsrc,
                                               lane_off, (i * 32 + it * 8) * ld * 2, NT);
    } else if (col < cols) {
#pragma unroll
      for (int it = 0; it < 4; ++it) {
        const int32_t row = i * 32 + it * 8 + (lane >> 3);
        if (row < rows) {
          uint16_t* at = out + (i * 32 + it * 8) * ld;
          if (col + 8 <= cols) stream16(at, v[it]);
          else stream8(at, v[it].x, v[it].y);  // cols % 4 == 0
        }
      }
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_wave_barrier();
  }
}
// float32 (for tests), straight from the accumulators as store_f32.
__device__ void store_tile_half(const v16f acc[4][4], float* tile, int32_t ld, int32_t rows,
                                int32_t cols, Stage&) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int32_t row = i * 32 + (lane & 31);
    if (row >= rows) continue;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int32_t col = wave * 64 + j * 32 + 8 * g + 4 * (lane >> 5);
        const v16f& a = acc[i][j];
        if (col < cols)
          stream16(tile + row * ld + col,
                   make_uint4(__float_as_uint(a[4 * g]), __float_as_uint(a[4 * g + 1]),
                              __float_as_uint(a[4 * g + 2]), __float_as_uint(a[4 * g + 3])));
      }
  }
}

// bfloat16 of a tile that stores every row and column (PH: a half tile's 128 rows),
// through the wave's region of the stage as pairs of 32 x 32 accumulator blocks: a whole
// tile's wave holds 8 pairs (block row p / 2, its 64 columns from 64 (p % 2)), a half
// tile's 4 (block row p, the wave's 64 columns). Two buffers of 32 rows 136 bytes apart
// (128 bytes of a pair's row and 8 of pad: the 32 rows of a lane half start on distinct
// banks) fill the region; each lane writes its row's 4 runs of 4 columns of both blocks
// (8 bytes each), reads back 16 bytes of a row, 8 lanes a row (as two 8-byte reads: the
// rows are 8-byte aligned), and a store writes 8 whole rows of 128 bytes. Pair p + 1 is
// converted and written while pair p's reads are in flight, and pair p's stores go out
// after them: the wave's LDS operations run in order, so a read after a write sees it and
// a write after a read (into the buffer the pair before last used) leaves it alone.
constexpr int PAIR_PITCH = 136;
constexpr int PAIR_BUF = 32 * PAIR_PITCH;
static_assert(2 * PAIR_BUF == 32 * PITCH, "a wave's two pair buffers fill its region of the stage");

template <bool PH>
__device__ void store_pairs(const v16f acc[4][4], uint16_t* tile, int32_t ld, Stage& stage) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  uint8_t* region = reinterpret_cast<uint8_t*>(&stage) + wave * 2 * PAIR_BUF;
  uint8_t* mine = region + (lane & 31) * PAIR_PITCH + 8 * (lane >> 5);
  const uint8_t* from = region + (lane >> 3) * PAIR_PITCH + (lane & 7) * 16;
  const __amdgpu_buffer_rsrc_t rsrc =
      __builtin_amdgcn_make_buffer_rsrc(tile, 0, 0x7fffffff, 0x00020000);
  const int32_t lane_off = ((lane >> 3) * ld + 8 * (lane & 7)) * 2;
  const FromAcc pairs{acc};
  constexpr int M = PH ? 4 : 8;
  auto write = [&](int p) {
    const int i = PH ? p : p >> 1, j0 = PH ? 0 : (p & 1) * 2;
    uint8_t* at = mine + (p & 1) * PAIR_BUF;
#pragma unroll
    for (int jb = 0; jb < 2; ++jb)
#pragma unroll
      for (int g = 0; g < 4; ++g) *reinterpret_cast<uint2*>(at + jb * 64 + g * 16) = pairs(i, j0 + jb, g);
  };
  write(0);
#pragma unroll
  for (int p = 0; p < M; ++p) {
    const uint8_t* at = from + (p & 1) * PAIR_BUF;
    uint2 v[8];
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      v[2 * it] = *reinterpret_cast<const uint2*>(at + it * 8 * PAIR_PITCH);
      v[2 * it + 1] = *reinterpret_cast<const uint2*>(at + it * 8 * PAIR_PITCH + 8);
    }
    if (p + 1 < M) write(p + 1);
    const int32_t row0 = PH ? p * 32 : (wave >> 1) * 128 + (p >> 1) * 32;
    const int32_t col0 = PH ? wave * 64 : (wave & 1) * 128 + (p & 1) * 64;
    const int32_t corner = (row0 * ld + col0) * 2;
#pragma unroll
    for (int it = 0; it < 4; ++it)
      __builtin_amdgcn_raw_buffer_store_b128(
          u32x4{v[2 * it].x, v[2 * it].y, v[2 * it + 1].x, v[2 * it + 1].y}, rsrc, lane_off,
          corner + it * 8 * ld * 2, NT);
  }
}

// The plain epilogue: the tile's rows [0, rows) and columns [0, cols) of a row-major
// output of pitch ld, from its corner.
template <typename T>
struct Plain {
  T* out;
  int32_t ld;
  __device__ __forceinline__ void store(const v16f acc[4][4], const Job& j, Stage& stage) const {
    if constexpr (std::is_same<T, uint16_t>::value) {
      if (j.cols >= BN && j.rows >= (j.half ? BM / 2 : BM)) {
        if (j.half) store_pairs<true>(acc, out + j.corner, ld, stage);
        else store_pairs<false>(acc, out + j.corner, ld, stage);
        return;
      }
    }
    if (j.half) store_tile_half(acc, out + j.corner, ld, j.rows, j.cols, stage);
    else store_tile(acc, out + j.corner, ld, j.rows, j.cols, stage);
  }
};

__device__ __forceinline__ Operand group_of(const Operand& B, int32_t group) {
  Operand b = B;
  b.values += static_cast<int64_t>(group) * B.rows * B.k;
  b.scales += static_cast<int64_t>(group) * B.rows * (B.k / 32);
  return b;
}

// The MXFP8 format's part of the shared pipeline (run_tiles); W: operands wide enough
// that the loads address them a K chunk at a time (chunk_at).
template <bool W>
struct MxOf {
  using Operand = bux::Operand;
  using Lds = bux::Lds;
  using Loads = bux::Loads;
  using Lanes = bux::Lanes;
  using Frag = bux::Frag;
  static constexpr bool HALVES = true;  // half tiles: 1 x 4 waves, 128 rows
  __device__ static __forceinline__ Loads loads_a(const Operand& a, int32_t row0) {
    return loads_for(a, row0);
  }
  __device__ static __forceinline__ Loads loads_b(const Operand& b, int32_t group, int32_t row0) {
    return loads_for(group_of(b, group), row0);
  }
  __device__ static __forceinline__ void issue(const Loads& la, const Loads& lb, int32_t ks,
                                               uint32_t lds0, int st, bool half) {
    bux::issue<W>(la, lb, ks, lds0, st, half);
  }
  __device__ static __forceinline__ void wait_loads(int32_t steps) { bux::wait_loads(steps); }
  template <bool H>
  __device__ static __forceinline__ Lanes lanes_of() { return bux::lanes_of<H>(); }
  template <bool H>
  __device__ static __forceinline__ void read_frag(Frag& f, const Lds& lds, const Lanes& ln, int st,
                                                   int32_t ks) {
    bux::read_frag<H>(f, lds, ln, st, ks);
  }
  __device__ static __forceinline__ void mask_frag(Frag& f, int32_t ks, int32_t lo, int32_t hi) {
    bux::mask_frag(f, ks, lo, hi);
  }
  template <bool LOAD, bool READ, bool H>
  __device__ static __forceinline__ void step(const Frag& cur, Frag& nxt, const Loads& la,
                                              const Loads& lb, const Lds& lds, uint32_t lds0,
                                              const Lanes& ln, int32_t ks_load, int st_load,
                                              int32_t ks_next, int st_next, v16f acc[4][4]) {
    if constexpr (H)
      bux::step_half<LOAD, READ, W>(cur, nxt, la, lb, lds, lds0, ln, ks_load, st_load, ks_next,
                                 st_next, acc);
    else
      bux::step<LOAD, READ, W>(cur, nxt, la, lb, lds, lds0, ln, ks_load, st_load, ks_next, st_next, acc);
  }
};
using Mx = MxOf<false>;

// The kernels: one workgroup a CU.
template <typename T, bool W>
__global__ __launch_bounds__(THREADS) __attribute__((amdgpu_waves_per_eu(1, 1))) void rows_kernel(
    Operand A, Operand B, int32_t groups, int32_t n, int32_t height,
    const int32_t* __restrict__ starts, const Tile* __restrict__ tiles, int32_t col_tiles,
    T* __restrict__ y) {
  extern __shared__ __align__(16) uint8_t smem[];
  if (!list_fits(starts, groups, A.rows, height)) return;
  Lds& lds = *reinterpret_cast<Lds*>(smem);
  const RowsTiles<false, true> list{tiles, groups, n, height, col_tiles, A.k / BK, A.k};
  const int32_t count = starts[groups + 1] * col_tiles;
  run_tiles<MxOf<W>>(list, count, A, B, lds, Plain<T>{y, n});
}

// rows_kernel with each group's rows of a from a_starts[g] (the reference's `starts`).
template <typename T, bool W>
__global__ __launch_bounds__(THREADS) __attribute__((amdgpu_waves_per_eu(1, 1))) void rows_started_kernel(
    Operand A, Operand B, int32_t groups, int32_t n, int32_t height,
    const int32_t* __restrict__ starts, const int32_t* __restrict__ a_starts,
    const Tile* __restrict__ tiles, int32_t col_tiles, T* __restrict__ y) {
  extern __shared__ __align__(16) uint8_t smem[];
  if (!list_fits(starts, groups, A.rows, height)) return;
  Lds& lds = *reinterpret_cast<Lds*>(smem);
  const StartedTiles<true> list{tiles, starts, a_starts, groups, n, height, col_tiles, A.k / BK};
  const int32_t count = starts[groups + 1] * col_tiles;
  run_tiles<MxOf<W>>(list, count, A, B, lds, Plain<T>{y, n});
}

template <typename T, bool W>
__global__ __launch_bounds__(THREADS) __attribute__((amdgpu_waves_per_eu(1, 1))) void contract_kernel(
    Operand A, Operand B, int32_t groups, const int32_t* __restrict__ starts, int32_t d_tiles,
    int32_t f_tiles, T* __restrict__ dw) {
  extern __shared__ __align__(16) uint8_t smem[];
  if (!list_fits(starts, groups, -1, 0)) return;
  Lds& lds = *reinterpret_cast<Lds*>(smem);
  const ContractTiles list{starts, A.rows, B.rows, d_tiles, f_tiles, BK};
  const int32_t count = groups * d_tiles * f_tiles;
  run_tiles<MxOf<W>>(list, count, A, B, lds, Plain<T>{dw, B.rows});
}

// Whether an operand of `rows` rows fits the loads' 32-bit offsets within a K chunk
// (a tile's reads past its rows included): rows x 64 bytes, whatever its K.
constexpr int64_t MAX_ROWS = (1LL << 31) / BK - BM;  // 33,554,176
bool rows_fit(int64_t rows) { return rows <= MAX_ROWS; }
// Whether an operand of `rows` rows of `k` bytes of K (and a tile's reads past its rows)
// fits one buffer resource and 32-bit offsets (MxOf<false>); wider ones go a K chunk at
// a time (MxOf<true>).
bool narrow(int64_t rows, int64_t k) { return (rows + BM) * k < (1LL << 31); }

template <typename T, bool W = false>
int launch_rows(const Operand& A, const Operand& B, int32_t groups, int64_t n, int64_t height,
                const int32_t* starts, const Tile* tiles, int64_t slots, void* y, hipStream_t s) {
  if (!W && !(narrow(A.rows, A.k) && narrow(B.rows, B.k)))
    return launch_rows<T, true>(A, B, groups, n, height, starts, tiles, slots, y, s);
  const int64_t col_tiles = ceil_div(n, BN);
  if (slots * col_tiles >= (1LL << 31)) return fail(BUX_E_ARGUMENT, "bux_mx_grouped_rows: too many tiles");
  unsigned blocks = 0;
  if (int rc = grid_for(slots * col_tiles, &blocks)) return rc;
  if (int rc = allow_lds(rows_kernel<T, W>, sizeof(Lds), "rows_kernel")) return rc;
  hipLaunchKernelGGL((rows_kernel<T, W>), dim3(blocks), dim3(THREADS), sizeof(Lds), s, A, B, groups,
                     static_cast<int32_t>(n), static_cast<int32_t>(height), starts, tiles,
                     static_cast<int32_t>(col_tiles), static_cast<T*>(y));
  return launched("rows_kernel");
}

template <typename T, bool W = false>
int launch_rows_started(const Operand& A, const Operand& B, int32_t groups, int64_t n,
                        int64_t height, const int32_t* starts, const int32_t* a_starts,
                        const Tile* tiles, int64_t slots, void* y, hipStream_t s) {
  if (!W && !(narrow(A.rows, A.k) && narrow(B.rows, B.k)))
    return launch_rows_started<T, true>(A, B, groups, n, height, starts, a_starts, tiles, slots,
                                        y, s);
  const int64_t col_tiles = ceil_div(n, BN);
  if (slots * col_tiles >= (1LL << 31)) return fail(BUX_E_ARGUMENT, "bux_mx_grouped_rows_started: too many tiles");
  unsigned blocks = 0;
  if (int rc = grid_for(slots * col_tiles, &blocks)) return rc;
  if (int rc = allow_lds(rows_started_kernel<T, W>, sizeof(Lds), "rows_started_kernel")) return rc;
  hipLaunchKernelGGL((rows_started_kernel<T, W>), dim3(blocks), dim3(THREADS), sizeof(Lds), s, A, B,
                     groups, static_cast<int32_t>(n), static_cast<int32_t>(height), starts,
                     a_starts, tiles, static_cast<int32_t>(col_tiles), static_cast<T*>(y));
  return launched("rows_started_kernel");
}

template <typename T, bool W = false>
int launch_contract(const Operand& A, const Operand& B, int32_t groups, const int32_t* starts,
                    void* dw, hipStream_t s) {
  if (!W && !(narrow(A.rows, A.k) && narrow(B.rows, B.k)))
    return launch_contract<T, true>(A, B, groups, starts, dw, s);
  const int64_t d_tiles = ceil_div(A.rows, BM), f_tiles = ceil_div(B.rows, BN);
  const int64_t tiles = static_cast<int64_t>(groups) * d_tiles * f_tiles;
  if (tiles >= (1LL << 31)) return fail(BUX_E_ARGUMENT, "bux_mx_grouped_contract: too many tiles");
  unsigned blocks = 0;
  if (int rc = grid_for(tiles, &blocks)) return rc;
  if (int rc = allow_lds(contract_kernel<T, W>, sizeof(Lds), "contract_kernel")) return rc;
  hipLaunchKernelGGL((contract_kernel<T, W>), dim3(blocks), dim3(THREADS), sizeof(Lds), s, A, B, groups,
                     starts, static_cast<int32_t>(d_tiles), static_cast<int32_t>(f_tiles),
                     static_cast<T*>(dw));
  return launched("contract_kernel");
}


// --- the fused activation: the up GEMM's tiles straight to h in MXFP8 ---------------
//
// bux_mx_grouped_glu is the rows GEMM of the experts' up projection followed by
// bux_glu_quantize, in one kernel and a small second one: the epilogue stores the
// product (bfloat16, which the backward takes), computes h = act(gate) (up + offset) w
// from the product's bfloat16 values and the row's weight exactly as the activation
// kernel does, and writes both of h's MXFP8 copies, so that no pass reads the product
// back. (The reference fuses the same epilogue into its Blackwell up GEMM,
// grouped_cudnn.activated, grouped_cudnn.py:161-205, for groups padded to 256 rows.)
//
// h's column copy takes absolute blocks of 32 rows. Tiles here start at each group's
// first row rounded down to 32 (the rows before it, another group's, are computed and
// not stored), so every block of the tile that the tile's group holds whole is
// quantized in the epilogue. A block with a group's first row strictly inside it is no
// tile's whole: glu_edges_kernel quantizes those (at most one a group) from the stored
// product afterwards. The results are bit for bit those of the two unfused kernels.

// The fused GEMM's tiles: the 32-aligned tile list by 256-column tiles of the product.
struct GluTiles {
  static constexpr bool HALVES = false;
  const Tile* tiles;
  const int32_t* starts;
  int32_t groups, n, height, col_tiles, k_steps;
  __device__ bool job(int32_t id, Job& j) const {
    const Tile t = tiles[id / col_tiles];
    const int32_t hi = smaller(t.hi, height);
    if (hi <= t.lo) return false;
    const int32_t col0 = (id % col_tiles) * BN;
    const int32_t first = starts[t.group];  // group `groups`: the groups' end
    j.rows = hi - t.lo;
    j.row_lo = first > t.lo ? first - t.lo : 0;
    j.cols = smaller(n - col0, BN);
    j.a_row0 = t.lo;
    j.b_row0 = col0;
    j.group = t.group < groups ? t.group : 0;
    j.ks_begin = 0;
    j.n = t.group < groups ? k_steps : 0;  // rows past the groups: zeros
    j.mask = false;
    j.half = false;
    j.mlo = j.mhi = 0;
    j.corner = static_cast<int64_t>(t.lo) * n + col0;
    return true;
  }
};

// Two floats to two E4M3 codes in the low 16 bits (v_cvt_pk_fp8_f32).
__device__ __forceinline__ uint32_t e4m3x2(float a, float b) {
  return static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false)) & 0xffffu;
}
__device__ __forceinline__ float low_bf16(uint32_t p) { return bf16_to_f32(static_cast<uint16_t>(p & 0xffffu)); }
__device__ __forceinline__ float high_bf16(uint32_t p) { return bf16_to_f32(static_cast<uint16_t>(p >> 16)); }

// The fused epilogue's outputs. The product's columns are (up, gate) pairs of units:
// unit u's up at column 2u, its gate at 2u + 1 (the experts' (f, 2) kernels flattened).
// K: the gated activation (Kind<BUX_SWISH | BUX_QUICK_GELU | BUX_SITU, true>).
template <typename K>
struct GluOut {
  const uint16_t* weights;  // bfloat16 (rows,): each row's weight
  uint16_t* projected;      // bfloat16 (rows, n): the product
  uint8_t* values;          // h along its units, tiled: codes (kf/64, height, 64)
  uint8_t* scales;          //   and scale bytes (kf/128, height, 4)
  uint8_t* t_values;        // h^T along the rows, tiled: codes (height/64, f, 64)
  uint8_t* t_scales;        //   and scale bytes (height/128, f, 4)
  Act act;
  int32_t rows, n, f, height;
  int32_t live;  // rows below it have values: min(the groups' end, rows); set on the device

  // A wave's 128 rows x 64 units of the tile, 32 rows at a time: lane l holds row l % 32
  // and, of each of its four 32-column accumulator blocks jj, units 16 jj + 4 g + 2 (l / 32)
  // and + 1 (g = 0..3: the accumulator's registers 4 g .. 4 g + 3 are the two units' up
  // and gate).
  __device__ void store(const v16f acc[4][4], const Job& j, Stage& stage) const {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1, half = lane >> 5, r32 = lane & 31;
    const int32_t lo = j.a_row0, first = lo + j.row_lo, end = lo + j.rows;
    float w[4];
    bool on[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int32_t r = lo + wm * 128 + i * 32 + r32;
      on[i] = r >= first && r < end && r < live;
      w[i] = on[i] ? bf16_to_f32(weights[r]) : 0.0f;
    }
    // the product as stored, bfloat16 pairs (unit u's up and gate): the accumulators are
    // read once
    uint2 pk[4][4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int jj = 0; jj < 4; ++jj)
#pragma unroll
        for (int g = 0; g < 4; ++g) pk[i][jj][g] = FromAcc{acc}(i, jj, g);
    // rows [first, min(end, rows))
    store_bf16<true>([&](int i, int jj, int g) { return pk[i][jj][g]; }, projected + j.corner, n,
                     smaller(end, rows) - lo, j.cols, stage, j.row_lo);
    const int32_t u0 = (j.b_row0 >> 1) + wn * 64;  // the wave's first unit
    // h of 32 rows x 64 units in this wave's part of the stage, a row 33 words apart
    uint32_t* region = reinterpret_cast<uint32_t*>(reinterpret_cast<uint8_t*>(&stage) +
                                                   wave * 32 * PITCH);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      // one block of 32 rows at a time: nothing of the next is computed ahead
      __builtin_amdgcn_sched_barrier(0);
      const int32_t r0 = lo + wm * 128 + i * 32, r = r0 + r32;
      uint32_t hp[4][4];  // h of units 16 jj + 4 g + 2 half, + 1: a bfloat16 pair
      float amax[2] = {0.0f, 0.0f};
#pragma unroll
      for (int jj = 0; jj < 4; ++jj)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const uint32_t p0 = pk[i][jj][g].x, p1 = pk[i][jj][g].y;
          const int32_t u = u0 + 16 * jj + 4 * g + 2 * half;
          float h0 = 0.0f, h1 = 0.0f;
          if (on[i] && u < f) {
            h0 = glu_unit<K>(act, low_bf16(p0), high_bf16(p0), w[i]);
            h1 = glu_unit<K>(act, low_bf16(p1), high_bf16(p1), w[i]);
          }
          hp[jj][g] = pack_bf16x2(h0, h1);
          amax[jj >> 1] = fmaxf(amax[jj >> 1],
                                fmaxf(fabsf(low_bf16(hp[jj][g])), fabsf(high_bf16(hp[jj][g]))));
        }

      // h along its units: the wave's blocks of 32 units of row r are jj 0-1 and 2-3,
      // each half in this lane and half in lane l ^ 32
#pragma unroll
      for (int b = 0; b < 2; ++b) amax[b] = fmaxf(amax[b], __shfl_xor(amax[b], 32));
      const int e0 = scale_exponent_bf16(amax[0]), e1 = scale_exponent_bf16(amax[1]);
      const float down0 = power_of_two_down(e0), down1 = power_of_two_down(e1);
      uint32_t piece[4][4];  // the two codes of hp[jj][g]
#pragma unroll
      for (int jj = 0; jj < 4; ++jj)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const float down = jj < 2 ? down0 : down1;
          piece[jj][g] = e4m3x2(clip448(low_bf16(hp[jj][g]) * down),
                                clip448(high_bf16(hp[jj][g]) * down));
        }
      // Lane half 0 gathers block 0's 32 codes, half 1 block 1's: each sends the other
      // its pieces of the other's block. Word t of a block is units 4 t .. 4 t + 3, half
      // 0's piece of (jj, g) = (t / 4, t % 4) then half 1's.
      uint32_t sent[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int t0 = 2 * q, t1 = 2 * q + 1;
        const uint32_t a0 = half ? piece[t0 >> 2][t0 & 3] : piece[2 + (t0 >> 2)][t0 & 3];
        const uint32_t a1 = half ? piece[t1 >> 2][t1 & 3] : piece[2 + (t1 >> 2)][t1 & 3];
        sent[q] = __shfl_xor(a0 | (a1 << 16), 32);
      }
      uint32_t word[8];
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        const uint32_t mine = half ? piece[2 + (t >> 2)][t & 3] : piece[t >> 2][t & 3];
        const uint32_t other = (sent[t >> 1] >> (16 * (t & 1))) & 0xffffu;
        word[t] = half ? (other | (mine << 16)) : (mine | (other << 16));
      }
      if (r >= first && r < end) {
        uint4* at = reinterpret_cast<uint4*>(
            values + (static_cast<int64_t>(u0 >> 6) * height + r) * 64 + 32 * half);
        at[0] = make_uint4(word[0], word[1], word[2], word[3]);
        at[1] = make_uint4(word[4], word[5], word[6], word[7]);
        scales[(static_cast<int64_t>(j.b_row0 >> 8) * height + r) * 4 + 2 * wn + half] =
            static_cast<uint8_t>((half ? e1 : e0) + 127);
      }

      // h^T along the rows: the 32-row block from r0 if this tile holds all of it.
      // Through the region: lane (pu, rh) reads units u0 + 2 pu, + 1 of rows 16 rh ..
      // 16 rh + 15 and writes their 16 codes, half of each unit's 32.
#pragma unroll
      for (int jj = 0; jj < 4; ++jj)
#pragma unroll
        for (int g = 0; g < 4; ++g) region[r32 * 33 + 8 * jj + 2 * g + half] = hp[jj][g];
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      __builtin_amdgcn_wave_barrier();
      if (r0 >= first && r0 + 32 <= end) {
        const int pu = lane & 31, rh = lane >> 5;
        uint32_t v[16];
        float m0 = 0.0f, m1 = 0.0f;
#pragma unroll
        for (int k = 0; k < 16; ++k) {
          v[k] = region[(16 * rh + k) * 33 + pu];
          m0 = fmaxf(m0, fabsf(low_bf16(v[k])));
          m1 = fmaxf(m1, fabsf(high_bf16(v[k])));
        }
        m0 = fmaxf(m0, __shfl_xor(m0, 32));
        m1 = fmaxf(m1, __shfl_xor(m1, 32));
        const int t0 = scale_exponent_bf16(m0), t1 = scale_exponent_bf16(m1);
        const float d0 = power_of_two_down(t0), d1 = power_of_two_down(t1);
        uint32_t c0[4], c1[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          c0[q] = e4m3x4(clip448(low_bf16(v[4 * q]) * d0), clip448(low_bf16(v[4 * q + 1]) * d0),
                         clip448(low_bf16(v[4 * q + 2]) * d0), clip448(low_bf16(v[4 * q + 3]) * d0));
          c1[q] = e4m3x4(clip448(high_bf16(v[4 * q]) * d1), clip448(high_bf16(v[4 * q + 1]) * d1),
                         clip448(high_bf16(v[4 * q + 2]) * d1), clip448(high_bf16(v[4 * q + 3]) * d1));
        }
        const int32_t u = u0 + 2 * pu;
        if (u < f) {
          uint8_t* at = t_values + (static_cast<int64_t>(r0 >> 6) * f + u) * 64 + (r0 & 63) + 16 * rh;
          *reinterpret_cast<uint4*>(at) = make_uint4(c0[0], c0[1], c0[2], c0[3]);
          *reinterpret_cast<uint4*>(at + 64) = make_uint4(c1[0], c1[1], c1[2], c1[3]);
          if (rh == 0) {
            uint8_t* sc = t_scales + (static_cast<int64_t>(r0 >> 7) * f + u) * 4 + ((r0 >> 5) & 3);
            sc[0] = static_cast<uint8_t>(t0 + 127);
            sc[4] = static_cast<uint8_t>(t1 + 127);
          }
        }
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      __builtin_amdgcn_wave_barrier();
    }
  }
};

template <typename K>
__global__ __launch_bounds__(THREADS) __attribute__((amdgpu_waves_per_eu(1, 1))) void glu_kernel(
    Operand A, Operand B, int32_t groups, int32_t height, const int32_t* __restrict__ starts,
    const Tile* __restrict__ tiles, int32_t col_tiles, GluOut<K> out) {
  extern __shared__ __align__(16) uint8_t smem[];
  Lds& lds = *reinterpret_cast<Lds*>(smem);
  const GluTiles list{tiles, starts, groups, B.rows, height, col_tiles, A.k / BK};
  out.live = smaller(starts[groups], out.rows);
  const int32_t count = starts[groups + 1] * col_tiles;
  run_tiles<Mx>(list, count, A, B, lds, out);
}

// h^T's blocks of 32 rows with a group's first row strictly inside, which no tile holds
// whole: quantized from the stored product as bux_glu_quantize does (rows from the
// groups' end, or from `rows`, are 0). Workgroup g takes the block of group g's first
// row (g = groups: the groups' end), unless group g - 1's first row is inside the same
// block too; its lane t unit 256 blockIdx.y + t.
template <typename K>
__global__ __launch_bounds__(THREADS) void glu_edges_kernel(
    const int32_t* __restrict__ starts, int32_t groups, const uint16_t* __restrict__ projected,
    const uint16_t* __restrict__ weights, Act act, int32_t rows, int32_t f, int32_t height,
    uint8_t* __restrict__ t_values, uint8_t* __restrict__ t_scales) {
  const int g = blockIdx.x;
  const int32_t first = starts[g];
  if ((first & 31) == 0 || first >= height) return;
  if (g > 0) {
    const int32_t before = starts[g - 1];
    if ((before & 31) != 0 && (before >> 5) == (first >> 5)) return;
  }
  const int32_t live = smaller(starts[groups], rows), r0 = first & ~31;
  const int32_t u = static_cast<int32_t>(blockIdx.y) * THREADS + threadIdx.x;
  if (u < f) {
    float v[32], amax = 0.0f;
#pragma unroll
    for (int k = 0; k < 32; ++k) {
      const int32_t r = r0 + k;
      float h = 0.0f;
      if (r < live) {
        const uint32_t p = *reinterpret_cast<const uint32_t*>(projected + (static_cast<int64_t>(r) * f + u) * 2);
        h = low_bf16(pack_bf16x2(glu_unit<K>(act, low_bf16(p), high_bf16(p), bf16_to_f32(weights[r])), 0.0f));
      }
      v[k] = h;
      amax = fmaxf(amax, fabsf(h));
    }
    const int e = scale_exponent_bf16(amax);
    const float down = power_of_two_down(e);
    uint32_t c[8];
#pragma unroll
    for (int q = 0; q < 8; ++q)
      c[q] = e4m3x4(clip448(v[4 * q] * down), clip448(v[4 * q + 1] * down),
                    clip448(v[4 * q + 2] * down), clip448(v[4 * q + 3] * down));
    uint8_t* at = t_values + (static_cast<int64_t>(r0 >> 6) * f + u) * 64 + (r0 & 63);
    *reinterpret_cast<uint4*>(at) = make_uint4(c[0], c[1], c[2], c[3]);
    *reinterpret_cast<uint4*>(at + 16) = make_uint4(c[4], c[5], c[6], c[7]);
    t_scales[(static_cast<int64_t>(r0 >> 7) * f + u) * 4 + ((r0 >> 5) & 3)] = static_cast<uint8_t>(e + 127);
  }
}

// Tiles of the 32-aligned list: tiles of the height's rows plus, a group (and the rows
// past them), one more and the up to 31 rows before its first.
int64_t glu_slots(int32_t groups, int64_t height) {
  return ceil_div(height + 32 * static_cast<int64_t>(groups + 1), BM) + groups + 1;
}

// --- the activation's gradient in the down dgrad's epilogue ---------------------------
//
// bux_mx_grouped_dglu is the rows GEMM of the down projection's dgrad (dh = dy W[g],
// W[g] f x k) followed by bux_glu_backward_quantize, in one kernel and two small ones:
// the epilogue rounds dh to bfloat16 as the GEMM's output would hold it, reads the
// product's (up, gate) pairs of its units and each row's weight, computes d projected
// (the activation's gradient) and each row's share of its weight's gradient exactly as
// the quantizing backward kernel does, and writes both of d projected's MXFP8 copies,
// so that dh never goes to memory. (The reference's grouped_cudnn.activation_grad,
// grouped_cudnn.py:211-263, for groups padded to 256 rows.)
//
// As in the forward, tiles start at each group's first row rounded down to 32, and the
// column copy's blocks with a group's first row strictly inside are no tile's whole:
// the epilogue leaves d projected's rows of such a block in a slot of the workspace (32
// rows, the slot of the block's first group that starts inside it), from which
// dglu_edges_kernel quantizes them. A row's weight gradient: each 64 columns of d
// projected a partial sum in the quantizing kernel's order of additions, then
// glu_weights_kernel adds them in order. The results are the unfused kernels' bits.

// The slot of 32-row block B: the first g <= groups whose first row lies strictly
// inside the block, or -1.
__device__ __forceinline__ int32_t edge_slot(const int32_t* starts, int32_t groups, int32_t block) {
  const int32_t at = 32 * block;
  int32_t lo = 0, hi = groups + 1;  // the first g with starts[g] > at
  while (lo < hi) {
    const int32_t mid = (lo + hi) >> 1;
    if (starts[mid] > at) hi = mid;
    else lo = mid + 1;
  }
  return lo <= groups && starts[lo] < at + 32 ? lo : -1;
}

// Eight bfloat16 of a uint4 as floats.
__device__ __forceinline__ void floats8(const uint4& q, float* v) {
  const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    v[2 * j] = low_bf16(w[j]);
    v[2 * j + 1] = high_bf16(w[j]);
  }
}

// Two E4M3 words (8 codes) of eight bfloat16 scaled by `down`.
__device__ __forceinline__ uint2 codes8(const uint4& q, float down) {
  float v[8];
  floats8(q, v);
  return make_uint2(e4m3x4(clip448(v[0] * down), clip448(v[1] * down), clip448(v[2] * down),
                           clip448(v[3] * down)),
                    e4m3x4(clip448(v[4] * down), clip448(v[5] * down), clip448(v[6] * down),
                           clip448(v[7] * down)));
}

__device__ __forceinline__ float amax8(const uint4& q) {
  float v[8];
  floats8(q, v);
  float a = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j) a = fmaxf(a, fabsf(v[j]));
  return a;
}

// The fused dgrad's outputs. d projected's columns are (up, gate) pairs of units, as
// the product's: unit u's at 2u and 2u + 1 (n2 = 2 f columns).
// K: the gated activation (Kind<BUX_SWISH | BUX_QUICK_GELU | BUX_SITU, true>).
template <typename K>
struct DGluOut {
  const uint16_t* projected;  // bfloat16 (rows, n2): the up GEMM's product
  const uint16_t* weights;    // bfloat16 (rows,): each row's weight
  uint16_t* d_projected;      // bfloat16 (rows, n2), or NULL
  uint8_t* values;            // d projected along its columns, tiled: codes (k2/64, height, 64)
  uint8_t* scales;            //   and scale bytes (k2/128, height, 4)
  uint8_t* t_values;          // along the rows, tiled: codes (height/64, n2, 64)
  uint8_t* t_scales;          //   and scale bytes (height/128, n2, 4)
  float* partials;            // (rows, tiles): a row's weight-gradient share a 64 columns
  uint16_t* edges;            // (groups + 1, 32, n2): rows of blocks with a first row inside
  const int32_t* starts;
  Act act;
  int32_t rows, f, n2, height, tiles, groups;
  int32_t chunks;  // 64-column chunks of the row copy (its K, 2 f padded to 128)
  int32_t live;  // rows below it have values: min(the groups' end, rows); set on the device

  // A wave's 128 rows x 128 units of the tile, 32 rows at a time: lane l holds row l % 32
  // and, of each 32-unit accumulator block jj, units 32 jj + 8 g + 4 (l / 32) .. + 3 (run
  // g = 0..3: registers 4 g .. 4 g + 3), i.e. d projected's columns 64 jj + 16 g +
  // 8 (l / 32) .. + 7 of the wave's.
  __device__ __forceinline__ void store(const v16f acc[4][4], const Job& j, Stage& stage) const {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1, half = lane >> 5, r32 = lane & 31;
    const int32_t lo = j.a_row0, first = lo + j.row_lo, end = lo + j.rows;
    const int32_t u0 = j.b_row0 + wn * 128;  // the wave's first unit
    // the tile's first and last blocks, where a group's first row lies inside: slots
    const int32_t head = (first & 31) != 0 ? first >> 5 : -1;
    const int32_t tail = (end & 31) != 0 ? end >> 5 : -1;
    const int32_t head_slot = head >= 0 ? edge_slot(starts, groups, head) : -1;
    const int32_t tail_slot = tail >= 0 ? edge_slot(starts, groups, tail) : -1;
    uint32_t* region = reinterpret_cast<uint32_t*>(reinterpret_cast<uint8_t*>(&stage) +
                                                   wave * 32 * PITCH);
    // the product's 4 runs of (up, gate) pairs of accumulator block jj of row block i
    auto load_runs = [&](int i, int jj, uint4 (&pr)[4]) {
      const int32_t r = lo + wm * 128 + i * 32 + r32;
      const bool on = r >= first && r < end && r < live;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int32_t u = u0 + 32 * jj + 8 * g + 4 * half;
        pr[g] = on && u < f ? *reinterpret_cast<const uint4*>(projected + static_cast<int64_t>(r) * n2 + 2 * u)
                            : make_uint4(0, 0, 0, 0);
      }
    };
    uint4 pr[4];
    load_runs(0, 0, pr);
    // (fully unrolled: the accumulators are indexed by constants)
#pragma clang loop unroll(full)
    for (int i = 0; i < 4; ++i) {
      const int32_t r0 = lo + wm * 128 + i * 32, r = r0 + r32;
      const bool mine = r >= first && r < end;  // rows the tile holds
      const bool on = mine && r < live;
      const float w = on ? bf16_to_f32(weights[r]) : 0.0f;
      const int block = r0 >> 5;
      const int32_t slot = block == head ? head_slot : (block == tail ? tail_slot : -1);
      const bool whole = r0 >= first && r0 + 32 <= end;  // the column copy's block
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        __builtin_amdgcn_sched_barrier(0);
        const int32_t c64 = (u0 >> 5) + jj;  // the 64 columns of d projected
        // d projected (bfloat16 pairs, 8 columns a run) and each run's sum of weight terms
        uint4 dp[4];
        float sum[4];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int32_t u = u0 + 32 * jj + 8 * g + 4 * half;
          float p[8], v[8];
          floats8(pr[g], p);
          // dh as the GEMM's bfloat16 output holds it
          const uint2 dh = FromAcc{acc}(i, jj, g);
          const float d[4] = {low_bf16(dh.x), high_bf16(dh.x), low_bf16(dh.y), high_bf16(dh.y)};
          float s = 0.0f;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            float term = 0.0f;
            v[2 * e] = v[2 * e + 1] = 0.0f;
            if (on && u < f) glu_unit_grad<K>(act, p[2 * e], p[2 * e + 1], w, d[e], &v[2 * e], &v[2 * e + 1], &term);
            s += term;
          }
          sum[g] = s;
          dp[g] = make_uint4(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]),
                             pack_bf16x2(v[4], v[5]), pack_bf16x2(v[6], v[7]));
        }
        // the next runs' product goes out while this block's copies are made
        if (jj + 1 < 4) load_runs(i, jj + 1, pr);
        else if (i + 1 < 4) load_runs(i + 1, 0, pr);
        // the row's share of its weight's gradient: the quantizing kernel's 8 chunks of 4
        // units (chunk 2 g + half) added pairwise, pairs of pairs, then the halves
        float x[4];
#pragma unroll
        for (int g = 0; g < 4; ++g) x[g] = sum[g] + __shfl_xor(sum[g], 32);
        const float part = (x[0] + x[1]) + (x[2] + x[3]);
        if (half == 0 && mine && r < rows && c64 < tiles)
          partials[static_cast<int64_t>(r) * tiles + c64] = part;
        // along the columns: blocks b = 0, 1 of 32 (runs 2 b, 2 b + 1 of both halves)
        float am[2];
#pragma unroll
        for (int b = 0; b < 2; ++b) {
          am[b] = fmaxf(amax8(dp[2 * b]), amax8(dp[2 * b + 1]));
          am[b] = fmaxf(am[b], __shfl_xor(am[b], 32));
        }
        const int e0 = scale_exponent_bf16(am[0]), e1 = scale_exponent_bf16(am[1]);
        uint2 piece[4];
#pragma unroll
        for (int g = 0; g < 4; ++g) piece[g] = codes8(dp[g], power_of_two_down(g < 2 ? e0 : e1));
        // Lane half h stores block h's 32 codes: it sends the other half its pieces of the
        // other block (runs 2 (1 - h), + 1) and receives the other half's of its own. Run
        // 2 h + q's columns 16 q + 8 (source half) .. + 7 of the block are words
        // 4 q + 2 (source half), + 1 of the 8.
        // (Selects, not indices by the lane half: an array indexed by a lane's value
        // goes to scratch memory.)
        const uint2 own0 = half ? piece[2] : piece[0], own1 = half ? piece[3] : piece[1];
        const uint2 oth0 = half ? piece[0] : piece[2], oth1 = half ? piece[1] : piece[3];
        const uint32_t s0 = __shfl_xor(oth0.x, 32), s1 = __shfl_xor(oth0.y, 32);
        const uint32_t s2 = __shfl_xor(oth1.x, 32), s3 = __shfl_xor(oth1.y, 32);
        const uint4 run0 = half ? make_uint4(s0, s1, own0.x, own0.y) : make_uint4(own0.x, own0.y, s0, s1);
        const uint4 run1 = half ? make_uint4(s2, s3, own1.x, own1.y) : make_uint4(own1.x, own1.y, s2, s3);
        if (mine && c64 < chunks) {
          uint4* at = reinterpret_cast<uint4*>(values + (static_cast<int64_t>(c64) * height + r) * 64 + 32 * half);
          at[0] = run0;
          at[1] = run1;
          const int32_t bb = 2 * c64 + half;
          scales[(static_cast<int64_t>(bb >> 2) * height + r) * 4 + (bb & 3)] =
              static_cast<uint8_t>((half ? e1 : e0) + 127);
        }
        // the bfloat16 values where asked for, and the rows of an edge block
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int32_t u = u0 + 32 * jj + 8 * g + 4 * half;
          if (mine && u < f) {
            if (d_projected != nullptr && r < rows)
              *reinterpret_cast<uint4*>(d_projected + static_cast<int64_t>(r) * n2 + 2 * u) = dp[g];
            if (slot >= 0)
              *reinterpret_cast<uint4*>(edges + (static_cast<int64_t>(slot) * 32 + r32) * n2 + 2 * u) = dp[g];
          }
        }
        // Along the rows, if this tile holds all of the block from r0: through the region,
        // 64 units (128 columns) at a time, a row 65 words apart; after the second of two
        // accumulator blocks, lane l takes word column l (units u0 + 64 (jj / 2) + l's two
        // columns) down the 32 rows.
        if (whole) {
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            uint32_t* at = region + r32 * 65 + (jj & 1) * 32 + 8 * g + 4 * half;
            at[0] = dp[g].x;
            at[1] = dp[g].y;
            at[2] = dp[g].z;
            at[3] = dp[g].w;
          }
          if (jj & 1) {
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            __builtin_amdgcn_wave_barrier();
            uint32_t v[32];
            float m0 = 0.0f, m1 = 0.0f;
#pragma unroll
            for (int k = 0; k < 32; ++k) {
              v[k] = region[k * 65 + lane];
              m0 = fmaxf(m0, fabsf(low_bf16(v[k])));
              m1 = fmaxf(m1, fabsf(high_bf16(v[k])));
            }
            const int t0 = scale_exponent_bf16(m0), t1 = scale_exponent_bf16(m1);
            const float d0 = power_of_two_down(t0), d1 = power_of_two_down(t1);
            uint32_t c0[8], c1[8];
#pragma unroll
            for (int q = 0; q < 8; ++q) {
              c0[q] = e4m3x4(clip448(low_bf16(v[4 * q]) * d0), clip448(low_bf16(v[4 * q + 1]) * d0),
                             clip448(low_bf16(v[4 * q + 2]) * d0), clip448(low_bf16(v[4 * q + 3]) * d0));
              c1[q] = e4m3x4(clip448(high_bf16(v[4 * q]) * d1), clip448(high_bf16(v[4 * q + 1]) * d1),
                             clip448(high_bf16(v[4 * q + 2]) * d1), clip448(high_bf16(v[4 * q + 3]) * d1));
            }
            const int32_t u = u0 + 32 * (jj - 1) + lane;
            if (u < f) {
              const int64_t c = 2 * static_cast<int64_t>(u);
              uint4* at = reinterpret_cast<uint4*>(t_values + (static_cast<int64_t>(r0 >> 6) * n2 + c) * 64 + (r0 & 63));
              at[0] = make_uint4(c0[0], c0[1], c0[2], c0[3]);
              at[1] = make_uint4(c0[4], c0[5], c0[6], c0[7]);
              at[4] = make_uint4(c1[0], c1[1], c1[2], c1[3]);
              at[5] = make_uint4(c1[4], c1[5], c1[6], c1[7]);
              uint8_t* sc = t_scales + (static_cast<int64_t>(r0 >> 7) * n2 + c) * 4 + ((r0 >> 5) & 3);
              sc[0] = static_cast<uint8_t>(t0 + 127);
              sc[4] = static_cast<uint8_t>(t1 + 127);
            }
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            __builtin_amdgcn_wave_barrier();
          }
        }
      }
    }
  }
};

template <typename K>
__global__ __launch_bounds__(THREADS) __attribute__((amdgpu_waves_per_eu(1, 1))) void dglu_kernel(
    Operand A, Operand B, int32_t groups, int32_t height, const int32_t* __restrict__ starts,
    const Tile* __restrict__ tiles, int32_t col_tiles, DGluOut<K> out) {
  extern __shared__ __align__(16) uint8_t smem[];
  Lds& lds = *reinterpret_cast<Lds*>(smem);
  const GluTiles list{tiles, starts, groups, B.rows, height, col_tiles, A.k / BK};
  out.live = smaller(starts[groups], out.rows);
  const int32_t count = starts[groups + 1] * col_tiles;
  run_tiles<Mx>(list, count, A, B, lds, out);
}

// d projected's column-copy blocks of 32 rows with a group's first row strictly inside,
// from the rows the fused kernel left in the block's slot. Workgroup g takes the block of
// group g's first row if g is its slot (no earlier group's first row strictly inside
// it); its lane t column 256 blockIdx.y + t.
__global__ __launch_bounds__(THREADS) void dglu_edges_kernel(
    const int32_t* __restrict__ starts, int32_t groups, const uint16_t* __restrict__ edges,
    int32_t n2, int32_t height, uint8_t* __restrict__ t_values, uint8_t* __restrict__ t_scales) {
  const int g = blockIdx.x;
  const int32_t first = starts[g];
  if ((first & 31) == 0 || first >= height) return;
  if (g > 0) {
    const int32_t before = starts[g - 1];
    if ((before & 31) != 0 && (before >> 5) == (first >> 5)) return;
  }
  const int32_t c = static_cast<int32_t>(blockIdx.y) * THREADS + threadIdx.x;
  if (c >= n2) return;
  const int32_t r0 = first & ~31;
  float v[32], amax = 0.0f;
#pragma unroll
  for (int k = 0; k < 32; ++k) {
    v[k] = bf16_to_f32(edges[(static_cast<int64_t>(g) * 32 + k) * n2 + c]);
    amax = fmaxf(amax, fabsf(v[k]));
  }
  const int e = scale_exponent_bf16(amax);
  const float down = power_of_two_down(e);
  uint32_t w[8];
#pragma unroll
  for (int q = 0; q < 8; ++q)
    w[q] = e4m3x4(clip448(v[4 * q] * down), clip448(v[4 * q + 1] * down),
                  clip448(v[4 * q + 2] * down), clip448(v[4 * q + 3] * down));
  uint8_t* at = t_values + (static_cast<int64_t>(r0 >> 6) * n2 + c) * 64 + (r0 & 63);
  *reinterpret_cast<uint4*>(at) = make_uint4(w[0], w[1], w[2], w[3]);
  *reinterpret_cast<uint4*>(at + 16) = make_uint4(w[4], w[5], w[6], w[7]);
  t_scales[(static_cast<int64_t>(r0 >> 7) * n2 + c) * 4 + ((r0 >> 5) & 3)] = static_cast<uint8_t>(e + 127);
}

}  // namespace
}  // namespace bux

namespace bux {
namespace {

// The checks of a rows GEMM's arguments, `name` its entry point.
int check_rows(const char* name, const uint8_t* a_values, const uint8_t* a_scales,
               const uint8_t* b_values, const uint8_t* b_scales, int32_t groups, int64_t m,
               int64_t n, int64_t k, int64_t height, int out_dtype, const void* y) {
  BUX_CHECK(groups >= 1 && groups <= MAX_GROUPS, "%s: groups=%d outside [1, %d]", name, groups,
            MAX_GROUPS);
  BUX_CHECK(m >= 0 && n > 0 && k > 0 && height >= 0 && height < (1LL << 31) && m < (1LL << 31),
            "%s: bad shape m=%lld n=%lld k=%lld height=%lld", name, (long long)m, (long long)n,
            (long long)k, (long long)height);
  BUX_CHECK(k % 128 == 0, "%s: k=%lld is not a multiple of 128 (the tiled layout's padded K)",
            name, (long long)k);
  BUX_CHECK(n % 4 == 0, "%s: n=%lld is not a multiple of 4", name, (long long)n);
  BUX_CHECK(rows_fit(m) && rows_fit(n), "%s: an operand of %lld rows exceeds %lld", name,
            (long long)(m > n ? m : n), (long long)MAX_ROWS);
  BUX_CHECK(out_dtype == BUX_BF16 || out_dtype == BUX_F32, "%s: out_dtype=%d", name, out_dtype);
  BUX_CHECK(b_values && b_scales && y && (m == 0 || (a_values && a_scales)), "%s: NULL buffer",
            name);
  return BUX_OK;
}

int check_contract(const char* name, const uint8_t* a_values, const uint8_t* a_scales,
                   const uint8_t* b_values, const uint8_t* b_scales, int32_t groups, int64_t d,
                   int64_t f, int64_t m, int out_dtype, const void* dw) {
  BUX_CHECK(groups >= 1 && groups <= MAX_GROUPS, "%s: groups=%d outside [1, %d]", name, groups,
            MAX_GROUPS);
  BUX_CHECK(d > 0 && f > 0 && m >= 0 && m < (1LL << 31), "%s: bad shape d=%lld f=%lld m=%lld",
            name, (long long)d, (long long)f, (long long)m);
  BUX_CHECK(m % 128 == 0, "%s: m=%lld is not a multiple of 128", name, (long long)m);
  BUX_CHECK(f % 4 == 0, "%s: f=%lld is not a multiple of 4", name, (long long)f);
  BUX_CHECK(rows_fit(d) && rows_fit(f), "%s: an operand of %lld rows exceeds %lld", name,
            (long long)(d > f ? d : f), (long long)MAX_ROWS);
  BUX_CHECK(out_dtype == BUX_BF16 || out_dtype == BUX_F32, "%s: out_dtype=%d", name, out_dtype);
  BUX_CHECK(dw && (m == 0 || (a_values && a_scales && b_values && b_scales)), "%s: NULL buffer",
            name);
  return BUX_OK;
}

int launch_rows_of(const uint8_t* a_values, const uint8_t* a_scales, const uint8_t* b_values,
                   const uint8_t* b_scales, const void* list, int32_t groups, int64_t m, int64_t n,
                   int64_t k, int64_t height, int out_dtype, void* y, hipStream_t s) {
  // Rows of the groups past a's m rows read 0 (the resource ends there) or the
  // following K chunk's rows: a's m must cover every row the groups hold.
  const Operand A{a_values, a_scales, static_cast<int32_t>(k), static_cast<int32_t>(m)};
  const Operand B{b_values, b_scales, static_cast<int32_t>(k), static_cast<int32_t>(n)};
  const int64_t slots = row_slots(groups, m, height);
  int32_t* starts = starts_in(list);
  Tile* tiles = tiles_in(list, groups);
  return out_dtype == BUX_BF16
             ? launch_rows<uint16_t>(A, B, groups, n, height, starts, tiles, slots, y, s)
             : launch_rows<float>(A, B, groups, n, height, starts, tiles, slots, y, s);
}

int launch_contract_of(const uint8_t* a_values, const uint8_t* a_scales, const uint8_t* b_values,
                       const uint8_t* b_scales, const int32_t* starts, int32_t groups, int64_t d,
                       int64_t f, int64_t m, int out_dtype, void* dw, hipStream_t s) {
  // The operands' K is m: each of a's d rows (b's f rows) is m bytes.
  const Operand A{a_values, a_scales, static_cast<int32_t>(m), static_cast<int32_t>(d)};
  const Operand B{b_values, b_scales, static_cast<int32_t>(m), static_cast<int32_t>(f)};
  return out_dtype == BUX_BF16 ? launch_contract<uint16_t>(A, B, groups, starts, dw, s)
                               : launch_contract<float>(A, B, groups, starts, dw, s);
}

}  // namespace
}  // namespace bux

extern "C" size_t bux_mx_grouped_rows_workspace_size(int32_t groups, int64_t m, int64_t height) {
  using namespace bux;
  return starts_bytes(groups) + static_cast<size_t>(row_slots(groups, m, height)) * sizeof(Tile);
}

extern "C" int bux_mx_grouped_tiles(const int32_t* sizes, int32_t groups, int64_t m,
                                    int64_t height, void* list, size_t list_bytes, void* stream) {
  using namespace bux;
  clear_error();
  BUX_CHECK(groups >= 1 && groups <= MAX_GROUPS, "bux_mx_grouped_tiles: groups=%d outside [1, %d]",
            groups, MAX_GROUPS);
  BUX_CHECK(m >= 0 && height >= 0 && height < (1LL << 31) && m < (1LL << 31),
            "bux_mx_grouped_tiles: bad shape m=%lld height=%lld", (long long)m, (long long)height);
  BUX_CHECK(sizes != nullptr, "bux_mx_grouped_tiles: NULL sizes");
  const size_t need = bux_mx_grouped_rows_workspace_size(groups, m, height);
  if (list == nullptr || list_bytes < need)
    return fail(BUX_E_WORKSPACE, "bux_mx_grouped_tiles: list of %zu bytes, %zu needed", list_bytes,
                need);
  hipLaunchKernelGGL(prologue_kernel, dim3(1), dim3(THREADS), 0, as_stream(stream), sizes, groups,
                     height, row_slots(groups, m, height), 1, starts_in(list), tiles_in(list, groups),
                     header_in(list), m, nullptr);
  return launched("prologue_kernel");
}

extern "C" int bux_mx_grouped_rows(const uint8_t* a_values, const uint8_t* a_scales,
                                   const uint8_t* b_values, const uint8_t* b_scales,
                                   const int32_t* sizes, int32_t groups, int64_t m, int64_t n,
                                   int64_t k, int64_t height, int out_dtype, void* y,
                                   void* workspace, size_t workspace_bytes, void* stream) {
  using namespace bux;
  clear_error();
  if (int rc = check_rows("bux_mx_grouped_rows", a_values, a_scales, b_values, b_scales, groups, m,
                          n, k, height, out_dtype, y))
    return rc;
  BUX_CHECK(sizes != nullptr, "bux_mx_grouped_rows: NULL buffer");
  const size_t need = bux_mx_grouped_rows_workspace_size(groups, m, height);
  if (workspace == nullptr || workspace_bytes < need)
    return fail(BUX_E_WORKSPACE, "bux_mx_grouped_rows: workspace of %zu bytes, %zu needed",
                workspace_bytes, need);
  if (height == 0) return BUX_OK;
  hipStream_t s = as_stream(stream);
  hipLaunchKernelGGL(prologue_kernel, dim3(1), dim3(THREADS), 0, s, sizes, groups, height,
                     row_slots(groups, m, height), 1, starts_in(workspace),
                     tiles_in(workspace, groups), header_in(workspace), m, nullptr);
  if (int rc = launched("prologue_kernel")) return rc;
  return launch_rows_of(a_values, a_scales, b_values, b_scales, workspace, groups, m, n, k, height,
                        out_dtype, y, s);
}

extern "C" int bux_mx_grouped_rows_started(const uint8_t* a_values, const uint8_t* a_scales,
                                           const uint8_t* b_values, const uint8_t* b_scales,
                                           const int32_t* sizes, const int32_t* starts,
                                           int32_t groups, int64_t m, int64_t n, int64_t k,
                                           int64_t height, int out_dtype, void* y,
                                           void* workspace, size_t workspace_bytes,
                                           void* stream) {
  using namespace bux;
  clear_error();
  if (int rc = check_rows("bux_mx_grouped_rows_started", a_values, a_scales, b_values, b_scales,
                          groups, m, n, k, height, out_dtype, y))
    return rc;
  BUX_CHECK(sizes != nullptr && starts != nullptr, "bux_mx_grouped_rows_started: NULL sizes or starts");
  const size_t need = bux_mx_grouped_rows_workspace_size(groups, m, height);
  if (workspace == nullptr || workspace_bytes < need)
    return fail(BUX_E_WORKSPACE, "bux_mx_grouped_rows_started: workspace of %zu bytes, %zu needed",
                workspace_bytes, need);
  if (height == 0) return BUX_OK;
  hipStream_t s = as_stream(stream);
  const int64_t slots = row_slots(groups, m, height);
  hipLaunchKernelGGL(prologue_kernel, dim3(1), dim3(THREADS), 0, s, sizes, groups, height, slots,
                     1, starts_in(workspace), tiles_in(workspace, groups), header_in(workspace), m,
                     starts);
  if (int rc = launched("prologue_kernel")) return rc;
  // a's rows past m read 0 (the resource ends there): the groups' rows are the caller's
  const Operand A{a_values, a_scales, static_cast<int32_t>(k), static_cast<int32_t>(m)};
  const Operand B{b_values, b_scales, static_cast<int32_t>(k), static_cast<int32_t>(n)};
  return out_dtype == BUX_BF16
             ? launch_rows_started<uint16_t>(A, B, groups, n, height, starts_in(workspace), starts,
                                             tiles_in(workspace, groups), slots, y, s)
             : launch_rows_started<float>(A, B, groups, n, height, starts_in(workspace), starts,
                                          tiles_in(workspace, groups), slots, y, s);
}

// --- bux_mx_grouped_rows without a workspace -------------------------------------------
//
// For callers that cannot allocate (graph capture, serving loops): the rows GEMM's
// workspace -- the group starts and the tile list its prologue writes in full on every
// call, so nothing in it needs clearing -- in a static device array of SCRATCH_BYTES,
// each GPU its own copy, held until the process ends. Every call on a GPU shares that
// GPU's array: two calls that overlap on one GPU (two streams, two host threads) race.
namespace bux {
namespace {

constexpr size_t SCRATCH_BYTES = BUX_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) uint8_t scratch[SCRATCH_BYTES];

constexpr int MAX_DEVICES = 64;
std::mutex scratch_lock;
void* scratch_at[MAX_DEVICES] = {};  // each device's address of `scratch`, once known

// The current device's address of `scratch` (host code never passes the array's own
// name, a host-side stand-in, to a kernel).
int scratch_of(void** out) {
  int device = 0;
  hipError_t err = hipGetDevice(&device);
  if (err != hipSuccess) return fail(BUX_E_DEVICE, "the current device: %s", hipGetErrorString(err));
  if (device < 0 || device >= MAX_DEVICES)
    return fail(BUX_E_DEVICE, "device %d: the scratch arrays cover devices 0 to %d", device,
                MAX_DEVICES - 1);
  std::lock_guard<std::mutex> hold(scratch_lock);
  if (scratch_at[device] == nullptr) {
    void* at = nullptr;
    err = hipGetSymbolAddress(&at, HIP_SYMBOL(scratch));
    if (err != hipSuccess || at == nullptr)
      return fail(BUX_E_DEVICE, "device %d: the scratch array's address: %s", device,
                  hipGetErrorString(err));
    scratch_at[device] = at;
  }
  *out = scratch_at[device];
  return BUX_OK;
}

}  // namespace
}  // namespace bux

extern "C" int bux_mx_grouped_rows_noalloc(const uint8_t* a_values, const uint8_t* a_scales,
                                           const uint8_t* b_values, const uint8_t* b_scales,
                                           const int32_t* sizes, int32_t groups, int64_t m,
                                           int64_t n, int64_t k, int64_t height, int out_dtype,
                                           void* y, void* stream) {
  using namespace bux;
  clear_error();
  if (int rc = check_rows("bux_mx_grouped_rows_noalloc", a_values, a_scales, b_values, b_scales,
                          groups, m, n, k, height, out_dtype, y))
    return rc;
  BUX_CHECK(sizes != nullptr, "bux_mx_grouped_rows_noalloc: NULL buffer");
  const size_t need = bux_mx_grouped_rows_workspace_size(groups, m, height);
  if (need > SCRATCH_BYTES)
    return fail(BUX_E_WORKSPACE,
                "bux_mx_grouped_rows_noalloc: groups=%d, m=%lld, height=%lld need a workspace of "
                "%zu bytes, past its fixed %zu (use bux_mx_grouped_rows with a workspace)",
                groups, (long long)m, (long long)height, need, SCRATCH_BYTES);
  if (height == 0) return BUX_OK;
  void* ws = nullptr;
  if (int rc = scratch_of(&ws)) return rc;
  hipStream_t s = as_stream(stream);
  hipLaunchKernelGGL(prologue_kernel, dim3(1), dim3(THREADS), 0, s, sizes, groups, height,
                     row_slots(groups, m, height), 1, starts_in(ws), tiles_in(ws, groups),
                     header_in(ws), m, nullptr);
  if (int rc = launched("prologue_kernel")) return rc;
  return launch_rows_of(a_values, a_scales, b_values, b_scales, ws, groups, m, n, k, height,
                        out_dtype, y, s);
}

extern "C" int bux_mx_grouped_rows_listed(const uint8_t* a_values, const uint8_t* a_scales,
                                          const uint8_t* b_values, const uint8_t* b_scales,
                                          void* list, size_t list_bytes, int32_t groups,
                                          int64_t m, int64_t n, int64_t k, int64_t height,
                                          int out_dtype, void* y, void* stream) {
  using namespace bux;
  clear_error();
  if (int rc = check_rows("bux_mx_grouped_rows_listed", a_values, a_scales, b_values, b_scales,
                          groups, m, n, k, height, out_dtype, y))
    return rc;
  BUX_CHECK(list != nullptr, "bux_mx_grouped_rows_listed: NULL list");
  const size_t need = bux_mx_grouped_rows_workspace_size(groups, m, height);
  if (list_bytes < need)
    return fail(BUX_E_WORKSPACE,
                "bux_mx_grouped_rows_listed: a list of %zu bytes, not one for groups=%d m=%lld "
                "height=%lld (%zu bytes)", list_bytes, groups, (long long)m, (long long)height, need);
  if (height == 0) return BUX_OK;
  return launch_rows_of(a_values, a_scales, b_values, b_scales, list, groups, m, n, k, height,
                        out_dtype, y, as_stream(stream));
}

extern "C" size_t bux_mx_grouped_contract_workspace_size(int32_t groups) {
  using namespace bux;
  return starts_bytes(groups);  // a list of the group starts alone: header, starts
}

extern "C" int bux_mx_grouped_contract(const uint8_t* a_values, const uint8_t* a_scales,
                                       const uint8_t* b_values, const uint8_t* b_scales,
                                       const int32_t* sizes, int32_t groups, int64_t d, int64_t f,
                                       int64_t m, int out_dtype, void* dw, void* workspace,
                                       size_t workspace_bytes, void* stream) {
  using namespace bux;
  clear_error();
  if (int rc = check_contract("bux_mx_grouped_contract", a_values, a_scales, b_values, b_scales,
                              groups, d, f, m, out_dtype, dw))
    return rc;
  BUX_CHECK(sizes != nullptr, "bux_mx_grouped_contract: NULL buffer");
  const size_t need = bux_mx_grouped_contract_workspace_size(groups);
  if (workspace == nullptr || workspace_bytes < need)
    return fail(BUX_E_WORKSPACE, "bux_mx_grouped_contract: workspace of %zu bytes, %zu needed",
                workspace_bytes, need);
  hipStream_t s = as_stream(stream);
  // the starts capped at the contract's K (m rows), as the rows GEMM caps them at its rows
  hipLaunchKernelGGL(prologue_kernel, dim3(1), dim3(THREADS), 0, s, sizes, groups, 0, 0, 1,
                     starts_in(workspace), nullptr, header_in(workspace), m, nullptr);
  if (int rc = launched("prologue_kernel")) return rc;
  return launch_contract_of(a_values, a_scales, b_values, b_scales, starts_in(workspace), groups,
                            d, f, m,
                            out_dtype, dw, s);
}

extern "C" int bux_mx_grouped_contract_listed(const uint8_t* a_values, const uint8_t* a_scales,
                                              const uint8_t* b_values, const uint8_t* b_scales,
                                              void* list, size_t list_bytes, int32_t groups,
                                              int64_t d, int64_t f, int64_t m, int out_dtype,
                                              void* dw, void* stream) {
  using namespace bux;
  clear_error();
  if (int rc = check_contract("bux_mx_grouped_contract_listed", a_values, a_scales, b_values,
                              b_scales, groups, d, f, m, out_dtype, dw))
    return rc;
  BUX_CHECK(list != nullptr, "bux_mx_grouped_contract_listed: NULL list");
  if (list_bytes < starts_bytes(groups))
    return fail(BUX_E_WORKSPACE,
                "bux_mx_grouped_contract_listed: a list of %zu bytes, not one for groups=%d",
                list_bytes, groups);
  return launch_contract_of(a_values, a_scales, b_values, b_scales, starts_in(list), groups, d, f,
                            m, out_dtype, dw, as_stream(stream));
}

extern "C" size_t bux_mx_grouped_glu_workspace_size(int32_t groups, int64_t height) {
  using namespace bux;
  return starts_bytes(groups) + static_cast<size_t>(glu_slots(groups, height)) * sizeof(Tile);
}

extern "C" int bux_mx_grouped_glu(const uint8_t* a_values, const uint8_t* a_scales,
                                  const uint8_t* b_values, const uint8_t* b_scales,
                                  const int32_t* sizes, int32_t groups, int64_t height, int64_t n,
                                  int64_t k, int64_t rows, const uint16_t* weights,
                                  const bux_ffn* ffn, uint16_t* projected,
                                  uint8_t* values, uint8_t* scales, uint8_t* t_values,
                                  uint8_t* t_scales, void* workspace, size_t workspace_bytes,
                                  void* stream) {
  using namespace bux;
  clear_error();
  BUX_CHECK(groups >= 1 && groups <= MAX_GROUPS, "bux_mx_grouped_glu: groups=%d outside [1, %d]",
            groups, MAX_GROUPS);
  BUX_CHECK(height >= 0 && height % 128 == 0 && height < (1LL << 31) && n > 0 && n % 64 == 0 &&
                k > 0 && k % 128 == 0 && rows >= 0 && rows <= height,
            "bux_mx_grouped_glu: bad shape height=%lld n=%lld k=%lld rows=%lld (height a "
            "multiple of 128, n of 64, k of 128, rows at most height)",
            (long long)height, (long long)n, (long long)k, (long long)rows);
  BUX_CHECK(narrow(height, k) && narrow(n, k),
            "bux_mx_grouped_glu: an operand of %lld x %lld bytes exceeds 2 GiB",
            (long long)(height > n ? height : n), (long long)k);
  Act act;
  if (int rc = act_of("bux_mx_grouped_glu", ffn, &act)) return rc;
  BUX_CHECK(act.gated && (act.kind == BUX_SWISH || act.kind == BUX_QUICK_GELU || act.kind == BUX_SITU),
            "bux_mx_grouped_glu: the fused epilogue is of a gated BUX_SWISH, BUX_QUICK_GELU or "
            "BUX_SITU, not activation %d%s", act.kind, act.gated ? "" : " plain");
  BUX_CHECK(sizes && b_values && b_scales &&
                (height == 0 || (a_values && a_scales && values && scales && t_values && t_scales)) &&
                (rows == 0 || (weights && projected)),
            "bux_mx_grouped_glu: NULL buffer");
  const size_t need = bux_mx_grouped_glu_workspace_size(groups, height);
  if (workspace == nullptr || workspace_bytes < need)
    return fail(BUX_E_WORKSPACE, "bux_mx_grouped_glu: workspace of %zu bytes, %zu needed",
                workspace_bytes, need);
  if (height == 0) return BUX_OK;
  hipStream_t s = as_stream(stream);
  int32_t* starts = starts_in(workspace);
  Tile* tiles = tiles_in(workspace, groups);
  const int64_t slots = glu_slots(groups, height);
  const int64_t col_tiles = ceil_div(n, BN);
  if (slots * col_tiles >= (1LL << 31)) return fail(BUX_E_ARGUMENT, "bux_mx_grouped_glu: too many tiles");
  hipLaunchKernelGGL(prologue_kernel, dim3(1), dim3(THREADS), 0, s, sizes, groups, height, slots,
                     32, starts, tiles, nullptr, 0, nullptr);
  if (int rc = launched("prologue_kernel")) return rc;
  const Operand A{a_values, a_scales, static_cast<int32_t>(k), static_cast<int32_t>(height)};
  const Operand B{b_values, b_scales, static_cast<int32_t>(k), static_cast<int32_t>(n)};
  const int32_t f = static_cast<int32_t>(n / 2);
  unsigned blocks = 0;
  if (int rc = grid_for(slots * col_tiles, &blocks)) return rc;
  auto run = [&](auto kind) {
    using K = decltype(kind);
    const GluOut<K> out{weights, projected, values, scales, t_values, t_scales, act,
                        static_cast<int32_t>(rows), static_cast<int32_t>(n), f,
                        static_cast<int32_t>(height), 0};
    if (int rc = allow_lds(glu_kernel<K>, sizeof(Lds), "glu_kernel")) return rc;
    hipLaunchKernelGGL(glu_kernel<K>, dim3(blocks), dim3(THREADS), sizeof(Lds), s, A, B, groups,
                       static_cast<int32_t>(height), starts, tiles, static_cast<int32_t>(col_tiles),
                       out);
    if (int rc = launched("glu_kernel")) return rc;
    hipLaunchKernelGGL(glu_edges_kernel<K>,
                       dim3(static_cast<unsigned>(groups + 1), static_cast<unsigned>(ceil_div(f, THREADS))),
                       dim3(THREADS), 0, s, starts, groups, projected, weights, act,
                       static_cast<int32_t>(rows), f, static_cast<int32_t>(height), t_values,
                       t_scales);
    return launched("glu_edges_kernel");
  };
  if (act.kind == BUX_QUICK_GELU) return run(Kind<BUX_QUICK_GELU, true>{});
  if (act.kind == BUX_SITU) return run(Kind<BUX_SITU, true>{});
  return run(Kind<BUX_SWISH, true>{});
}

// The fused dgrad's workspace: the tile list (the fused up GEMM's), then the rows'
// weight-gradient partials (a float a row and 64 columns of d projected), then the edge
// blocks' slots (32 rows of d projected a group and one for the groups' end).
namespace bux {
namespace {
int64_t dglu_tiles(int64_t f) { return ceil_div(2 * f, 128) * 2; }
size_t dglu_partials_at(int32_t groups, int64_t height) {
  return align256(starts_bytes(groups) + static_cast<size_t>(glu_slots(groups, height)) * sizeof(Tile));
}
size_t dglu_edges_at(int32_t groups, int64_t height, int64_t rows, int64_t f) {
  return dglu_partials_at(groups, height) +
         align256(static_cast<size_t>(rows) * static_cast<size_t>(dglu_tiles(f)) * sizeof(float));
}
}  // namespace
}  // namespace bux

extern "C" size_t bux_mx_grouped_dglu_workspace_size(int32_t groups, int64_t height, int64_t rows,
                                                     int64_t f) {
  using namespace bux;
  return dglu_edges_at(groups, height, rows, f) +
         static_cast<size_t>(groups + 1) * 32 * static_cast<size_t>(2 * f) * sizeof(uint16_t);
}

extern "C" int bux_mx_grouped_dglu(const uint8_t* a_values, const uint8_t* a_scales,
                                   const uint8_t* b_values, const uint8_t* b_scales,
                                   const int32_t* sizes, int32_t groups, int64_t height, int64_t f,
                                   int64_t k, int64_t rows, const uint16_t* projected,
                                   const uint16_t* weights, const bux_ffn* ffn,
                                   uint16_t* d_projected, uint8_t* values, uint8_t* scales,
                                   uint8_t* t_values, uint8_t* t_scales, uint16_t* d_weights,
                                   void* workspace, size_t workspace_bytes, void* stream) {
  using namespace bux;
  clear_error();
  BUX_CHECK(groups >= 1 && groups <= MAX_GROUPS, "bux_mx_grouped_dglu: groups=%d outside [1, %d]",
            groups, MAX_GROUPS);
  BUX_CHECK(height >= 0 && height % 128 == 0 && height < (1LL << 31) && f > 0 && f % 32 == 0 &&
                k > 0 && k % 128 == 0 && rows >= 0 && rows <= height,
            "bux_mx_grouped_dglu: bad shape height=%lld f=%lld k=%lld rows=%lld (height a "
            "multiple of 128, f of 32, k of 128, rows at most height)",
            (long long)height, (long long)f, (long long)k, (long long)rows);
  BUX_CHECK(narrow(height, k) && narrow(f, k),
            "bux_mx_grouped_dglu: an operand of %lld x %lld bytes exceeds 2 GiB",
            (long long)(height > f ? height : f), (long long)k);
  Act act;
  if (int rc = act_of("bux_mx_grouped_dglu", ffn, &act)) return rc;
  BUX_CHECK(act.gated && (act.kind == BUX_SWISH || act.kind == BUX_QUICK_GELU || act.kind == BUX_SITU),
            "bux_mx_grouped_dglu: the fused epilogue is of a gated BUX_SWISH, BUX_QUICK_GELU or "
            "BUX_SITU, not activation %d%s", act.kind, act.gated ? "" : " plain");
  BUX_CHECK(sizes && b_values && b_scales &&
                (height == 0 || (a_values && a_scales && values && scales && t_values && t_scales)) &&
                (rows == 0 || (weights && projected && d_weights)),
            "bux_mx_grouped_dglu: NULL buffer");
  const size_t need = bux_mx_grouped_dglu_workspace_size(groups, height, rows, f);
  if (workspace == nullptr || workspace_bytes < need)
    return fail(BUX_E_WORKSPACE, "bux_mx_grouped_dglu: workspace of %zu bytes, %zu needed",
                workspace_bytes, need);
  if (height == 0) return BUX_OK;
  hipStream_t s = as_stream(stream);
  int32_t* starts = starts_in(workspace);
  Tile* tiles = tiles_in(workspace, groups);
  uint8_t* base = static_cast<uint8_t*>(workspace);
  float* partials = reinterpret_cast<float*>(base + dglu_partials_at(groups, height));
  uint16_t* edges = reinterpret_cast<uint16_t*>(base + dglu_edges_at(groups, height, rows, f));
  const int64_t slots = glu_slots(groups, height);
  const int64_t col_tiles = ceil_div(f, BN);
  if (slots * col_tiles >= (1LL << 31)) return fail(BUX_E_ARGUMENT, "bux_mx_grouped_dglu: too many tiles");
  hipLaunchKernelGGL(prologue_kernel, dim3(1), dim3(THREADS), 0, s, sizes, groups, height, slots,
                     32, starts, tiles, nullptr, 0, nullptr);
  if (int rc = launched("prologue_kernel")) return rc;
  const Operand A{a_values, a_scales, static_cast<int32_t>(k), static_cast<int32_t>(height)};
  const Operand B{b_values, b_scales, static_cast<int32_t>(k), static_cast<int32_t>(f)};
  const int32_t n2 = static_cast<int32_t>(2 * f), tiles64 = static_cast<int32_t>(dglu_tiles(f));
  unsigned blocks = 0;
  if (int rc = grid_for(slots * col_tiles, &blocks)) return rc;
  auto run = [&](auto kind) {
    using K = decltype(kind);
    const DGluOut<K> out{projected, weights, d_projected, values, scales, t_values, t_scales,
                         partials, edges, starts, act, static_cast<int32_t>(rows),
                         static_cast<int32_t>(f), n2, static_cast<int32_t>(height), tiles64,
                         groups, static_cast<int32_t>(ceil_div(n2, 128) * 2), 0};
    if (int rc = allow_lds(dglu_kernel<K>, sizeof(Lds), "dglu_kernel")) return rc;
    hipLaunchKernelGGL(dglu_kernel<K>, dim3(blocks), dim3(THREADS), sizeof(Lds), s, A, B, groups,
                       static_cast<int32_t>(height), starts, tiles, static_cast<int32_t>(col_tiles),
                       out);
    return launched("dglu_kernel");
  };
  int rc = act.kind == BUX_QUICK_GELU ? run(Kind<BUX_QUICK_GELU, true>{})
           : act.kind == BUX_SITU     ? run(Kind<BUX_SITU, true>{})
                                      : run(Kind<BUX_SWISH, true>{});
  if (rc != BUX_OK) return rc;
  hipLaunchKernelGGL(dglu_edges_kernel,
                     dim3(static_cast<unsigned>(groups + 1), static_cast<unsigned>(ceil_div(n2, THREADS))),
                     dim3(THREADS), 0, s, starts, groups, edges, n2, static_cast<int32_t>(height),
                     t_values, t_scales);
  if (int rc2 = launched("dglu_edges_kernel")) return rc2;
  return launch_glu_weights(partials, rows, tiles64, starts + groups, d_weights, s);
}
