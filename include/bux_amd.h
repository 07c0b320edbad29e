/* bux_amd: the MoE expert path of bux (pilot7747/bux) as hand-written HIP kernels for
 * MI355X (gfx950), behind a plain C ABI.
 *
 * Every entry point enqueues its kernels on the caller's HIP stream (`stream`, a
 * hipStream_t; NULL for the default stream) and returns at once: no host
 * synchronisation, no allocation. Buffers are device pointers owned by the caller;
 * inputs are read only; outputs may hold anything on entry, and every element of them
 * is written (0 where the reference's result is 0). Scratch memory comes in as a
 * `workspace` of at least the size the matching `*_workspace_size` call returns.
 *
 * Return value: 0 on success; otherwise a nonzero BUX_E_* code, with a message that
 * `bux_last_error` returns on the same thread. Shapes are checked on the host before
 * any kernel is launched.
 *
 * Rows read through an index (a pick's token, index / index_div) come from a matrix
 * whose rows the call also takes (`sources`, `tokens`, `n`): a row that lies outside
 * it, or a negative index, reads as a row of 0. The reference's indices (the sort's
 * order) are always inside; the bound keeps every read inside the caller's buffer.
 *
 * Layouts (row-major throughout):
 *   bfloat16   uint16_t bit patterns;
 *   MXFP8      an (r, c) matrix in blocks of 32 along its rows -- the reference's
 *              `Blocks` (src/bux/architecture/precision/blockscaled.py:43-56): E4M3
 *              codes and one E8M0 scale byte a block -- in the tiled layout the grouped
 *              GEMMs load, which, as the reference's `Tiled` (experts/grouped_mxfp8.py:
 *              93-103) does for its kernels, pads c to K = whole 128s (codes 0, scale
 *              bytes 1) and lays K out in chunks:
 *                codes   uint8 [K / 64][r][64]:  element (i, j) at ((j / 64) r + i) 64 + j % 64
 *                scales  uint8 [K / 128][r][4]:  block b of row i at ((b / 4) r + i) 4 + b % 4
 *              A stack of g matrices is g of these one after another.
 *
 * References are to files under /root/reference (pilot7747/bux).
 */
#ifndef BUX_AMD_H
#define BUX_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  BUX_OK = 0,
  BUX_E_ARGUMENT = 1, /* a shape, pointer or flag the entry point does not take */
  BUX_E_WORKSPACE = 2, /* the workspace is smaller than *_workspace_size says */
  BUX_E_LAUNCH = 3, /* the HIP runtime refused a launch */
  BUX_E_DEVICE = 4 /* the current device is not a gfx950 */
};

/* The message of the last failed call on this thread ("" if none). */
const char* bux_last_error(void);

/* The library's version, major * 10000 + minor * 100 + patch. */
int bux_version(void);

/* ---------------------------------------------------------------------------------
 * a-1. Sort the picks by expert.
 *
 * Replaces moe.sort_by_expert (src/bux/architecture/experts/moe.py:776-791) with
 * in_range (:794), and the group offsets the grouped GEMMs derive from the sizes
 * (grouped_mxfp8.py:142, ``cumsum(sizes) - sizes``).
 *
 * idx       int32 [n_picks]: each pick's expert (a token's k picks in a row).
 * order     int32 [n_picks]: the picks sorted by expert, stably; picks outside
 *           [0, num_experts) sort last.
 * inverse   int32 [n_picks]: inverse[order[i]] = i.
 * sizes     int32 [num_experts]: picks of each expert.
 * offsets   int32 [num_experts + 1]: cumsum(sizes) - sizes, then sum(sizes) (the
 *           rows that hold values, `filled` of grouped_blockscaled.py:180).
 */
size_t bux_moe_permute_workspace_size(int64_t n_picks, int32_t num_experts);
int bux_moe_permute(const int32_t* idx, int64_t n_picks, int32_t num_experts, int32_t* order,
                    int32_t* inverse, int32_t* sizes, int32_t* offsets, void* workspace,
                    size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------------
 * a-4. MXFP8 quantization of a matrix and of its transpose, in one pass.
 *
 * Replaces grouped_triton.quantized_twice (src/bux/architecture/experts/
 * grouped_triton.py:44-101) and, off a Blackwell GPU, grouped_blockscaled._quantized
 * (grouped_blockscaled.py:296-317) with blockscaled.mx_twice / mx_quantize
 * (precision/blockscaled.py:282-356): per 32 values, the scale 2^e with
 * e = ceil_log2(amax / 448) clipped to [-126, 126] (byte e + 127, 1 for a block of
 * zeros), each value times 2^-e clipped to +-448 and rounded to nearest even E4M3.
 *
 * x         bfloat16 [groups, rows, cols] (a stack of `groups` matrices), or, with an
 *           index, the matrix the rows are read from, [sources, cols].
 * index     NULL, or int32 [rows]: row i is x[index[i] / index_div] (groups must be 1),
 *           a row whose index is negative, or whose source row is not below `sources`,
 *           reading 0 -- the reference's `Picked` rows, tokens[order // k]
 *           (grouped_blockscaled.py:53-62, grouped_triton.py:208-214).
 * sources   with an index, x's rows (ignored without one).
 * rows      rows of the matrix (x's, or the index's entries).
 * height    rows of the copies, a multiple of 32, >= rows; rows from `rows` on are 0
 *           (the reference pads to whole tiles, grouped_blockscaled.py:122-128).
 * filled    NULL (every row holds values) or a device int32: rows from *filled on
 *           quantize as 0 (grouped_blockscaled.py:314).
 * flags     BUX_MX_ROWS: write values and scales, x (height, cols) in MXFP8 along its
 *           rows, tiled with K = cols rounded up to 128: [groups, K/64, height, 64] and
 *           [groups, K/128, height, 4]. BUX_MX_COLUMNS: write t_values and t_scales,
 *           x^T (cols, height) likewise with K = height rounded up to 128:
 *           [groups, K/64, cols, 64] and [groups, K/128, cols, 4].
 *           With BUX_MX_TILES as well, the scale is one per 32 x 32 tile of x, which
 *           both copies take (so they hold the same codes, transposed): the mxfp8_2d
 *           recipe's weights, blockscaled.mx_tiles_twice (src/bux/architecture/
 *           precision/blockscaled.py:294-309).
 *           With BUX_MX_HALVES, x's columns are a GLU's (up, gate) pairs, read as its
 *           halves (quantized_twice's `halves`, grouped_triton.py:49,61-62, and
 *           grouped_cudnn.halves_of, grouped_cudnn.py:150-155): in each 64 columns of
 *           the copies, the 32 pairs' gates, then their ups; cols a multiple of 64.
 *           cols must be a multiple of 32.
 */
enum { BUX_MX_ROWS = 1, BUX_MX_COLUMNS = 2, BUX_MX_TILES = 4, BUX_MX_HALVES = 8 };
int bux_mx_quantize(const uint16_t* x, const int32_t* index, int32_t index_div, int64_t sources,
                    int64_t groups, int64_t rows, int64_t cols, int64_t height,
                    const int32_t* filled, int flags, uint8_t* values, uint8_t* scales,
                    uint8_t* t_values, uint8_t* t_scales, void* stream);
/* bux_mx_quantize_f32: the same of a float32 x (the reference quantizes any float dtype
 * the same way, in float32: blockscaled._in_e4m3, precision/blockscaled.py:323-343; its
 * layer's tokens and kernels in float32, experts/moe.py:846 and
 * grouped_blockscaled.py:129): a block's scale from its largest magnitude's float32
 * quotient by 448, the codes of x times 2^-e. */
int bux_mx_quantize_f32(const float* x, const int32_t* index, int32_t index_div,
                        int64_t sources, int64_t groups, int64_t rows, int64_t cols,
                        int64_t height, const int32_t* filled, int flags, uint8_t* values,
                        uint8_t* scales, uint8_t* t_values, uint8_t* t_scales, void* stream);

/* ---------------------------------------------------------------------------------
 * a-6. Grouped MXFP8 GEMM over rows: y[i] = a[i] b[g(i)]^T.
 *
 * Replaces grouped_mxfp8.rows (src/bux/architecture/experts/grouped_mxfp8.py:116-154)
 * with its tile list tiles_of (:157-182), and off Blackwell grouped_blockscaled._times
 * (grouped_blockscaled.py:220-233): float32 sums, rows past sum(sizes) are 0.
 *
 * a_values/a_scales  MXFP8 tiled, m rows of k bytes: the rows, group 0's first.
 * b_values/b_scales  MXFP8 tiled, a stack of groups matrices of n rows of k bytes.
 * sizes     device int32 [groups], summing to at most m (a negative size counts as 0,
 *           and sizes summing past max(m, height) give the last groups fewer rows).
 * k         the tiled K: the contracted length rounded up to a multiple of 128.
 * y         [height, n], bfloat16 (out_dtype BUX_BF16) or float32 (BUX_F32); rows
 *           from sum(sizes) to height are 0. Any height: a's quantized copy may be
 *           padded past the height of y (e.g. to whole tiles) and rows of the groups
 *           past height are not stored. n must be a multiple of 4.
 * Sizes: m, n and height up to 33,554,176 rows (a K chunk's rows x 64 bytes within 2 GiB);
 * an operand's bytes have no cap (past 2 GiB the kernel loads it one K chunk at a time
 * from a 64-bit base).
 */
enum { BUX_BF16 = 0, BUX_F32 = 1 };
size_t bux_mx_grouped_rows_workspace_size(int32_t groups, int64_t m, int64_t height);
int bux_mx_grouped_rows(const uint8_t* a_values, const uint8_t* a_scales, const uint8_t* b_values,
                        const uint8_t* b_scales, const int32_t* sizes, int32_t groups, int64_t m,
                        int64_t n, int64_t k, int64_t height, int out_dtype, void* y,
                        void* workspace, size_t workspace_bytes, void* stream);

/* bux_mx_grouped_rows_started: bux_mx_grouped_rows with each group's rows of a where
 * `starts` (int32 [groups], on the device) puts them: group g's sizes[g] rows of a from
 * row starts[g] on (the reference's `starts`, grouped_mxfp8.py:116-154, for groups laid
 * out apart, e.g. at whole tiles as grouped_glu.padded lays them, grouped_glu.py:
 * 239-272); y's rows stay packed (group g's from sum(sizes[:g])), and rows past the
 * groups are 0. m: a's rows, past every group's last; the same workspace as
 * bux_mx_grouped_rows. a's rows between the groups are read where a group's last tile
 * reaches over them, and never reach y.
 */
int bux_mx_grouped_rows_started(const uint8_t* a_values, const uint8_t* a_scales,
                                const uint8_t* b_values, const uint8_t* b_scales,
                                const int32_t* sizes, const int32_t* starts, int32_t groups,
                                int64_t m, int64_t n, int64_t k, int64_t height, int out_dtype,
                                void* y, void* workspace, size_t workspace_bytes, void* stream);

/* bux_mx_grouped_tiles: the rows GEMM's device prologue on its own, the reference's
 * tiles_of (grouped_mxfp8.py:157-182), whose result its rows and contract take as
 * `tiles` and `starts` (:116, :185): the group starts and the ragged tile list of
 * `sizes` for a of m rows and y of `height` rows, into `list`
 * (bux_mx_grouped_rows_workspace_size(groups, m, height) bytes). The list opens with a
 * header of its dimensions: int32 words BUX_LIST_MAGIC, groups, m, height and a status
 * word, 0 when made.
 * bux_mx_grouped_rows_listed / bux_mx_grouped_contract_listed: bux_mx_grouped_rows /
 * bux_mx_grouped_contract on such a list (`list_bytes` its size), made from the same
 * sizes (and, for rows, the same groups, m and height), in place of their own
 * prologue: one list serves every GEMM of a layer's step. A list shorter than those
 * dimensions need is refused on the host (BUX_E_WORKSPACE); one whose header names
 * other dimensions is refused by the GEMM kernel itself as it starts: it writes nothing
 * and sets the list's status word to BUX_LIST_REFUSED.
 */
enum { BUX_LIST_MAGIC = 0x54585542, BUX_LIST_REFUSED = 1 };
int bux_mx_grouped_tiles(const int32_t* sizes, int32_t groups, int64_t m, int64_t height,
                         void* list, size_t list_bytes, void* stream);
int bux_mx_grouped_rows_listed(const uint8_t* a_values, const uint8_t* a_scales,
                               const uint8_t* b_values, const uint8_t* b_scales, void* list,
                               size_t list_bytes, int32_t groups, int64_t m, int64_t n, int64_t k,
                               int64_t height, int out_dtype, void* y, void* stream);
int bux_mx_grouped_contract_listed(const uint8_t* a_values, const uint8_t* a_scales,
                                   const uint8_t* b_values, const uint8_t* b_scales, void* list,
                                   size_t list_bytes, int32_t groups, int64_t d, int64_t f,
                                   int64_t m, int out_dtype, void* dw, void* stream);

/* bux_mx_grouped_rows_noalloc: bux_mx_grouped_rows with no workspace argument and no
 * allocation of any kind. It has no counterpart in the reference: it is for callers that
 * cannot allocate (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc). Its workspace -- the group starts and the tile list -- lives in a
 * static device array of BUX_NOALLOC_SCRATCH_BYTES on each GPU, held until the process
 * ends; a call whose bux_mx_grouped_rows_workspace_size(groups, m, height) exceeds it
 * fails with BUX_E_WORKSPACE (256 KiB: e.g. 1024 groups and 3.5 M rows). Nothing in the
 * array needs clearing (each call's prologue writes all it reads), but every call on a
 * GPU shares that GPU's array: calls that overlap on one GPU (two streams, two host
 * threads) race. Same outputs as bux_mx_grouped_rows, bit for bit. The array's address
 * is looked up once per device, on the first call there, and kept for the process:
 * after a hipDeviceReset (or a reload of the library's code object) that address is
 * stale, so the entry point must not be used across a device reset.
 */
enum { BUX_NOALLOC_SCRATCH_BYTES = 262144 };
int bux_mx_grouped_rows_noalloc(const uint8_t* a_values, const uint8_t* a_scales,
                                const uint8_t* b_values, const uint8_t* b_scales,
                                const int32_t* sizes, int32_t groups, int64_t m, int64_t n,
                                int64_t k, int64_t height, int out_dtype, void* y, void* stream);

/* ---------------------------------------------------------------------------------
 * a-7. Grouped MXFP8 GEMM contracting each group's rows: dw[g] = a[:, g] b[:, g]^T.
 *
 * Replaces grouped_mxfp8.contract (grouped_mxfp8.py:185-210) with its edge tiles
 * _edges (:240-256), and off Blackwell grouped_blockscaled._contract
 * (grouped_blockscaled.py:236-250): in a block of 32 that two groups share, each
 * group's sum takes a's codes of its own rows only (the others count as 0, under the
 * block's one scale); float32 sums.
 *
 * a_values/a_scales  MXFP8 tiled, d rows of m bytes: x^T in blocks along the rows m.
 * b_values/b_scales  MXFP8 tiled, f rows of m bytes: dy^T likewise.
 * sizes     device int32 [groups]; sum(sizes) <= m; m a multiple of 128.
 * dw        [groups, d, f], bfloat16 or float32 (out_dtype); 0 for an empty group.
 *           f must be a multiple of 4.
 * Sizes: d and f up to 33,554,176 rows, m below 2^31; an operand's bytes have no cap, as
 * for bux_mx_grouped_rows.
 */
size_t bux_mx_grouped_contract_workspace_size(int32_t groups);
int bux_mx_grouped_contract(const uint8_t* a_values, const uint8_t* a_scales,
                            const uint8_t* b_values, const uint8_t* b_scales,
                            const int32_t* sizes, int32_t groups, int64_t d, int64_t f,
                            int64_t m, int out_dtype, void* dw, void* workspace,
                            size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------------
 * a-10. bfloat16 grouped GEMMs (the experts in "compute" precision).
 *
 * bux_bf16_grouped_rows replaces grouped.dot / jax.lax.ragged_dot
 * (src/bux/architecture/experts/grouped.py:90-102): y[i] = x[i] w[g(i)], float32
 * sums, bfloat16 out, rows past sum(sizes) 0. x bfloat16 [m, k]; w bfloat16
 * [groups, k, n] (w_transposed 0) or [groups, n, k] (1: y[i] = x[i] w[g]^T, the dgrad).
 * bux_bf16_grouped_contract replaces grouped.weight_grad (grouped.py:105-146):
 * dw[g] = x[rows of g]^T dy[rows of g], x [m, k], dy [m, n] -> dw [groups, k, n]; 0 for
 * an empty group.
 * Any n and k. With n and k multiples of 8 and every operand (plus a tile of 256 past
 * it each way) under 2 GiB, the operands' rows go to LDS by 16-byte direct loads; other
 * shapes (the reference's ragged_dot takes any) are read an element at a time by
 * slower kernels with the same sums and rounding. m under 2^31. workspace:
 * bux_bf16_grouped_rows_workspace_size(groups, m) /
 * bux_bf16_grouped_contract_workspace_size(groups) bytes (the group starts and the
 * tile list that each call builds on the device).
 */
size_t bux_bf16_grouped_rows_workspace_size(int32_t groups, int64_t m);
int bux_bf16_grouped_rows(const uint16_t* x, const uint16_t* w, int w_transposed,
                          const int32_t* sizes, int32_t groups, int64_t m, int64_t n, int64_t k,
                          uint16_t* y, void* workspace, size_t workspace_bytes, void* stream);
size_t bux_bf16_grouped_contract_workspace_size(int32_t groups);
int bux_bf16_grouped_contract(const uint16_t* x, const uint16_t* dy, const int32_t* sizes,
                              int32_t groups, int64_t m, int64_t k, int64_t n, uint16_t* dw,
                              void* workspace, size_t workspace_bytes, void* stream);
/* The same two GEMMs for a layer in float32 (ragged_dot and its transpose of float32
 * operands, grouped.py:90-146 with x in float32): x, w, dy, y and dw float32, float32
 * products and sums (v_mfma_f32_32x32x2_f32), any n and k; the same workspaces. */
int bux_bf16_grouped_rows_f32(const float* x, const float* w, int w_transposed,
                              const int32_t* sizes, int32_t groups, int64_t m, int64_t n,
                              int64_t k, float* y, void* workspace, size_t workspace_bytes,
                              void* stream);
int bux_bf16_grouped_contract_f32(const float* x, const float* dy, const int32_t* sizes,
                                  int32_t groups, int64_t m, int64_t k, int64_t n, float* dw,
                                  void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------------
 * a-2 / a-3. The token path's gathers and sums.
 *
 * bux_token_rows replaces moe.token_rows (moe.py:991-1016) and picked_weights
 * (:1027-1032): rows[i] = z[order[i] / k] for i < m (width columns, bfloat16), z
 * [tokens, width]; a row of 0 where order[i] / k lies outside [0, tokens).
 * Any width; a multiple of 8 moves 16 bytes a lane.
 * bux_token_sums replaces grouped_blockscaled.sum_by_token (grouped_blockscaled.py:
 * 141-148) and moe.token_sums (moe.py:1035-1066): out[t] = sum_j y[inverse[t k + j]]
 * added in float32 in pick order, rounded once to bfloat16; an inverse outside
 * [0, y_rows) adds 0.
 */
int bux_token_rows(const uint16_t* z, int64_t tokens, const int32_t* order, int64_t m, int32_t k,
                   int64_t width, uint16_t* rows, void* stream);
int bux_token_sums(const uint16_t* y, int64_t y_rows, const int32_t* inverse, int64_t tokens,
                   int32_t k, int64_t width, uint16_t* out, void* stream);
/* bux_token_sums_f32: the same for float32 y (a layer in float32): float32 sums in the
 * same order, stored as they are (no rounding). */
int bux_token_sums_f32(const float* y, int64_t y_rows, const int32_t* inverse, int64_t tokens,
                       int32_t k, int64_t width, float* out, void* stream);

/* ---------------------------------------------------------------------------------
 * a-8. The experts' activation between the two GEMMs, times each row's weight.
 *
 * Replaces moe.weighted_units (moe.py:898-910) = weighted(hidden_units(...))
 * (:913-926) with layers/mlp.activate (layers/mlp.py:20-35) of
 * common/functional.activation (functional.py:12-40), settings config.MLPConfig's
 * (config.py:204-221):
 *   gated (gated_mlp, projected (m, f, 2): [..., 0] up, [..., 1] gate, moe.py:845):
 *     h = act(min(gate, limit)) * (cap(clip(up)) + up_offset) * w
 *   plain (mlp, projected (m, f)):
 *     h = act(cap(clip(up))) * w
 * clip(u) = u clipped to [-limit, limit] when `clamped` (limit None in the reference:
 * clamped 0); cap(u) = up_softcap tanh(u / up_softcap) when `capped`. act one of
 *   BUX_SWISH       x sigmoid(x)              BUX_QUICK_GELU  x sigmoid(1.702 x)
 *   BUX_RELU        max(x, 0)                 BUX_RELU2       max(x, 0)^2
 *   BUX_GELU        x Phi(x) (erf)            BUX_GELU_TANH   gelu's tanh form
 *   BUX_SIGMOID     sigmoid(x)                BUX_TANH        tanh(x)
 *   BUX_SOFTPLUS    log(1 + e^x)              BUX_SITU        4 tanh(x / 4) sigmoid(x)
 * (quick_gelu's 1.702 as jax multiplies a bfloat16 by it: 1.703125). float32 inside,
 * one rounding to bfloat16. Rows from *filled on (if filled is not NULL) give 0.
 * The backward gives d projected (projected's shape) and d weights (m), the VJP that
 * jax takes of the forward after its jax.checkpoint recompute (moe.py:906-910), with
 * clip's and minimum's gradient 1 inside, 1/2 at the limit, 0 outside, relu's 0 at 0.
 * f a multiple of 4.
 */
enum {
  BUX_SWISH = 0, BUX_QUICK_GELU = 1, BUX_RELU = 2, BUX_RELU2 = 3, BUX_GELU = 4,
  BUX_GELU_TANH = 5, BUX_SIGMOID = 6, BUX_TANH = 7, BUX_SOFTPLUS = 8, BUX_SITU = 9
};
typedef struct bux_ffn {
  int32_t activation; /* BUX_SWISH .. BUX_SITU */
  int32_t gated;      /* 1: gated_mlp, projected (m, f, 2); 0: mlp, projected (m, f) */
  int32_t clamped;    /* 1: `limit` clips (limit >= 0) */
  float limit;
  int32_t capped;     /* 1: `up_softcap` caps up (up_softcap > 0) */
  float up_softcap;
  float up_offset;    /* gated only */
} bux_ffn;
int bux_glu_forward(const uint16_t* projected, const uint16_t* weights, const int32_t* filled,
                    int64_t m, int64_t f, const bux_ffn* ffn, uint16_t* h, void* stream);
int bux_glu_backward(const uint16_t* projected, const uint16_t* weights, const uint16_t* dh,
                     const int32_t* filled, int64_t m, int64_t f, const bux_ffn* ffn,
                     uint16_t* d_projected, uint16_t* d_weights, void* stream);
/* The same for a layer in float32: every buffer above float32, one rounding to float32,
 * quick_gelu's 1.702 as a float32 (as bux_glu_quantize_f32). */
int bux_glu_forward_f32(const float* projected, const float* weights, const int32_t* filled,
                        int64_t m, int64_t f, const bux_ffn* ffn, float* h, void* stream);
int bux_glu_backward_f32(const float* projected, const float* weights, const float* dh,
                         const int32_t* filled, int64_t m, int64_t f, const bux_ffn* ffn,
                         float* d_projected, float* d_weights, void* stream);

/* ---------------------------------------------------------------------------------
 * a-8. The experts' biases (MLPConfig.bias, config.py:214).
 *
 * Rows are the picks sorted by expert; offsets (int32 [experts + 1], nondecreasing,
 * bux_moe_permute's) put row r in the expert e with offsets[e] <= r < offsets[e + 1]
 * and past offsets[experts] in none.
 * bux_expert_bias_add replaces moe.by_expert and the add (moe.py:857-861,876-885):
 *   x[r] = x[r] + bias[e(r)] in place, both bfloat16, one rounding (rows in no expert
 *   add 0). x [m, width], bias [experts, width]: the up bias ((E, f, p) flattened).
 * bux_expert_sums replaces by_expert's gradient (the one-hot matmul's transpose,
 *   moe.py:876-885, and weighted's, :922-925, for the down bias):
 *   out[e] = sum over rows r of e of v_r, in float32, out float32 [experts, width];
 *   v_r = x[src(r)], or with weights (bfloat16 [m]) x[src(r)] * weights[r] rounded
 *   to bfloat16; src(r) = r, or with index index[r] / index_div (a pick's token: x
 *   then [sources, width], a source row outside it reading 0). Rows at or past m (an
 *   expert's offsets reaching beyond them) add nothing.
 * bux_token_sums_biased replaces the down bias's forward (moe.py:866-870):
 *   out[t] = sum_by_token(y) + sum_by_token(bias[e(r)] * weights[r]), each sum as
 *   bux_token_sums adds it (the products rounded to bfloat16 first), their sum rounded.
 * bux_expert_bias_weight_grad adds the down bias's share of the weights' gradient
 *   (weighted's VJP, moe.py:922-925): d_weights[r] += sum_c dy[src(r)][c] bias[e(r)][c]
 *   (products rounded to bfloat16, summed in float32, rounded, then added in bfloat16);
 *   src(r) as bux_expert_sums's, dy [sources, width] with an index.
 */
int bux_expert_bias_add(uint16_t* x, int64_t m, int64_t width, const uint16_t* bias,
                        const int32_t* offsets, int32_t experts, void* stream);
int bux_expert_sums(const uint16_t* x, const int32_t* index, int32_t index_div, int64_t sources,
                    const uint16_t* weights, int64_t m, int64_t width, const int32_t* offsets,
                    int32_t experts, float* out, void* stream);
int bux_token_sums_biased(const uint16_t* y, int64_t y_rows, const int32_t* inverse,
                          int64_t tokens, int32_t k, int64_t width, const uint16_t* bias,
                          const int32_t* offsets, int32_t experts, const uint16_t* weights,
                          uint16_t* out, void* stream);
int bux_expert_bias_weight_grad(const uint16_t* dy, const int32_t* index, int32_t index_div,
                                int64_t sources, int64_t m, int64_t width, const uint16_t* bias,
                                const int32_t* offsets, int32_t experts, uint16_t* d_weights,
                                void* stream);
/* The same four for a layer in float32 (moe.py:848-849: by_expert casts the biases to
 * x's dtype): every bfloat16 buffer above float32, each rounding float32 arithmetic's own
 * (the sums the same sums in the same order). */
int bux_expert_bias_add_f32(float* x, int64_t m, int64_t width, const float* bias,
                            const int32_t* offsets, int32_t experts, void* stream);
int bux_expert_sums_f32(const float* x, const int32_t* index, int32_t index_div, int64_t sources,
                        const float* weights, int64_t m, int64_t width, const int32_t* offsets,
                        int32_t experts, float* out, void* stream);
int bux_token_sums_biased_f32(const float* y, int64_t y_rows, const int32_t* inverse,
                              int64_t tokens, int32_t k, int64_t width, const float* bias,
                              const int32_t* offsets, int32_t experts, const float* weights,
                              float* out, void* stream);
int bux_expert_bias_weight_grad_f32(const float* dy, const int32_t* index, int32_t index_div,
                                    int64_t sources, int64_t m, int64_t width, const float* bias,
                                    const int32_t* offsets, int32_t experts, float* d_weights,
                                    void* stream);

/* ---------------------------------------------------------------------------------
 * a-8. The per-expert norm of the experts' outputs (MoEConfig.expert_norm,
 * config.py:306).
 *
 * bux_expert_norm_forward replaces moe.experts' norm path (moe.py:871-872):
 *   out[r] = weighted(norm(y[r] + down_bias[e(r)]), weights[r]), bfloat16 [m, d];
 * y the down GEMM's rows (not summed, not weighted: the activation before it runs with
 * weights of 1, moe.py:871), down_bias [experts, d] or NULL, offsets/experts as the
 * biases' above; rows in no expert give 0. The norm is layers/norm.Norm
 * (layers/norm.py:14-78) of `bux_norm` in bfloat16 compute: gain = scale (1 + scale if
 * zero_centered), applied before the normalization with scale_input, else after it;
 * statistics in float32 (layernorm: centred, then over the root of the mean square plus
 * eps; rmsnorm: the latter alone); the result rounded to bfloat16, each later product
 * and sum rounded as the reference's bfloat16 ops round. scale [d] (affine) and bias
 * [d] (bias) bfloat16, else NULL. d a multiple of 8, at most 8192.
 * bux_expert_norm_backward: its VJP, given the tokens' gradient dy [sources, d] read
 * through index / index_div (the sort's order and k; dy [m, d] read row for row with
 * index NULL, sources then ignored): dv [m, d], the gradient to y (and, by
 * expert, to the down bias: bux_expert_sums of it); d_weights [m] (written: the norm
 * path's only use of the weights); d_scale and d_bias [d] float32 sums over the rows
 * (NULL where the norm has none). workspace:
 * bux_expert_norm_backward_workspace_size(m, d) bytes.
 */
enum { BUX_LAYERNORM = 0, BUX_RMSNORM = 1 };
typedef struct bux_norm {
  int32_t kind;          /* BUX_LAYERNORM or BUX_RMSNORM */
  int32_t affine;        /* a learned gain, `scale` */
  int32_t zero_centered; /* the gain is 1 + scale */
  int32_t scale_input;   /* the gain multiplies before the normalization */
  int32_t bias;          /* a learned bias, added last */
  float eps;
} bux_norm;
int bux_expert_norm_forward(const uint16_t* y, int64_t m, int64_t d, const uint16_t* down_bias,
                            const int32_t* offsets, int32_t experts, const bux_norm* norm,
                            const uint16_t* scale, const uint16_t* bias, const uint16_t* weights,
                            uint16_t* out, void* stream);
size_t bux_expert_norm_backward_workspace_size(int64_t m, int64_t d);
int bux_expert_norm_backward(const uint16_t* dy, const int32_t* index, int32_t index_div,
                             int64_t sources, const uint16_t* y, int64_t m, int64_t d,
                             const uint16_t* down_bias, const int32_t* offsets, int32_t experts,
                             const bux_norm* norm,
                             const uint16_t* scale, const uint16_t* bias,
                             const uint16_t* weights, uint16_t* dv, uint16_t* d_weights,
                             float* d_scale, float* d_bias, void* workspace,
                             size_t workspace_bytes, void* stream);
/* The same for a layer in float32 (layers/norm.py:14-78 in float32 compute): y, dy,
 * down_bias, scale, bias, weights, out, dv and d_weights float32, each rounding float32
 * arithmetic's own; the same workspace. */
int bux_expert_norm_forward_f32(const float* y, int64_t m, int64_t d, const float* down_bias,
                                const int32_t* offsets, int32_t experts, const bux_norm* norm,
                                const float* scale, const float* bias, const float* weights,
                                float* out, void* stream);
int bux_expert_norm_backward_f32(const float* dy, const int32_t* index, int32_t index_div,
                                 int64_t sources, const float* y, int64_t m, int64_t d,
                                 const float* down_bias, const int32_t* offsets, int32_t experts,
                                 const bux_norm* norm, const float* scale, const float* bias,
                                 const float* weights, float* dv, float* d_weights,
                                 float* d_scale, float* d_bias, void* workspace,
                                 size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------------
 * a-8 with a-4. The activation and its gradient, quantized as they are computed.
 *
 * The reference fuses the activation and the weight into its up GEMM's epilogue on
 * Blackwell (grouped_cudnn.activated / activation_grad, experts/grouped_cudnn.py:
 * 161-263) and otherwise quantizes the activation's bfloat16 result
 * (grouped_blockscaled._quantized, grouped_blockscaled.py:296-317); here one kernel
 * computes the bfloat16 values bux_glu_forward / bux_glu_backward compute and writes
 * both MXFP8 copies of them as bux_mx_quantize does (rows from *filled on as 0), with no
 * round trip of the bfloat16 result through memory.
 *
 * Any bux_ffn, gated or plain; f a multiple of 32.
 * bux_glu_quantize: h (m, f) of projected ((m, f, 2) gated, (m, f) plain) and the
 *   rows' weights (m);
 *   values/scales: h along its rows (K = f rounded up to 128), height rows;
 *   t_values/t_scales: h^T along its rows (K = height rounded up to 128), f rows;
 *   either copy NULL where its GEMM does not multiply in MXFP8 (at least one given);
 *   h: NULL, or bfloat16 [m, f] to store h as well.
 * bux_glu_backward_quantize: d projected (m, p f; p = 2 gated, 1 plain) of projected,
 *   the weights and dh (m, f); values/scales along its rows (K = p f rounded up to
 *   128), t_values/t_scales of its transpose (either NULL, as above); d_projected: NULL,
 *   or bfloat16 [m, p f]
 *   to store it as well; d_weights [m] as bux_glu_backward's (its float32 sum taken in
 *   another fixed order). workspace: bux_glu_backward_quantize_workspace_size(m, f)
 *   bytes.
 */
int bux_glu_quantize(const uint16_t* projected, const uint16_t* weights, const int32_t* filled,
                     int64_t m, int64_t f, const bux_ffn* ffn, int64_t height, uint16_t* h, uint8_t* values, uint8_t* scales,
                     uint8_t* t_values, uint8_t* t_scales, void* stream);
/* bux_glu_quantize_f32 / bux_glu_backward_quantize_f32: the same for a layer in float32
 *   (tokens and kernels float32: the reference computes the activation and its gradient
 *   in x's dtype, experts/moe.py:846-885): projected, weights, dh, h, d_projected and
 *   d_weights float32, each value the float32 result of the same arithmetic (no
 *   rounding to bfloat16), quantized as bux_mx_quantize_f32 quantizes. */
int bux_glu_quantize_f32(const float* projected, const float* weights, const int32_t* filled,
                         int64_t m, int64_t f, const bux_ffn* ffn, int64_t height, float* h,
                         uint8_t* values, uint8_t* scales, uint8_t* t_values, uint8_t* t_scales,
                         void* stream);
/* bux_mx_grouped_glu: the experts' up GEMM with the activation and both MXFP8 copies
 *   of h in its epilogue, the reference's fused up GEMM (grouped_cudnn.activated,
 *   src/bux/architecture/experts/grouped_cudnn.py:161-205), but for groups as they lie
 *   (no padding of each to 256 rows). The same outputs, bit for bit, as
 *   bux_mx_grouped_rows(a, b, sizes, m = height, n, k, height = rows) into projected,
 *   then bux_glu_quantize(projected, weights, filled = sum(sizes), rows, n / 2, ...,
 *   height):
 *   a_values/a_scales  x in MXFP8 along its rows, tiled, height rows of k bytes;
 *   b_values/b_scales  each expert's (n, k) up kernels, tiled; n = 2 f, columns in
 *     (up, gate) pairs; f a multiple of 32;
 *   projected  bfloat16 [rows, n] (rows <= height; past sum(sizes): 0);
 *   values/scales  h along its units (K = f rounded up to 128), height rows;
 *   t_values/t_scales  h^T along the rows (K = height, a multiple of 128), f rows;
 *   workspace  bux_mx_grouped_glu_workspace_size(groups, height) bytes.
 *   ffn: gated, of BUX_SWISH, BUX_QUICK_GELU or BUX_SITU (with any clamp, cap and
 *   offset): the activations of the reference's fused kernels' gated epilogues
 *   (grouped_glu.epilogue, experts/grouped_glu.py:119-140).
 */
size_t bux_mx_grouped_glu_workspace_size(int32_t groups, int64_t height);
int bux_mx_grouped_glu(const uint8_t* a_values, const uint8_t* a_scales, const uint8_t* b_values,
                       const uint8_t* b_scales, const int32_t* sizes, int32_t groups,
                       int64_t height, int64_t n, int64_t k, int64_t rows,
                       const uint16_t* weights, const bux_ffn* ffn, uint16_t* projected, uint8_t* values, uint8_t* scales, uint8_t* t_values,
                       uint8_t* t_scales, void* workspace, size_t workspace_bytes, void* stream);
size_t bux_glu_backward_quantize_workspace_size(int64_t m, int64_t f);
int bux_glu_backward_quantize(const uint16_t* projected, const uint16_t* weights,
                              const uint16_t* dh, const int32_t* filled, int64_t m, int64_t f,
                              const bux_ffn* ffn, int64_t height,
                              uint16_t* d_projected, uint8_t* values, uint8_t* scales,
                              uint8_t* t_values, uint8_t* t_scales, uint16_t* d_weights,
                              void* workspace, size_t workspace_bytes, void* stream);
int bux_glu_backward_quantize_f32(const float* projected, const float* weights, const float* dh,
                                  const int32_t* filled, int64_t m, int64_t f,
                                  const bux_ffn* ffn, int64_t height, float* d_projected,
                                  uint8_t* values, uint8_t* scales, uint8_t* t_values,
                                  uint8_t* t_scales, float* d_weights, void* workspace,
                                  size_t workspace_bytes, void* stream);
/* bux_mx_grouped_dglu: the experts' down dgrad with the activation's gradient and both
 *   MXFP8 copies of d projected in its epilogue, the reference's fused dgrad
 *   (grouped_cudnn.activation_grad, src/bux/architecture/experts/grouped_cudnn.py:
 *   211-263), but for groups as they lie. The same outputs, bit for bit, as
 *   bux_mx_grouped_rows(a, b, sizes, m = height, f, k, height = rows) into dh, then
 *   bux_glu_backward_quantize(projected, weights, dh, filled = sum(sizes), rows, f, ...,
 *   height); dh never goes to memory:
 *   a_values/a_scales  dy in MXFP8 along its rows, tiled, height rows of k bytes;
 *   b_values/b_scales  each expert's (f, k) down kernel along k, tiled; f a multiple
 *     of 32;
 *   projected  bfloat16 [rows, 2 f]: the up GEMM's product, (up, gate) pairs;
 *   weights    bfloat16 [rows]: each row's weight;
 *   d_projected  NULL, or bfloat16 [rows, 2 f] to store d projected as well;
 *   values/scales  d projected along its columns (K = 2 f rounded up to 128), height
 *     rows; t_values/t_scales  along the rows (K = height), 2 f rows;
 *   d_weights  bfloat16 [rows]: each row's weight's gradient (0 past sum(sizes));
 *   workspace  bux_mx_grouped_dglu_workspace_size(groups, height, rows, f) bytes.
 *   ffn: as bux_mx_grouped_glu's.
 */
size_t bux_mx_grouped_dglu_workspace_size(int32_t groups, int64_t height, int64_t rows, int64_t f);
int bux_mx_grouped_dglu(const uint8_t* a_values, const uint8_t* a_scales, const uint8_t* b_values,
                        const uint8_t* b_scales, const int32_t* sizes, int32_t groups,
                        int64_t height, int64_t f, int64_t k, int64_t rows,
                        const uint16_t* projected, const uint16_t* weights, const bux_ffn* ffn,
                        uint16_t* d_projected, uint8_t* values, uint8_t* scales,
                        uint8_t* t_values, uint8_t* t_scales, uint16_t* d_weights,
                        void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------------
 * The router (the path's feed: its picks are a-1's idx, its weights a-8's).
 *
 * Replaces MoE._route (src/bux/architecture/experts/moe.py:236-273) off training, with
 * MoE._logits (:275-284) and _limit_groups (:474-483):
 *   logits = (x @ kernel + bias) * logit_scale: x bfloat16 [t, d], kernel bfloat16
 *     [d, n_logits] (the router's nnx kernel, [in, out]), bias float32 [n_logits] or
 *     NULL; products exact, sums in float32 (MFMA);
 *   scores = softmax over all n_logits logits | sigmoid | sqrt(softplus), float32;
 *   the first `scored` are the experts' (routed and zero experts), the rest sinks;
 *   choice = scores[:scored] + choice_bias (float32 [scored] or NULL: the aux-free
 *     bias), at -inf outside the `keep` best of `groups` equal groups (a group scored by
 *     the sum of its two best choices, one if it holds one);
 *   idx = the k largest choices, the largest first, ties to the lower index;
 *   weights = the picked scores, and sinks = the sinks' scores, each divided by the
 *     picked scores' sum plus the sinks' sum (float32, in order) if normalize; both
 *     rounded to bfloat16, then times scaling rounded to bfloat16, the product rounded
 *     to bfloat16 (a python float times a bfloat16 array in jax).
 * Outputs: idx int32 [t, k]; weights bfloat16 [t, k]; sinks bfloat16 [t, n_logits -
 * scored] (NULL when there are none); scores float32 [t, scored] and logits float32
 * [t, n_logits], each NULL to skip. n_logits <= 1024, k <= 16, keep <= 16, groups <= 64
 * and dividing scored, d a multiple of 16. workspace: bux_route_workspace_size(d,
 * n_logits) bytes (the kernel transposed).
 */
enum { BUX_ROUTER_SOFTMAX = 0, BUX_ROUTER_SIGMOID = 1, BUX_ROUTER_SQRTSOFTPLUS = 2 };
size_t bux_route_workspace_size(int64_t d, int32_t n_logits);
int bux_route(const uint16_t* x, const uint16_t* kernel, const float* bias, int64_t t, int64_t d,
              int32_t n_logits, float logit_scale, int router, int32_t scored,
              const float* choice_bias, int32_t groups, int32_t keep, int32_t k, int normalize,
              float scaling, int32_t* idx, uint16_t* weights, uint16_t* sinks, float* scores,
              float* logits, void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------------
 * MXFP8 rows of bytes: what an expert-parallel dispatch in MXFP8 sends a token.
 *
 * bux_mx_pack_rows replaces parallel/experts._in_mxfp8 (src/bux/parallel/experts.py:
 * 659-663) = blockscaled.mx_packed(mx_quantize(z)) (src/bux/architecture/precision/
 * blockscaled.py:372-375, 312-314) with the pick of each sent row, _in_mxfp8(z)[order
 * // k] (experts.py:624): packed[i] (d + d/32 bytes: the E4M3 codes of the row
 * quantized in blocks of 32 along d, then its d/32 E8M0 scale bytes) of x[index[i] /
 * index_div] (x[i] with index NULL), i < m; x bfloat16 [n, d]. A source row outside
 * [0, n), or a negative index, packs as zeros.
 * bux_mx_unpack_rows replaces parallel/experts._from_mxfp8 (experts.py:666-672) =
 * dequantized(mx_unpacked(packed, d)).astype(bfloat16) (blockscaled.py:223-229,
 * 378-380): out[i][j] = code * 2^(scale byte - 127) in float32, rounded to bfloat16
 * (exact for products in bfloat16's normal range).
 * d a multiple of 32.
 */
int bux_mx_pack_rows(const uint16_t* x, const int32_t* index, int32_t index_div, int64_t n,
                     int64_t m, int64_t d, uint8_t* packed, void* stream);
int bux_mx_unpack_rows(const uint8_t* packed, int64_t m, int64_t d, uint16_t* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* BUX_AMD_H */
