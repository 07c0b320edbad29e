"""MXFP8 1x32 block-scaled quantization and dequantization, restated from bux.
TEST INFRASTRUCTURE ONLY (see `oracle`).

The spec (``src/bux/architecture/precision/blockscaled.py:323-356``), per block b of 32
values along the axis a GEMM contracts, x widened to float32 first (``:314``):

- ``amax = max|b|``;
- ``e = ceil_log2(amax / 448)``: the float32 quotient's bits, ``(bits >> 23) +
  (mantissa != 0) - 127``, clipped to [-126, 126] (``:346-351``);
- the scale byte is ``e + 127`` (E8M0's bits), 1..253; a block of zeros gets 1;
- each value is ``clip(v * 2^-e, -448, 448)`` rounded to nearest even E4M3 (OCP
  ``float8_e4m3fn``), a negative value that rounds to 0 giving 0x80 (``:340-342``).

Which copies the path makes (``grouped_blockscaled.py:181-184,206-208,296-317``): an
operand along its rows and its transpose along its rows (the original's columns), rows
from ``filled`` on as 0 first; a stack of matrices (each expert's W) one matrix at a
time.

Pins, run by ``tests/test_oracle.py``:

- `to_e4m3fn`: exhaustive over every finite bfloat16 value in [-448, 448] against
  torch's own ``float8_e4m3fn`` cast (an independent RNE implementation), and against
  a brute-force nearest-even search over the 254 finite codes;
- `ceil_log2`: exhaustive over every positive finite bfloat16 divided by 448, against
  ``math.ceil(math.log2(q))`` computed in exact rational arithmetic
  (``fractions.Fraction``), clipped;
- `in_e4m3`: the reference's invariants: a block of zeros gives byte 1; every scaled
  value lands within [-448, 448]; the scale is the least power of two doing so
  (brute force over exponents on random blocks); dequantization is within half an E4M3
  ulp of each value;
- `dequantized`: closed form ``value * 2^(byte - 127)`` checked against torch's
  ``float8_e4m3fn`` -> float32 cast for all 256 codes, and `e8m0_values` against
  torch's ``float8_e8m0fnu`` -> float32 cast for all 256 bytes;
- `mx_tiles_twice` (32 x 32 tiles): each tile's scale the least power of two that fits
  its largest magnitude (brute force over exponents), both copies the same codes
  transposed, and a matrix whose tiles each hold one magnitude quantizing as the 1 x 32
  blocks do;
- `mx_packed` / `mx_unpacked` / `in_mxfp8` / `from_mxfp8` (the expert-parallel
  dispatch's rows of bytes, parallel/experts.py:659-672): the reference's round trip
  (tests/test_precision.py:344-352: 8 x 64 rows pack to 66 bytes and unpack to the
  same values), and ``from_mxfp8`` exact (E4M3 codes through torch's float8 cast,
  times the scale, equal to the bfloat16 result).
"""

from typing import NamedTuple

import numpy as np

from oracle import bf16

E4M3_MAX = 448.0  # blockscaled.py:40
MX_BLOCK = 32  # blockscaled.py:277


class Blocks(NamedTuple):
    """An (r, c) matrix in MXFP8 along its rows (blockscaled.py:43-52): E4M3 codes
    (uint8, r x c) and E8M0 scale bytes (uint8, r x c/32). The canonical layout every
    bit-exact comparison uses."""

    values: np.ndarray
    scales: np.ndarray


def ceil_log2(x: np.ndarray) -> np.ndarray:
    """Return the least e with 2^e >= x (x >= 0, float32) from x's bits, clipped to
    [-126, 126] (blockscaled.py:346-351)."""
    bits = np.ascontiguousarray(x, np.float32).view(np.uint32)
    exponent = (bits >> 23).astype(np.int32) + ((bits & 0x7FFFFF) != 0)
    return np.clip(exponent - 127, -126, 126).astype(np.int32)


def power_of_two(e: np.ndarray) -> np.ndarray:
    """Return 2^e exactly for integers e in [-126, 127] (blockscaled.py:354-356)."""
    return ((np.asarray(e, np.int32) + 127).astype(np.uint32) << 23).view(np.float32)


def to_e4m3fn(x: np.ndarray) -> np.ndarray:
    """Return float32 values rounded to nearest even OCP E4M3 (float8_e4m3fn), as
    codes: 3 mantissa bits, bias 7, subnormals 2^-9 apart, no inf; overflow past the
    rounding range and NaN give 0x7F with the sign (ml_dtypes' non-saturating cast,
    which the path never reaches after its clip to +-448)."""
    x = np.asarray(x, np.float32)
    sign = np.signbit(x).astype(np.uint8) << 7
    a = np.abs(x).astype(np.float64)
    _, p = np.frexp(a)
    e = np.maximum(p - 1, -6)  # below 2^-6 the spacing is the subnormals' 2^-9
    quantum = np.ldexp(1.0, e - 3)
    q = np.rint(a / quantum) * quantum  # exact in float64; rint ties to even
    _, p2 = np.frexp(q)
    e2 = p2 - 1
    normal = q >= 2.0**-6
    with np.errstate(invalid="ignore", over="ignore"):
        mant = np.where(normal, q / np.ldexp(1.0, e2) * 8 - 8, 0)
        code = np.where(normal, ((e2 + 7) << 3) + mant, q / 2.0**-9)
    code = np.where(np.isnan(x) | (q > E4M3_MAX), 0x7F, code)
    return code.astype(np.uint8) | sign


_E4M3 = None


def e4m3_values() -> np.ndarray:
    """Return the float32 value of each of the 256 E4M3 codes (NaN at 0x7F, 0xFF)."""
    global _E4M3
    if _E4M3 is None:
        codes = np.arange(256)
        s, e, m = codes >> 7, (codes >> 3) & 15, codes & 7
        v = np.where(e == 0, np.ldexp(m.astype(np.float64), -9),
                     np.ldexp((8 + m).astype(np.float64), e - 10))
        v = np.where((e == 15) & (m == 7), np.nan, v)
        _E4M3 = np.where(s == 1, -v, v).astype(np.float32)
    return _E4M3


def in_e4m3(x: np.ndarray, blocks: str = "rows") -> tuple[np.ndarray, np.ndarray]:
    """Return x's (float32, r x c) E4M3 codes and its scales' biased exponents, in
    blocks of 32 along its ``rows``, down its ``columns`` or in 32 x 32 ``tiles``
    (blockscaled.py:323-343)."""
    x = np.asarray(x, np.float32)
    (r, c), b = x.shape, MX_BLOCK
    shape, axes = {
        "rows": ((r, c // b, b), (2,)),
        "columns": ((r // b, b, c), (1,)),
        "tiles": ((r // b, b, c // b, b), (1, 3)),
    }[blocks]
    blocked = x.reshape(shape)
    largest = np.abs(blocked).max(axis=axes).astype(np.float32)
    exponent = ceil_log2(largest / np.float32(E4M3_MAX))
    down = power_of_two(-exponent)
    scaled = blocked * np.expand_dims(down, axes)
    values = to_e4m3fn(np.clip(scaled, -E4M3_MAX, E4M3_MAX))
    return values.reshape(r, c), (exponent + 127).astype(np.uint8)


def mx_quantize(x: np.ndarray) -> Blocks:
    """Return x (float32, or bfloat16 bits as uint16) in MXFP8 along its rows
    (blockscaled.py:312-314)."""
    if x.dtype == np.uint16:
        x = bf16.to_f32(x)
    return Blocks(*in_e4m3(x, "rows"))


def mx_tiles_twice(w: np.ndarray) -> tuple[Blocks, Blocks]:
    """Return W and W^T in MXFP8 with a scale per 32 x 32 tile, each copy's blocks of 32
    along its rows taking its tile's scale, so that both hold the same codes
    (blockscaled.py:294-309, the mxfp8_2d recipe's weights)."""
    if w.dtype == np.uint16:
        w = bf16.to_f32(w)
    values, exponents = in_e4m3(w, "tiles")
    rows = np.repeat(exponents, MX_BLOCK, axis=0)
    columns = np.repeat(exponents.T, MX_BLOCK, axis=0)
    return Blocks(values, rows), Blocks(np.ascontiguousarray(values.T), np.ascontiguousarray(columns))


def mx_twice(x: np.ndarray) -> tuple[Blocks, Blocks]:
    """Return x and x^T in MXFP8, each along its rows (blockscaled.py:282-291, the
    XLA branch)."""
    return mx_quantize(x), mx_quantize(np.ascontiguousarray(x.T))


def e8m0_values() -> np.ndarray:
    """Return the float32 value of each E8M0 byte (``float8_e8m0fnu``): 2^(byte - 127),
    byte 0 giving 2^-127 (a float32 subnormal) and 255 NaN."""
    table = np.ldexp(np.float64(1.0), np.arange(255) - 127).astype(np.float32)
    return np.append(table, np.float32(np.nan)).astype(np.float32)


def dequantized(blocks: Blocks) -> np.ndarray:
    """Return the float32 values MXFP8 blocks hold: each code's value times its
    block's scale, ``scales.astype(float32)`` of E8M0 bytes (blockscaled.py:223-229)."""
    values, scales = blocks
    block = values.shape[-1] // scales.shape[-1]
    scale = e8m0_values()[scales]
    with np.errstate(over="ignore", invalid="ignore"):  # past float32: inf, as float32 gives
        return e4m3_values()[values] * np.repeat(scale, block, axis=-1)


def mx_packed(blocks: Blocks) -> np.ndarray:
    """Return each row of `blocks` as one row of bytes, its c codes then its c/32 scale
    bytes (blockscaled.py:372-375)."""
    return np.concatenate([blocks.values, blocks.scales], axis=-1).astype(np.uint8)


def mx_unpacked(packed: np.ndarray, c: int) -> Blocks:
    """Return the blocks of rows of `c` values that `mx_packed` made
    (blockscaled.py:378-380)."""
    return Blocks(packed[:, :c].copy(), packed[:, c:].copy())


def in_mxfp8(z: np.ndarray) -> np.ndarray:
    """Return each token (bfloat16 bits, n x d) in MXFP8 as a row of d + d/32 bytes
    (parallel/experts.py:659-663)."""
    return mx_packed(mx_quantize(z))


def from_mxfp8(packed: np.ndarray, d: int) -> np.ndarray:
    """Return rows of `in_mxfp8` bytes dequantized, as bfloat16 bits
    (parallel/experts.py:666-672: float32, then ``astype`` the tokens' dtype)."""
    return bf16.to_bf16(dequantized(mx_unpacked(packed, d)))


def halves_of(pairs: np.ndarray) -> np.ndarray:
    """Where columns of (up, gate) pairs (unit u's up at 2u, its gate at 2u + 1) lie in a
    GLU's halves: each 32 units take 64 columns, their gates first, then their ups
    (grouped_cudnn.halves_of, grouped_cudnn.py:150-155)."""
    unit, gate = np.asarray(pairs) // 2, np.asarray(pairs) % 2
    return unit // 32 * 64 + (1 - gate) * 32 + unit % 32


def read_as_halves(c: int) -> np.ndarray:
    """The column of pairs that each of c columns in halves reads (the Triton
    quantizer's `read`, grouped_triton.py:216-219)."""
    cs = np.arange(c)
    return cs // 64 * 64 + cs % 32 * 2 + (cs % 64 < 32).astype(np.int64)


def quantized_twice(
    x: np.ndarray,
    filled: int,
    columns: bool = True,
    index: np.ndarray | None = None,
    height: int | None = None,
    tiles: bool = False,
    halves: bool = False,
) -> tuple[Blocks, Blocks | None]:
    """Return the MXFP8 copies a grouped GEMM's operand takes
    (grouped_blockscaled.py:296-317 off a Blackwell GPU; grouped_triton.py:44-101 for
    ``index``): x along its rows and, if `columns`, x^T along its rows; rows from
    `filled` on as 0.

    Args:
        x: bfloat16 bits (uint16) or float32, (r, c) or a stack (g, r, c).
        filled: the rows that hold values; those from it on quantize as 0.
        columns: whether to return x^T too.
        index: rows to read, ``x[index]``, a row at -1 reading 0 (the Triton
            kernel's meaning, grouped_triton.py:208-214); None for x itself.
        height: rows of the copies, padded by 0 past x's (``ragged_dot``'s padding to
            whole tiles of 128, grouped_blockscaled.py:122-128); None for x's own.
        tiles: a scale per 32 x 32 tile, shared by both copies (`mx_tiles_twice`).
        halves: x's columns, (up, gate) pairs, read as a GLU's halves (`read_as_halves`).

    Returns:
        The copies; a stack gives stacks (values (g, r, c) and (g, c, r)).
    """
    if x.dtype == np.uint16:
        x = bf16.to_f32(x)
    x = np.asarray(x, np.float32)
    if halves:
        x = x[..., read_as_halves(x.shape[-1])]
    if index is not None:
        index = np.asarray(index)
        rows = x[np.maximum(index, 0)]
        x = np.where((index >= 0)[:, None], rows, np.float32(0))
    stack = x if x.ndim == 3 else x[None]
    g, r, c = stack.shape
    h = r if height is None else height
    padded = np.zeros((g, h, c), np.float32)
    padded[:, :r] = stack
    kept = np.where((np.arange(h) < filled)[None, :, None], padded, np.float32(0))
    if tiles:
        both = [mx_tiles_twice(m) for m in kept]
        rows_out = [b[0] for b in both]
        cols_out = [b[1] for b in both] if columns else None
    else:
        rows_out = [mx_quantize(m) for m in kept]
        cols_out = [mx_quantize(np.ascontiguousarray(m.T)) for m in kept] if columns else None

    def stacked(parts: list[Blocks]) -> Blocks:
        if x.ndim == 2:
            return parts[0]
        return Blocks(np.stack([p.values for p in parts]), np.stack([p.scales for p in parts]))

    return stacked(rows_out), (stacked(cols_out) if columns else None)
