"""MXFP8 grouped GEMMs of an MoE's experts, and the quantizer that feeds them, on
MI355X: the HIP library's entry points over torch tensors.

Mirrors, with the same argument meanings:

- `quantized_twice`: ``grouped_triton.quantized_twice``
  (src/bux/architecture/experts/grouped_triton.py:44-101), the semantics of
  ``blockscaled.mx_twice`` (src/bux/architecture/precision/blockscaled.py:282-356);
- `rows`: ``grouped_mxfp8.rows`` (src/bux/architecture/experts/grouped_mxfp8.py:116-154);
- `contract`: ``grouped_mxfp8.contract`` (grouped_mxfp8.py:185-210);
- `activated`: ``grouped_cudnn.activated`` (grouped_cudnn.py:161-205), the up GEMM with
  the activation and h's two MXFP8 copies in its epilogue.

Operands are `Tiled`: a matrix's MXFP8 blocks along its rows (the reference's
``Blocks``, src/bux/architecture/precision/blockscaled.py:43-56) in the layout the
GEMMs load, as the reference's ``Tiled`` (grouped_mxfp8.py:93-103) is for its kernels:
K (the row length) padded to whole 128s with codes 0 and scale bytes 1, E4M3 codes
(..., K/64, r, 64) and E8M0 scale bytes (..., K/128, r, 4). `tiled` and `canonical`
convert from and to the row-major ``Blocks`` layout (codes (..., r, c), scale bytes
(..., r, c/32)).
"""

import ctypes
from typing import NamedTuple

import torch

from bux_amd import _lib
from bux_amd.kernels import lib, ptr, require, stream, workspace

LANES = 128  # rows of the activations' copies: padded to whole tiles of them
K_ALIGN = 128  # the tiled layout's K: whole 128s


class Tiled(NamedTuple):
    """A matrix (or a stack of them) in MXFP8 along its rows, tiled.

    Row i's code j is ``values[..., j // 64, i, j % 64]`` and its block b's scale byte
    ``scales[..., b // 4, i, b % 4]``; codes past the matrix's columns are 0 and their
    scale bytes 1."""

    values: torch.Tensor  # uint8 (..., K/64, r, 64): E4M3 codes
    scales: torch.Tensor  # uint8 (..., K/128, r, 4): E8M0 biased exponents

    @property
    def height(self) -> int:
        """The matrix's rows."""
        return self.values.shape[-2]

    @property
    def k(self) -> int:
        """The padded row length, a multiple of 128."""
        return self.values.shape[-3] * 64


def whole(rows: int, tile: int = LANES) -> int:
    """Return `rows` rounded up to whole tiles (grouped_blockscaled.py:122-124)."""
    return -(-rows // tile) * tile


def _swap_last_but_one(x: torch.Tensor, lead: int) -> torch.Tensor:
    """Swap the two axes before the last, after `lead` leading axes."""
    return x.permute(*range(lead), lead + 1, lead, lead + 2)


def tiled(values: torch.Tensor, scales: torch.Tensor) -> Tiled:
    """Return row-major blocks (codes (..., r, c), scale bytes (..., r, c/32)) tiled."""
    *lead, r, c = values.shape
    kp = whole(c, K_ALIGN)
    v = torch.zeros(*lead, r, kp, dtype=torch.uint8, device=values.device)
    v[..., :c] = values
    sc = torch.ones(*lead, r, kp // 32, dtype=torch.uint8, device=values.device)
    sc[..., :c // 32] = scales
    n = len(lead)
    v = _swap_last_but_one(v.reshape(*lead, r, kp // 64, 64), n).contiguous()
    sc = _swap_last_but_one(sc.reshape(*lead, r, kp // 128, 4), n).contiguous()
    return Tiled(v, sc)


def canonical(t: Tiled, cols: int) -> tuple[torch.Tensor, torch.Tensor]:
    """Return tiled blocks row-major: codes (..., r, cols), scale bytes (..., r, cols/32)."""
    *lead, chunks, r, _ = t.values.shape
    n = len(lead)
    v = _swap_last_but_one(t.values, n).reshape(*lead, r, chunks * 64)
    sc = _swap_last_but_one(t.scales, n).reshape(*lead, r, chunks * 2)
    return v[..., :cols].contiguous(), sc[..., :cols // 32].contiguous()


def quantized_twice(
    x: torch.Tensor,
    filled: torch.Tensor | None = None,
    columns: bool = True,
    index: torch.Tensor | None = None,
    index_div: int = 1,
    height: int | None = None,
    rows: bool = True,
    tiles: bool = False,
    halves: bool = False,
) -> tuple[Tiled | None, Tiled | None]:
    """Return x in MXFP8 along its rows and, if `columns`, x^T along its rows, in one
    pass over x, both tiled; with `tiles`, a scale per 32 x 32 tile shared by both
    (``blockscaled.mx_tiles_twice``, blockscaled.py:294-309: the mxfp8_2d recipe's W).

    Args:
        x: bfloat16 or float32, a matrix (r, c) or a stack (g, r, c); with `index`, the
            matrix the rows are read from. c is a multiple of 32. (float32: the
            reference quantizes any float dtype alike, in float32, blockscaled.py:323-343.)
        filled: a device int32 (one element): rows from it on quantize as 0; None
            for every row.
        columns: whether to return x^T too.
        index: int32 (m,): row i is ``x[index[i] // index_div]``, 0 where the index
            is negative or that row lies past x's (the reference's ``Picked`` rows,
            ``tokens[order // k]``).
        index_div: the divisor of `index` (k, the picks a token).
        height: rows of the copies, a multiple of 32 (rows past x's are 0); None for
            x's (the index's) rows rounded up to 32.
        rows: whether to return the copy along the rows (False: None in its place).
        halves: x's columns are a GLU's (up, gate) pairs, read as its halves: in each
            64 columns the 32 pairs' gates, then their ups (the reference's `halves`,
            grouped_triton.py:49, grouped_cudnn.halves_of); c a multiple of 64.

    Returns:
        (x along rows, x^T along rows): `height` rows of K = c padded to 128, and c
        rows of K = height padded to 128 (a stack of g of each for a stack).
    """
    require(x, filled, index)
    if x.dtype not in (torch.bfloat16, torch.float32):
        raise TypeError(f"quantized_twice takes bfloat16 or float32, got {x.dtype}")
    if not isinstance(tiles, bool):
        raise TypeError(f"quantized_twice: tiles is a bool (the mxfp8_2d recipe's scales), "
                        f"not {type(tiles).__name__}")
    stack = x.dim() == 3
    if index is not None:
        if stack:
            raise ValueError("an index reads rows of one matrix")
        if index.dtype != torch.int32:
            raise TypeError("the index is int32")
        groups, r, c = 1, index.shape[0], x.shape[-1]
    else:
        groups, r, c = (x.shape if stack else (1, *x.shape))
    h = whole(r, 32) if height is None else height
    dev = x.device
    lead = (groups,) if stack else ()
    vals = scales = t_vals = t_scales = None
    flags = 0
    if rows:
        flags |= _lib.MX_ROWS
        kc = whole(c, K_ALIGN)
        vals = torch.empty(*lead, kc // 64, h, 64, dtype=torch.uint8, device=dev)
        scales = torch.empty(*lead, kc // 128, h, 4, dtype=torch.uint8, device=dev)
    if columns:
        flags |= _lib.MX_COLUMNS
        kh = whole(h, K_ALIGN)
        t_vals = torch.empty(*lead, kh // 64, c, 64, dtype=torch.uint8, device=dev)
        t_scales = torch.empty(*lead, kh // 128, c, 4, dtype=torch.uint8, device=dev)
    if tiles:
        flags |= _lib.MX_TILES
    if halves:
        flags |= _lib.MX_HALVES
    quantize = lib().bux_mx_quantize if x.dtype == torch.bfloat16 else lib().bux_mx_quantize_f32
    _lib.check(quantize(
        ptr(x), ptr(index), index_div, x.shape[0] if index is not None else 0, groups, r, c, h,
        ptr(filled), flags,
        ptr(vals), ptr(scales), ptr(t_vals), ptr(t_scales), stream()))
    along_rows = Tiled(vals, scales) if rows else None
    along_columns = Tiled(t_vals, t_scales) if columns else None
    return along_rows, along_columns


_DTYPES = {torch.bfloat16: _lib.BF16, torch.float32: _lib.F32}


class TileList(NamedTuple):
    """A rows GEMM's group starts and ragged tile list, made once on the device from the
    group sizes (the reference's ``tiles_of``, grouped_mxfp8.py:157-182) for every GEMM of
    a step that takes the same sizes."""

    buffer: torch.Tensor  # uint8: a header of the dimensions, the starts, the tile records
    groups: int
    m: int  # rows of the rows GEMMs' a
    height: int  # rows of their outputs


def tiles_of(sizes: torch.Tensor, m: int, height: int) -> TileList:
    """Return the tile list of `sizes` (int32 (g,) on the device) for rows GEMMs of a with
    m rows into outputs of `height` rows; `contract` takes it too (its starts)."""
    require(sizes)
    if sizes.dtype != torch.int32 or sizes.dim() != 1:
        raise ValueError(f"tiles_of: sizes {tuple(sizes.shape)} {sizes.dtype}")
    groups = sizes.shape[0]
    buf = workspace(lib().bux_mx_grouped_rows_workspace_size(groups, m, height), sizes.device)
    _lib.check(lib().bux_mx_grouped_tiles(ptr(sizes), groups, m, height, ptr(buf), buf.numel(),
                                          stream()))
    return TileList(buf, groups, m, height)


def rows(
    a: Tiled, b: Tiled, sizes: torch.Tensor, out: torch.dtype = torch.bfloat16,
    height: int | None = None, tiles: TileList | None = None, starts: torch.Tensor | None = None,
) -> torch.Tensor:
    """Return ``a @ b[g]^T`` for each group g's rows of a, (height, n), the rows past
    the groups 0.

    Args:
        a: the rows (m of K), group 0's first.
        b: the groups' matrices, a stack (g of n rows of K).
        sizes: int32 (g,) on the device: how many rows each group has.
        out: the output's dtype, bfloat16 or float32.
        height: rows of the output (a's rows past it are not stored); None for m.
        tiles: `tiles_of(sizes, m, height)`, made once for the step's GEMMs; None to make
            it here.
        starts: int32 (g,) on the device: where each group's rows of a start (the
            reference's `starts`, grouped_mxfp8.py:116-154); None for packed. y's rows
            stay packed either way.
    """
    require(a.values, a.scales, b.values, b.scales, sizes)
    if a.values.dim() != 3 or b.values.dim() != 4:
        raise ValueError(f"rows: a {tuple(a.values.shape)} is not one matrix or "
                         f"b {tuple(b.values.shape)} not a stack")
    m, k = a.height, a.k
    groups, n = b.values.shape[0], b.height
    if b.k != k or sizes.shape != (groups,) or sizes.dtype != torch.int32:
        raise ValueError(f"rows: a {tuple(a.values.shape)}, b {tuple(b.values.shape)}, "
                         f"sizes {tuple(sizes.shape)} {sizes.dtype}")
    h = m if height is None else height
    y = torch.empty(h, n, dtype=out, device=a.values.device)
    if starts is not None:
        require(starts)
        if starts.shape != (groups,) or starts.dtype != torch.int32 or tiles is not None:
            raise ValueError(f"rows: starts int32 ({groups},), without a tile list, not "
                             f"{starts.dtype} {tuple(starts.shape)}")
        ws = workspace(lib().bux_mx_grouped_rows_workspace_size(groups, m, h), y.device)
        _lib.check(lib().bux_mx_grouped_rows_started(
            ptr(a.values), ptr(a.scales), ptr(b.values), ptr(b.scales), ptr(sizes), ptr(starts),
            groups, m, n, k, h, _DTYPES[out], ptr(y), ptr(ws), ws.numel(), stream()))
        return y
    if tiles is not None:
        if (tiles.groups, tiles.m, tiles.height) != (groups, m, h):
            raise ValueError(f"rows: a tile list for {tiles.groups} groups, m={tiles.m}, "
                             f"height={tiles.height}, not {groups}, {m}, {h}")
        _lib.check(lib().bux_mx_grouped_rows_listed(
            ptr(a.values), ptr(a.scales), ptr(b.values), ptr(b.scales), ptr(tiles.buffer),
            tiles.buffer.numel(), groups, m, n, k, h, _DTYPES[out], ptr(y), stream()))
        return y
    ws = workspace(lib().bux_mx_grouped_rows_workspace_size(groups, m, h), y.device)
    _lib.check(lib().bux_mx_grouped_rows(
        ptr(a.values), ptr(a.scales), ptr(b.values), ptr(b.scales), ptr(sizes), groups, m, n, k,
        h, _DTYPES[out], ptr(y), ptr(ws), ws.numel(), stream()))
    return y


def activated(
    a: Tiled, b: Tiled, sizes: torch.Tensor, weights: torch.Tensor, ffn: _lib.FfnStruct,
    rows: int,
) -> tuple[torch.Tensor, Tiled, Tiled]:
    """Return the up GEMM's product ``a @ b[g]^T`` (rows, n) and h, its activation times
    each row's weight, in MXFP8 along its units and, as h^T, along the rows: the
    reference's ``grouped_cudnn.activated`` (grouped_cudnn.py:161-205), for groups as they
    lie. The same bits as `rows` followed by the activation's quantizer.

    Args:
        a: the rows (height of K), group 0's first: its height is the copies'.
        b: the groups' up kernels (g, n, K), columns in (up, gate) pairs.
        sizes: int32 (g,) on the device.
        weights: bfloat16 (rows,): each row's weight.
        ffn: the activation as ``moe.Ffn.struct`` gives it: gated, of swish,
            quick_gelu or situ.
        rows: rows of the product (at most a's height).
    """
    require(a.values, a.scales, b.values, b.scales, sizes, weights)
    if a.values.dim() != 3 or b.values.dim() != 4:
        raise ValueError(f"activated: a {tuple(a.values.shape)} is not one matrix or "
                         f"b {tuple(b.values.shape)} not a stack")
    height, k = a.height, a.k
    groups, n = b.values.shape[0], b.height
    if b.k != k or sizes.shape != (groups,) or sizes.dtype != torch.int32:
        raise ValueError(f"activated: a {tuple(a.values.shape)}, b {tuple(b.values.shape)}, "
                         f"sizes {tuple(sizes.shape)} {sizes.dtype}")
    if weights.dtype != torch.bfloat16 or weights.numel() < rows:
        raise ValueError(f"activated: weights {weights.dtype} of {weights.numel()} for {rows} rows")
    f = n // 2
    dev = a.values.device
    kf = whole(f, K_ALIGN)
    projected = torch.empty(rows, n, dtype=torch.bfloat16, device=dev)
    vals = torch.empty(kf // 64, height, 64, dtype=torch.uint8, device=dev)
    scales = torch.empty(kf // 128, height, 4, dtype=torch.uint8, device=dev)
    t_vals = torch.empty(height // 64, f, 64, dtype=torch.uint8, device=dev)
    t_scales = torch.empty(height // 128, f, 4, dtype=torch.uint8, device=dev)
    ws = workspace(lib().bux_mx_grouped_glu_workspace_size(groups, height), dev)
    _lib.check(lib().bux_mx_grouped_glu(
        ptr(a.values), ptr(a.scales), ptr(b.values), ptr(b.scales), ptr(sizes), groups, height, n,
        k, rows, ptr(weights.contiguous()), ctypes.byref(ffn), ptr(projected), ptr(vals),
        ptr(scales), ptr(t_vals), ptr(t_scales), ptr(ws), ws.numel(), stream()))
    return projected, Tiled(vals, scales), Tiled(t_vals, t_scales)


def activation_grad(
    a: Tiled, b: Tiled, sizes: torch.Tensor, projected: torch.Tensor, weights: torch.Tensor,
    ffn: _lib.FfnStruct, rows: int, keep: bool = False,
) -> tuple[Tiled, Tiled, torch.Tensor, torch.Tensor | None]:
    """Return the gradient of `activated`'s product (d projected) in MXFP8 along its
    columns and, transposed, along the rows, each row's weight's gradient, and with
    `keep` d projected in bfloat16: the down dgrad ``a @ b[g]^T`` (dh, which never goes
    to memory) through the activation's gradient, the reference's
    ``grouped_cudnn.activation_grad`` (grouped_cudnn.py:211-263), for groups as they lie.
    The same bits as `rows` followed by the activation's quantizing backward
    (``moe.weighted_units_backward_quantized``).

    Args:
        a: dy along d (height of K), group 0's first: its height is the copies'.
        b: the groups' down kernels along d, (g, f, K).
        sizes: int32 (g,) on the device.
        projected: bfloat16 (rows, 2 f): the up GEMM's product, (up, gate) pairs.
        weights: bfloat16 (rows,): each row's weight.
        ffn: the activation as ``moe.Ffn.struct`` gives it: gated, of swish,
            quick_gelu or situ.
        rows: rows of the product (at most a's height).
    """
    require(a.values, a.scales, b.values, b.scales, sizes, projected, weights)
    if a.values.dim() != 3 or b.values.dim() != 4:
        raise ValueError(f"activation_grad: a {tuple(a.values.shape)} is not one matrix or "
                         f"b {tuple(b.values.shape)} not a stack")
    height, k = a.height, a.k
    groups, f = b.values.shape[0], b.height
    if b.k != k or sizes.shape != (groups,) or sizes.dtype != torch.int32:
        raise ValueError(f"activation_grad: a {tuple(a.values.shape)}, b {tuple(b.values.shape)}, "
                         f"sizes {tuple(sizes.shape)} {sizes.dtype}")
    if (projected.dtype != torch.bfloat16 or projected.shape != (rows, 2 * f)
            or not projected.is_contiguous()):
        raise ValueError(f"activation_grad: projected {projected.dtype} {tuple(projected.shape)} "
                         f"is not a contiguous bfloat16 ({rows}, {2 * f})")
    if weights.dtype != torch.bfloat16 or weights.numel() < rows:
        raise ValueError(f"activation_grad: weights {weights.dtype} of {weights.numel()} for {rows} rows")
    dev = a.values.device
    n2 = 2 * f
    k2 = whole(n2, K_ALIGN)
    vals = torch.empty(k2 // 64, height, 64, dtype=torch.uint8, device=dev)
    scales = torch.empty(k2 // 128, height, 4, dtype=torch.uint8, device=dev)
    t_vals = torch.empty(height // 64, n2, 64, dtype=torch.uint8, device=dev)
    t_scales = torch.empty(height // 128, n2, 4, dtype=torch.uint8, device=dev)
    dw = torch.empty(rows, dtype=torch.bfloat16, device=dev)
    dp = torch.empty(rows, n2, dtype=torch.bfloat16, device=dev) if keep else None
    ws = workspace(lib().bux_mx_grouped_dglu_workspace_size(groups, height, rows, f), dev)
    _lib.check(lib().bux_mx_grouped_dglu(
        ptr(a.values), ptr(a.scales), ptr(b.values), ptr(b.scales), ptr(sizes), groups, height, f,
        k, rows, ptr(projected), ptr(weights.contiguous()), ctypes.byref(ffn), ptr(dp), ptr(vals),
        ptr(scales), ptr(t_vals), ptr(t_scales), ptr(dw), ptr(ws), ws.numel(), stream()))
    return Tiled(vals, scales), Tiled(t_vals, t_scales), dw, dp


def contract(
    a: Tiled, b: Tiled, sizes: torch.Tensor, out: torch.dtype = torch.bfloat16,
    tiles: TileList | None = None,
) -> torch.Tensor:
    """Return ``a[:, rows of g] b[:, rows of g]^T`` for each group g, (g, d, f).

    Args:
        a: x^T (d rows of m) in MXFP8 along m.
        b: dy^T (f rows of m) in MXFP8 along m.
        sizes: int32 (g,) on the device, summing to at most m.
        out: the output's dtype.
        tiles: a `tiles_of` list of the same sizes (its group starts); None to compute
            the starts here.
    """
    require(a.values, a.scales, b.values, b.scales, sizes)
    if a.values.dim() != 3 or b.values.dim() != 3:
        raise ValueError(f"contract: a {tuple(a.values.shape)}, b {tuple(b.values.shape)}")
    d, m = a.height, a.k
    f = b.height
    groups = sizes.shape[0]
    if b.k != m or sizes.dtype != torch.int32:
        raise ValueError(f"contract: a {tuple(a.values.shape)}, b {tuple(b.values.shape)}")
    dw = torch.empty(groups, d, f, dtype=out, device=a.values.device)
    if tiles is not None:
        if tiles.groups != groups:
            raise ValueError(f"contract: a tile list for {tiles.groups} groups, not {groups}")
        _lib.check(lib().bux_mx_grouped_contract_listed(
            ptr(a.values), ptr(a.scales), ptr(b.values), ptr(b.scales), ptr(tiles.buffer),
            tiles.buffer.numel(), groups, d, f, m, _DTYPES[out], ptr(dw), stream()))
        return dw
    ws = workspace(lib().bux_mx_grouped_contract_workspace_size(groups), dw.device)
    _lib.check(lib().bux_mx_grouped_contract(
        ptr(a.values), ptr(a.scales), ptr(b.values), ptr(b.scales), ptr(sizes), groups, d, f, m,
        _DTYPES[out], ptr(dw), ptr(ws), ws.numel(), stream()))
    return dw
