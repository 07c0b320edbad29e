"""MXFP8 grouped GEMMs of an MoE's experts, and the quantizer that feeds them, on
MI355X: the HIP library's entry points over torch tensors.

Mirrors, with the same argument meanings:

- `quantized_twice`: ``grouped_triton.quantized_twice``
  (src/bux/architecture/experts/grouped_triton.py:44-101), the semantics of
  ``blockscaled.mx_twice`` (src/bux/architecture/precision/blockscaled.py:282-356);
- `rows`: ``grouped_mxfp8.rows`` (src/bux/architecture/experts/grouped_mxfp8.py:116-154);
- `contract`: ``grouped_mxfp8.contract`` (grouped_mxfp8.py:185-210).

Operands are `Blocks` in the canonical layout (E4M3 codes (..., r, c) and E8M0 scale
bytes (..., r, c/32), row-major), which the kernels load as they are: the reference's
``Tiled`` (grouped_mxfp8.py:93-103) is a Blackwell tensor-memory layout with no
counterpart here.
"""

from typing import NamedTuple

import torch

from bux_amd import _lib
from bux_amd.kernels import lib, ptr, require, stream, workspace

LANES = 128  # rows a GEMM tile takes: copies are padded to whole tiles of them


class Blocks(NamedTuple):
    """A matrix (or a stack of them) in MXFP8 along its rows
    (src/bux/architecture/precision/blockscaled.py:43-56)."""

    values: torch.Tensor  # uint8 (..., r, c): E4M3 codes
    scales: torch.Tensor  # uint8 (..., r, c / 32): E8M0 biased exponents


def whole(rows: int, tile: int = LANES) -> int:
    """Return `rows` rounded up to whole tiles (grouped_blockscaled.py:122-124)."""
    return -(-rows // tile) * tile


def quantized_twice(
    x: torch.Tensor,
    filled: torch.Tensor | None = None,
    columns: bool = True,
    index: torch.Tensor | None = None,
    index_div: int = 1,
    height: int | None = None,
    rows: bool = True,
) -> tuple[Blocks | None, Blocks | None]:
    """Return x in MXFP8 along its rows and, if `columns`, x^T along its rows, in one
    pass over x.

    Args:
        x: bfloat16, a matrix (r, c) or a stack (g, r, c); with `index`, the matrix
            the rows are read from.
        filled: a device int32 (one element): rows from it on quantize as 0; None
            for every row.
        columns: whether to return x^T too.
        index: int32 (m,): row i is ``x[index[i] // index_div]``, 0 where the index
            is negative (the reference's ``Picked`` rows, ``tokens[order // k]``).
        index_div: the divisor of `index` (k, the picks a token).
        height: rows of the copies, a multiple of 32 (rows past x's are 0); None for
            x's (the index's) rows rounded up to 32.
        rows: whether to return the copy along the rows (False: None in its place).

    Returns:
        (x along rows, x^T along rows): stacks (g, height, c) and (g, c, height) for a
        stack.
    """
    require(x, filled, index)
    if x.dtype != torch.bfloat16:
        raise TypeError(f"quantized_twice takes bfloat16, got {x.dtype}")
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
        vals = torch.empty(*lead, h, c, dtype=torch.uint8, device=dev)
        scales = torch.empty(*lead, h, c // 32, dtype=torch.uint8, device=dev)
    if columns:
        flags |= _lib.MX_COLUMNS
        t_vals = torch.empty(*lead, c, h, dtype=torch.uint8, device=dev)
        t_scales = torch.empty(*lead, c, h // 32, dtype=torch.uint8, device=dev)
    _lib.check(lib().bux_mx_quantize(
        ptr(x), ptr(index), index_div, groups, r, c, h, ptr(filled), flags,
        ptr(vals), ptr(scales), ptr(t_vals), ptr(t_scales), stream()))
    along_rows = Blocks(vals, scales) if rows else None
    along_columns = Blocks(t_vals, t_scales) if columns else None
    return along_rows, along_columns


_DTYPES = {torch.bfloat16: _lib.BF16, torch.float32: _lib.F32}


def rows(
    a: Blocks, b: Blocks, sizes: torch.Tensor, out: torch.dtype = torch.bfloat16,
    height: int | None = None,
) -> torch.Tensor:
    """Return ``a @ b[g]^T`` for each group g's rows of a, (height, n), the rows past
    the groups 0.

    Args:
        a: the rows (m, k), group 0's first, in MXFP8 along k.
        b: the groups' matrices (g, n, k), in MXFP8 along k.
        sizes: int32 (g,) on the device: how many rows each group has.
        out: the output's dtype, bfloat16 or float32.
        height: rows of the output (a's rows past it are not stored); None for m.
    """
    require(a.values, a.scales, b.values, b.scales, sizes)
    m, k = a.values.shape
    groups, n, kb = b.values.shape
    if kb != k or sizes.shape != (groups,) or sizes.dtype != torch.int32:
        raise ValueError(f"rows: a {tuple(a.values.shape)}, b {tuple(b.values.shape)}, "
                         f"sizes {tuple(sizes.shape)} {sizes.dtype}")
    h = m if height is None else height
    y = torch.empty(h, n, dtype=out, device=a.values.device)
    ws = workspace(lib().bux_mx_grouped_rows_workspace_size(groups, m, h), y.device)
    _lib.check(lib().bux_mx_grouped_rows(
        ptr(a.values), ptr(a.scales), ptr(b.values), ptr(b.scales), ptr(sizes), groups, m, n, k,
        h, _DTYPES[out], ptr(y), ptr(ws), ws.numel(), stream()))
    return y


def contract(
    a: Blocks, b: Blocks, sizes: torch.Tensor, out: torch.dtype = torch.bfloat16
) -> torch.Tensor:
    """Return ``a[:, rows of g] b[:, rows of g]^T`` for each group g, (g, d, f).

    Args:
        a: x^T (d, m) in MXFP8 along m.
        b: dy^T (f, m) in MXFP8 along m.
        sizes: int32 (g,) on the device, summing to at most m.
        out: the output's dtype.
    """
    require(a.values, a.scales, b.values, b.scales, sizes)
    d, m = a.values.shape
    f, mb = b.values.shape
    groups = sizes.shape[0]
    if mb != m or sizes.dtype != torch.int32:
        raise ValueError(f"contract: a {tuple(a.values.shape)}, b {tuple(b.values.shape)}")
    dw = torch.empty(groups, d, f, dtype=out, device=a.values.device)
    ws = workspace(lib().bux_mx_grouped_contract_workspace_size(groups), dw.device)
    _lib.check(lib().bux_mx_grouped_contract(
        ptr(a.values), ptr(a.scales), ptr(b.values), ptr(b.scales), ptr(sizes), groups, d, f, m,
        _DTYPES[out], ptr(dw), ptr(ws), ws.numel(), stream()))
    return dw
