"""An expert-parallel dispatch's tokens in MXFP8 on MI355X: each token quantized once
into a row of bytes (codes, then scales), the rows of its picks gathered for the
exchange; and on arrival, the rows back to bfloat16.

Mirrors ``src/bux/parallel/experts.py``: `in_mxfp8` is ``_in_mxfp8`` (experts.py:
659-663, ``blockscaled.mx_packed(mx_quantize(z))``); `picked_in_mxfp8` is what
``_picked_in_mxfp8`` (experts.py:612-625) hands the exchange, ``_in_mxfp8(z)[order //
k]``; `from_mxfp8` is ``_from_mxfp8`` (experts.py:666-672). The exchange itself (a
ragged all-to-all over the expert mesh axis) is not here: on one GPU the packed rows
are what it would carry. `unpacked` gives the codes and scales of packed rows as
``blockscaled.mx_unpacked`` (blockscaled.py:378-380) does.
"""

import torch

from bux_amd import _lib
from bux_amd.kernels import lib, ptr, require, stream


def _pack(z: torch.Tensor, index: torch.Tensor | None, div: int, m: int) -> torch.Tensor:
    require(z, index)
    if z.dtype != torch.bfloat16 or z.dim() != 2:
        raise TypeError("z is a bfloat16 matrix (tokens, d)")
    if index is not None and index.dtype != torch.int32:
        raise TypeError("index is int32")
    n, d = z.shape
    packed = torch.empty(m, d + d // 32, dtype=torch.uint8, device=z.device)
    _lib.check(lib().bux_mx_pack_rows(ptr(z), ptr(index), div, n, m, d, ptr(packed), stream()))
    return packed


def in_mxfp8(z: torch.Tensor) -> torch.Tensor:
    """Return each token of z (bfloat16, n x d) in MXFP8 as a row of d + d/32 bytes:
    its E4M3 codes along d in blocks of 32, then the blocks' E8M0 scale bytes."""
    return _pack(z, None, 1, z.shape[0])


def picked_in_mxfp8(z: torch.Tensor, order: torch.Tensor, k: int) -> torch.Tensor:
    """Return ``in_mxfp8(z)[order // k]``: the packed row of each sorted pick's token,
    quantized from the token directly (the same bytes)."""
    return _pack(z, order, k, order.numel())


def from_mxfp8(packed: torch.Tensor, d: int) -> torch.Tensor:
    """Return rows of `in_mxfp8` bytes as bfloat16 (m x d): each code times its
    block's scale, in float32, rounded to bfloat16."""
    require(packed)
    if packed.dtype != torch.uint8 or packed.dim() != 2 or packed.shape[1] != d + d // 32:
        raise ValueError(f"packed is uint8 rows of {d + d // 32} bytes for d={d}")
    m = packed.shape[0]
    out = torch.empty(m, d, dtype=torch.bfloat16, device=packed.device)
    _lib.check(lib().bux_mx_unpack_rows(ptr(packed), m, d, ptr(out), stream()))
    return out


def unpacked(packed: torch.Tensor, d: int) -> tuple[torch.Tensor, torch.Tensor]:
    """Return packed rows' E4M3 codes (m x d) and E8M0 scale bytes (m x d/32), as
    uint8 views (blockscaled.mx_unpacked)."""
    return packed[:, :d], packed[:, d:]
