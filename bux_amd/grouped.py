"""The grouped GEMMs of the "compute" precision (no MXFP8) on MI355X.

Mirrors ``grouped.dot`` and ``grouped.weight_grad``
(src/bux/architecture/experts/grouped.py:90-146): float32 sums, out in the operands'
dtype (bfloat16, or float32 for a layer in float32), the rows past the groups 0.
"""

import torch

from bux_amd import _lib
from bux_amd.kernels import lib, ptr, require, stream, workspace


def _f32(name: str, *tensors: torch.Tensor) -> bool:
    """Whether the operands are float32 (all), not bfloat16 (all)."""
    kinds = {t.dtype for t in tensors}
    if kinds == {torch.float32}:
        return True
    if kinds == {torch.bfloat16}:
        return False
    raise TypeError(f"{name}: bfloat16 or float32 operands, one dtype, not {kinds}")


def dot(x: torch.Tensor, w: torch.Tensor, sizes: torch.Tensor, transposed: bool = False) -> torch.Tensor:
    """Return each group's rows of x times its matrix: x (m, k) and w (g, k, n), or
    with `transposed` w (g, n, k) and x w[g]^T; in x's dtype (bfloat16 or float32, w
    the same)."""
    require(x, w, sizes)
    f32 = _f32("dot", x, w)
    m, k = x.shape
    groups = w.shape[0]
    n = w.shape[1] if transposed else w.shape[2]
    if (w.shape[2] if transposed else w.shape[1]) != k:
        raise ValueError(f"dot: x {tuple(x.shape)}, w {tuple(w.shape)}, transposed={transposed}")
    y = torch.empty(m, n, dtype=x.dtype, device=x.device)
    ws = workspace(lib().bux_bf16_grouped_rows_workspace_size(groups, m), x.device)
    rows = lib().bux_bf16_grouped_rows_f32 if f32 else lib().bux_bf16_grouped_rows
    _lib.check(rows(ptr(x), ptr(w), int(transposed), ptr(sizes), groups, m, n, k, ptr(y), ptr(ws),
                    ws.numel(), stream()))
    return y


def weight_grad(x: torch.Tensor, dy: torch.Tensor, sizes: torch.Tensor) -> torch.Tensor:
    """Return ``x[rows of g]^T dy[rows of g]`` for each group g, (g, k, n), in x's dtype
    (bfloat16 or float32, dy the same)."""
    require(x, dy, sizes)
    f32 = _f32("weight_grad", x, dy)
    m, k = x.shape
    n = dy.shape[1]
    groups = sizes.shape[0]
    dw = torch.empty(groups, k, n, dtype=x.dtype, device=x.device)
    ws = workspace(lib().bux_bf16_grouped_contract_workspace_size(groups), x.device)
    contract = lib().bux_bf16_grouped_contract_f32 if f32 else lib().bux_bf16_grouped_contract
    _lib.check(contract(ptr(x), ptr(dy), ptr(sizes), groups, m, k, n, ptr(dw), ptr(ws), ws.numel(),
                        stream()))
    return dw
