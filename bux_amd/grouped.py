"""bfloat16 grouped GEMMs (the experts in "compute" precision) on MI355X.

Mirrors ``grouped.dot`` and ``grouped.weight_grad``
(src/bux/architecture/experts/grouped.py:90-146): float32 sums, bfloat16 out, the
rows past the groups 0.
"""

import torch

from bux_amd import _lib
from bux_amd.kernels import lib, ptr, require, stream, workspace


def dot(x: torch.Tensor, w: torch.Tensor, sizes: torch.Tensor, transposed: bool = False) -> torch.Tensor:
    """Return each group's rows of x times its matrix: x (m, k) and w (g, k, n), or
    with `transposed` w (g, n, k) and x w[g]^T."""
    require(x, w, sizes)
    m, k = x.shape
    groups = w.shape[0]
    n = w.shape[1] if transposed else w.shape[2]
    if (w.shape[2] if transposed else w.shape[1]) != k:
        raise ValueError(f"dot: x {tuple(x.shape)}, w {tuple(w.shape)}, transposed={transposed}")
    y = torch.empty(m, n, dtype=torch.bfloat16, device=x.device)
    ws = workspace(lib().bux_bf16_grouped_rows_workspace_size(groups, m), x.device)
    _lib.check(lib().bux_bf16_grouped_rows(
        ptr(x), ptr(w), int(transposed), ptr(sizes), groups, m, n, k, ptr(y), ptr(ws),
        ws.numel(), stream()))
    return y


def weight_grad(x: torch.Tensor, dy: torch.Tensor, sizes: torch.Tensor) -> torch.Tensor:
    """Return ``x[rows of g]^T dy[rows of g]`` for each group g, (g, k, n)."""
    require(x, dy, sizes)
    m, k = x.shape
    n = dy.shape[1]
    groups = sizes.shape[0]
    dw = torch.empty(groups, k, n, dtype=torch.bfloat16, device=x.device)
    ws = workspace(lib().bux_bf16_grouped_contract_workspace_size(groups), x.device)
    _lib.check(lib().bux_bf16_grouped_contract(
        ptr(x), ptr(dy), ptr(sizes), groups, m, k, n, ptr(dw), ptr(ws), ws.numel(), stream()))
    return dw
