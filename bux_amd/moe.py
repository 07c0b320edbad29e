"""An MoE's token path and routed experts on MI355X: sort the picks by expert, run the
experts' two grouped GEMMs with their activation between, sum each token's picks; and
the backward of all of it.

Mirrors (src/bux/architecture/experts/):

- `sort_by_expert`: ``moe.sort_by_expert`` (moe.py:776-797);
- `token_rows`, `picked_weights`: ``moe.token_rows``, ``moe.picked_weights``
  (moe.py:991-1032);
- `sum_by_token`: ``grouped_blockscaled.sum_by_token`` (grouped_blockscaled.py:141-148),
  ``moe.token_sums`` (moe.py:1035-1066);
- `weighted_units`, `weighted_units_backward`: ``moe.weighted_units`` (moe.py:898-926)
  with ``layers/mlp.activate`` (layers/mlp.py:20-35);
- `experts_forward`, `experts_backward`: ``moe.routed`` (moe.py:733-773) into
  ``moe.experts`` (moe.py:799-873) on one device, with ``grouped_blockscaled.
  ragged_dot``'s forward and backward (grouped_blockscaled.py:92-211) for each GEMM in
  MXFP8, or ``grouped.ragged_dot`` (grouped.py:42-102) in "compute" (bfloat16).

Every op enqueues HIP kernels of ``libbux_amd.so`` on the current stream; torch only
allocates the buffers.
"""

from typing import NamedTuple

import torch

from bux_amd import _lib, grouped, grouped_mxfp8
from bux_amd.grouped_mxfp8 import Tiled
from bux_amd.kernels import lib, ptr, require, stream, workspace
from bux_amd.spans import span


class Sorted(NamedTuple):
    """The picks sorted by expert (moe.py:776-791), and the groups' offsets."""

    order: torch.Tensor  # int32 (M,): the picks, sorted by expert, stably
    inverse: torch.Tensor  # int32 (M,): where each pick went
    sizes: torch.Tensor  # int32 (E,): each expert's picks
    offsets: torch.Tensor  # int32 (E + 1,): cumsum(sizes) - sizes, then sum(sizes)

    @property
    def filled(self) -> torch.Tensor:
        """The rows that hold values, sum(sizes), as a device int32 of one element."""
        return self.offsets[-1:]


def sort_by_expert(idx: torch.Tensor, num_experts: int) -> Sorted:
    """Return the flat picks `idx` (int32, k a token) sorted by expert, each expert's in
    token order; picks outside [0, num_experts) sort last and count for none."""
    require(idx)
    if idx.dtype != torch.int32:
        raise TypeError("idx is int32")
    n = idx.numel()
    dev = idx.device
    order = torch.empty(n, dtype=torch.int32, device=dev)
    inverse = torch.empty(n, dtype=torch.int32, device=dev)
    sizes = torch.empty(num_experts, dtype=torch.int32, device=dev)
    offsets = torch.empty(num_experts + 1, dtype=torch.int32, device=dev)
    ws = workspace(lib().bux_moe_permute_workspace_size(n, num_experts), dev)
    _lib.check(lib().bux_moe_permute(ptr(idx), n, num_experts, ptr(order), ptr(inverse),
                                     ptr(sizes), ptr(offsets), ptr(ws), ws.numel(), stream()))
    return Sorted(order, inverse, sizes, offsets)


def token_rows(z: torch.Tensor, order: torch.Tensor, k: int) -> torch.Tensor:
    """Return ``z[order // k]`` (bfloat16 rows)."""
    require(z, order)
    m, width = order.shape[0], z.shape[-1]
    rows = torch.empty(m, width, dtype=z.dtype, device=z.device)
    _lib.check(lib().bux_token_rows(ptr(z), ptr(order), m, k, width, ptr(rows), stream()))
    return rows


def picked_weights(weights: torch.Tensor, order: torch.Tensor) -> torch.Tensor:
    """Return each sorted pick's weight, ``weights.reshape(-1)[order]``."""
    return token_rows(weights.reshape(-1, 1), order, 1).reshape(-1)


def sum_by_token(y: torch.Tensor, inverse: torch.Tensor) -> torch.Tensor:
    """Return each token's sum of its k rows of y at `inverse` (t, k), added in float32;
    a row outside y adds 0."""
    require(y, inverse)
    tokens, k = inverse.shape
    width = y.shape[-1]
    out = torch.empty(tokens, width, dtype=y.dtype, device=y.device)
    _lib.check(lib().bux_token_sums(ptr(y), y.shape[0], ptr(inverse), tokens, k, width,
                                    ptr(out), stream()))
    return out


class Ffn(NamedTuple):
    """An expert FFN's gated activation (config.py:204-221): ``act(gate) * (up +
    up_offset)``, `limit` clipping up to [-limit, limit] and the gate from above."""

    activation: str = "swish"  # or "quick_gelu"
    limit: float | None = None
    up_offset: float = 0.0

    def codes(self) -> tuple[int, float, float]:
        kind = {"swish": _lib.SWISH, "quick_gelu": _lib.QUICK_GELU}[self.activation]
        return kind, (0.0 if self.limit is None else float(self.limit)), float(self.up_offset)


def weighted_units(ffn: Ffn, projected: torch.Tensor, weights: torch.Tensor,
                   filled: torch.Tensor | None = None) -> torch.Tensor:
    """Return each row's hidden units times its weight, (m, f), from projected
    (m, f, 2) ([..., 0] up, [..., 1] gate) and the rows' weights (m,); rows from
    `filled` on are 0."""
    require(projected, weights, filled)
    m, f = projected.shape[0], projected.shape[1]
    h = torch.empty(m, f, dtype=torch.bfloat16, device=projected.device)
    kind, limit, offset = ffn.codes()
    _lib.check(lib().bux_glu_forward(ptr(projected), ptr(weights), ptr(filled), m, f, kind, limit,
                                     offset, ptr(h), stream()))
    return h


def weighted_units_quantized(ffn: Ffn, projected: torch.Tensor, weights: torch.Tensor,
                             filled: torch.Tensor | None, height: int, keep: bool = False
                             ) -> tuple[Tiled, Tiled, torch.Tensor | None]:
    """Return `weighted_units` in MXFP8 along its rows and, as h^T, along m (both tiled,
    `height` rows of the copies), computed and quantized in one pass; with `keep`, h
    itself (bfloat16 (m, f)) too, else None."""
    require(projected, weights, filled)
    m, f = projected.shape[0], projected.shape[1]
    dev = projected.device
    kf, kh = grouped_mxfp8.whole(f, grouped_mxfp8.K_ALIGN), grouped_mxfp8.whole(height, grouped_mxfp8.K_ALIGN)
    vals = torch.empty(kf // 64, height, 64, dtype=torch.uint8, device=dev)
    scales = torch.empty(kf // 128, height, 4, dtype=torch.uint8, device=dev)
    t_vals = torch.empty(kh // 64, f, 64, dtype=torch.uint8, device=dev)
    t_scales = torch.empty(kh // 128, f, 4, dtype=torch.uint8, device=dev)
    h = torch.empty(m, f, dtype=torch.bfloat16, device=dev) if keep else None
    kind, limit, offset = ffn.codes()
    _lib.check(lib().bux_glu_quantize(
        ptr(projected), ptr(weights), ptr(filled), m, f, kind, limit, offset, height, ptr(h),
        ptr(vals), ptr(scales), ptr(t_vals), ptr(t_scales), stream()))
    return Tiled(vals, scales), Tiled(t_vals, t_scales), h


def weighted_units_backward_quantized(
    ffn: Ffn, projected: torch.Tensor, weights: torch.Tensor, dh: torch.Tensor,
    filled: torch.Tensor | None, height: int, keep: bool = False,
) -> tuple[Tiled, Tiled, torch.Tensor, torch.Tensor | None]:
    """Return the gradient of `weighted_units` to projected in MXFP8 along its rows (2f)
    and, transposed, along m (both tiled, `height` rows of the copies), the gradient to
    the weights (m,), and with `keep` the bfloat16 gradient to projected (m, f, 2)."""
    require(projected, weights, dh, filled)
    m, f = projected.shape[0], projected.shape[1]
    dev = projected.device
    kp, kh = grouped_mxfp8.whole(2 * f, grouped_mxfp8.K_ALIGN), grouped_mxfp8.whole(height, grouped_mxfp8.K_ALIGN)
    vals = torch.empty(kp // 64, height, 64, dtype=torch.uint8, device=dev)
    scales = torch.empty(kp // 128, height, 4, dtype=torch.uint8, device=dev)
    t_vals = torch.empty(kh // 64, 2 * f, 64, dtype=torch.uint8, device=dev)
    t_scales = torch.empty(kh // 128, 2 * f, 4, dtype=torch.uint8, device=dev)
    dw = torch.empty(m, dtype=torch.bfloat16, device=dev)
    dp = torch.empty(m, f, 2, dtype=torch.bfloat16, device=dev) if keep else None
    ws = workspace(lib().bux_glu_backward_quantize_workspace_size(m, f), dev)
    kind, limit, offset = ffn.codes()
    _lib.check(lib().bux_glu_backward_quantize(
        ptr(projected), ptr(weights), ptr(dh), ptr(filled), m, f, kind, limit, offset, height,
        ptr(dp), ptr(vals), ptr(scales), ptr(t_vals), ptr(t_scales), ptr(dw), ptr(ws), ws.numel(),
        stream()))
    return Tiled(vals, scales), Tiled(t_vals, t_scales), dw, dp


def weighted_units_backward(ffn: Ffn, projected: torch.Tensor, weights: torch.Tensor,
                            dh: torch.Tensor, filled: torch.Tensor | None = None
                            ) -> tuple[torch.Tensor, torch.Tensor]:
    """Return the gradients of `weighted_units` to projected (m, f, 2) and to the
    weights (m,)."""
    require(projected, weights, dh, filled)
    m, f = projected.shape[0], projected.shape[1]
    dp = torch.empty(m, f, 2, dtype=torch.bfloat16, device=projected.device)
    dw = torch.empty(m, dtype=torch.bfloat16, device=projected.device)
    kind, limit, offset = ffn.codes()
    _lib.check(lib().bux_glu_backward(ptr(projected), ptr(weights), ptr(dh), ptr(filled), m, f,
                                      kind, limit, offset, ptr(dp), ptr(dw), stream()))
    return dp, dw


# --- The layer: routed -> experts, forward and backward ------------------------------


MX_FORMATS = ("mxfp8", "mxfp8_2d")


def _check_fmt(fmt: str) -> None:
    """The grouped GEMMs' formats bux allows (train/config.py:822)."""
    if fmt not in (*MX_FORMATS, "compute"):
        raise ValueError(f"the routed experts multiply in compute, mxfp8, mxfp8_2d: not {fmt}")


class MxWeights(NamedTuple):
    """The experts' kernels in MXFP8 as the GEMMs take them, each along what its GEMM
    contracts (the reference's ``grouped_glu.Weights``, grouped_glu.py:78-90, which
    ``moe.experts`` takes as `quantized`, moe.py:799)."""

    up_n: Tiled  # each W_up along n (the dgrad's)
    up_k: Tiled  # each W_up^T along d (the forward's)
    down_n: Tiled  # each W_down along d (the dgrad's)
    down_k: Tiled  # each W_down^T along f (the forward's)


def in_mxfp8(up: torch.Tensor, down: torch.Tensor, fmt: str = "mxfp8") -> MxWeights:
    """Return the experts' kernels (E, d, f, 2) and (E, f, d) in MXFP8 for `fmt`
    (the reference's ``grouped_glu.in_mxfp8``, grouped_glu.py:187-203): once per
    optimizer step, for every forward and backward that step runs."""
    _check_fmt(fmt)
    if fmt not in MX_FORMATS:
        raise ValueError(f"in_mxfp8: {fmt!r} is not an MXFP8 format")
    e, d, f, p = up.shape
    tiles = fmt == "mxfp8_2d"
    up_n, up_k = grouped_mxfp8.quantized_twice(up.reshape(e, d, f * p), tiles=tiles)
    down_n, down_k = grouped_mxfp8.quantized_twice(down, tiles=tiles)
    return MxWeights(up_n, up_k, down_n, down_k)


class Saved(NamedTuple):
    """What the layer's backward takes of its forward (grouped_blockscaled.py:84's Saved
    for each GEMM, and the activation's input, which jax.checkpoint recomputes from)."""

    sorted: Sorted
    k: int
    row_weights: torch.Tensor  # bfloat16 (m,)
    projected: torch.Tensor  # bfloat16 (m, 2f)
    h: torch.Tensor | None  # bfloat16 (m, f): compute format, or kept for inspection
    x_m: Tiled | None  # x^T along the rows (wgrad of up)
    up_n: Tiled | None  # each W_up along n (dgrad of up)
    h_m: Tiled | None  # h^T along the rows (wgrad of down)
    down_n: Tiled | None  # each W_down along n (dgrad of down)
    rows: torch.Tensor | None  # the picks' rows, compute format only
    tiles: grouped_mxfp8.TileList | None = None  # the MXFP8 GEMMs' tile list, made once


def experts_forward(
    z: torch.Tensor, idx: torch.Tensor, weights: torch.Tensor, up: torch.Tensor,
    down: torch.Tensor, ffn: Ffn = Ffn(), fmt: str = "mxfp8", intermediates: bool = False,
    fused: bool = False, quantized: MxWeights | None = None,
) -> tuple[torch.Tensor, Saved]:
    """Return the routed experts' output (t, d), bfloat16, and what the backward takes.
    In MXFP8 the activation goes straight to its quantized copies; with `intermediates`
    it is kept in bfloat16 too (Saved.h).

    Args:
        z: the tokens, bfloat16 (t, d).
        idx: each token's k experts, int32 (t, k).
        weights: their weights, bfloat16 (t, k).
        up: the experts' up and gate kernels, bfloat16 (E, d, f, 2).
        down: the experts' down kernels, bfloat16 (E, f, d).
        ffn: the activation.
        fmt: "mxfp8" (Transformer Engine's recipe: every operand in blocks of 32 along
            what its GEMM contracts), "mxfp8_2d" (the same, but each W with a scale per
            32 x 32 tile, shared by its two copies: blockscaled.MXFP8_2D,
            blockscaled.py:306-309), or "compute" for bfloat16 GEMMs.
        quantized: the kernels already in MXFP8 (`in_mxfp8(up, down, fmt)`), as the
            reference's `quantized` (moe.py:799); None to quantize them here.
        fused: in MXFP8 (without `intermediates`), the activation and h's two copies in
            the up GEMM's epilogue (`grouped_mxfp8.activated`): the same bits, in one
            GEMM kernel instead of the GEMM and the activation's quantizer.
    """
    t, k = idx.shape
    e, d, f, p = up.shape
    m = t * k
    with span("permute"):
        s = sort_by_expert(idx, e)
        filled = s.filled
        row_weights = picked_weights(weights, s.order)
    up2 = up.reshape(e, d, f * p)
    x_m = up_n = h_m = down_n = rows = None
    _check_fmt(fmt)
    mx, tiles = fmt in MX_FORMATS, fmt == "mxfp8_2d"
    listed = None
    if mx:
        height = grouped_mxfp8.whole(m)
        with span("tile list"):
            # one tile list for the step's six GEMMs: a of `height` rows, outputs of m
            listed = grouped_mxfp8.tiles_of(s.sizes, height, m)
        with span("quantize x"):
            x_k, x_m = grouped_mxfp8.quantized_twice(z, filled, True, s.order, k, height)
        if quantized is not None:
            up_n, up_k = quantized.up_n, quantized.up_k
        else:
            with span("quantize W_up"):
                up_n, up_k = grouped_mxfp8.quantized_twice(up2, tiles=tiles)
        if fused and not intermediates:
            with span("up fprop + activation + quantize h"):
                projected, h_k, h_m = grouped_mxfp8.activated(x_k, up_k, s.sizes, row_weights,
                                                              ffn.codes(), m)
            h = None
        else:
            with span("up fprop"):
                projected = grouped_mxfp8.rows(x_k, up_k, s.sizes, height=m, tiles=listed)
    else:
        with span("gather x"):
            rows = token_rows(z, s.order, k)
        with span("up fprop"):
            projected = grouped.dot(rows, up2, s.sizes)
    if mx:
        if not (fused and not intermediates):
            with span("activation + quantize h"):
                h_k, h_m, h = weighted_units_quantized(ffn, projected.view(m, f, p), row_weights,
                                                       filled, height, intermediates)
        if quantized is not None:
            down_n, down_k = quantized.down_n, quantized.down_k
        else:
            with span("quantize W_down"):
                down_n, down_k = grouped_mxfp8.quantized_twice(down, tiles=tiles)
        with span("down fprop"):
            y = grouped_mxfp8.rows(h_k, down_k, s.sizes, height=m, tiles=listed)
    else:
        with span("activation"):
            h = weighted_units(ffn, projected.view(m, f, p), row_weights, filled)
        with span("down fprop"):
            y = grouped.dot(h, down, s.sizes)
    with span("combine"):
        out = sum_by_token(y, s.inverse.view(t, k))
    return out, Saved(s, k, row_weights, projected, h, x_m, up_n, h_m, down_n, rows, listed)


def experts_backward(saved: Saved, dy: torch.Tensor, up: torch.Tensor, down: torch.Tensor,
                     ffn: Ffn = Ffn(), fmt: str = "mxfp8", intermediates: bool = False
                     ) -> dict[str, torch.Tensor]:
    """Return the gradients of `experts_forward`'s output, dy (t, d), to z, the
    weights (t, k), up (E, d, f, 2) and down (E, f, d), all bfloat16; with
    `intermediates`, also the gradients between the GEMMs: "dh" (m, f) of the down
    GEMM's input, "dp" (m, 2f) of the up GEMM's output, "dx" (m, d) of its input and
    "d_row_weights" (m,)."""
    s, k = saved.sorted, saved.k
    t = dy.shape[0]
    e, d, f, p = up.shape
    m = t * k
    filled = s.filled
    up2 = up.reshape(e, d, f * p)
    _check_fmt(fmt)
    mx = fmt in MX_FORMATS
    if mx:
        height = grouped_mxfp8.whole(m)
        with span("quantize dy"):
            dy_n, dy_m = grouped_mxfp8.quantized_twice(dy, filled, True, s.order, k, height)
        with span("down dgrad"):
            dh = grouped_mxfp8.rows(dy_n, saved.down_n, s.sizes, height=m, tiles=saved.tiles)
        with span("down wgrad"):
            d_down = grouped_mxfp8.contract(saved.h_m, dy_m, s.sizes, tiles=saved.tiles)
    else:
        with span("gather dy"):
            dy_rows = token_rows(dy, s.order, k)
        with span("down dgrad"):
            dh = grouped.dot(dy_rows, down, s.sizes, transposed=True)
        with span("down wgrad"):
            d_down = grouped.weight_grad(saved.h, dy_rows, s.sizes)
    if mx:
        with span("activation backward + quantize dp"):
            dp_n, dp_m, d_rows_w, dp = weighted_units_backward_quantized(
                ffn, saved.projected.view(m, f, p), saved.row_weights, dh, filled, height,
                intermediates)
        if dp is not None:
            dp = dp.view(m, f * p)
        with span("up dgrad"):
            dx = grouped_mxfp8.rows(dp_n, saved.up_n, s.sizes, height=m, tiles=saved.tiles)
        with span("up wgrad"):
            d_up = grouped_mxfp8.contract(saved.x_m, dp_m, s.sizes, tiles=saved.tiles)
    else:
        with span("activation backward"):
            dp, d_rows_w = weighted_units_backward(ffn, saved.projected.view(m, f, p),
                                                   saved.row_weights, dh, filled)
        dp = dp.view(m, f * p)
        with span("up dgrad"):
            dx = grouped.dot(dp, up2, s.sizes, transposed=True)
        with span("up wgrad"):
            d_up = grouped.weight_grad(saved.rows, dp, s.sizes)
    with span("combine dx"):
        dz = sum_by_token(dx, s.inverse.view(t, k))
        d_weights = token_rows(d_rows_w.view(m, 1), s.inverse, 1).view(t, k)
    grads = {"z": dz, "weights": d_weights, "up": d_up.view(e, d, f, p), "down": d_down}
    if intermediates:
        grads.update(dh=dh, dp=dp, dx=dx, d_row_weights=d_rows_w)
    return grads
