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

import ctypes
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
    """Return ``z[order // k]`` (bfloat16 or float32 rows), a row of 0 where ``order //
    k`` lies outside z's rows (a negative entry too; the sort's orders never do)."""
    require(z, order)
    if z.dtype == torch.float32:  # a float32 row moves as twice the 16-bit words
        return token_rows(z.view(torch.int16), order, k).view(torch.float32)
    m, width = order.shape[0], z.shape[-1]
    rows = torch.empty(m, width, dtype=z.dtype, device=z.device)
    _lib.check(lib().bux_token_rows(ptr(z), z.shape[0], ptr(order), m, k, width, ptr(rows),
                                    stream()))
    return rows


def picked_weights(weights: torch.Tensor, order: torch.Tensor) -> torch.Tensor:
    """Return each sorted pick's weight, ``weights.reshape(-1)[order]``."""
    return token_rows(weights.reshape(-1, 1), order, 1).reshape(-1)


def sum_by_token(y: torch.Tensor, inverse: torch.Tensor) -> torch.Tensor:
    """Return each token's sum of its k rows of y at `inverse` (t, k), added in float32
    and given y's dtype (bfloat16 or float32); a row outside y adds 0."""
    require(y, inverse)
    tokens, k = inverse.shape
    width = y.shape[-1]
    out = torch.empty(tokens, width, dtype=y.dtype, device=y.device)
    sums = lib().bux_token_sums_f32 if y.dtype == torch.float32 else lib().bux_token_sums
    _lib.check(sums(ptr(y), y.shape[0], ptr(inverse), tokens, k, width, ptr(out), stream()))
    return out


class Ffn(NamedTuple):
    """An expert FFN's activation settings (config.MLPConfig, config.py:204-221):
    ``act(gate) * (up + up_offset)`` gated, ``act(up)`` plain, `limit` clipping up to
    [-limit, limit] (and a gate from above), `up_softcap` capping up to ``c tanh(up /
    c)`` (layers/mlp.py:20-35). Gating follows the projection's shape, (m, f, 2) gated
    or (m, f, 1) plain, as ``moe.hidden_units`` reads it (moe.py:913-919)."""

    activation: str = "swish"  # any of _lib.ACTIVATIONS
    limit: float | None = None
    up_offset: float = 0.0
    up_softcap: float | None = None

    def struct(self, gated: bool = True) -> _lib.FfnStruct:
        """Return the settings as the library's ``bux_ffn``."""
        if self.activation not in _lib.ACTIVATIONS:
            raise ValueError(f"no activation {self.activation!r}: one of {list(_lib.ACTIVATIONS)}")
        return _lib.FfnStruct(
            _lib.ACTIVATIONS[self.activation], int(gated), int(self.limit is not None),
            0.0 if self.limit is None else float(self.limit), int(self.up_softcap is not None),
            0.0 if self.up_softcap is None else float(self.up_softcap), float(self.up_offset))

    def fusable(self, gated: bool) -> bool:
        """Whether the fused up GEMM (`grouped_mxfp8.activated`) runs these settings: a
        gated swish, quick_gelu or situ (grouped_glu.epilogue's gated forms,
        experts/grouped_glu.py:119-136)."""
        return gated and self.activation in ("swish", "quick_gelu", "situ")


def _f32(*tensors: torch.Tensor) -> bool:
    """Whether the activation's inputs are float32 (all of them), not bfloat16 (all)."""
    kinds = {t.dtype for t in tensors}
    if kinds == {torch.float32}:
        return True
    if kinds == {torch.bfloat16}:
        return False
    raise TypeError(f"the activation's inputs are all bfloat16 or all float32, not {kinds}")


def _gating(projected: torch.Tensor) -> tuple[int, int, bool]:
    """(m, f, gated) of projected (m, f, 2) or (m, f, 1)."""
    if projected.dim() != 3 or projected.shape[2] not in (1, 2):
        raise ValueError(f"projected is (m, f, 2) or (m, f, 1), not {tuple(projected.shape)}")
    return projected.shape[0], projected.shape[1], projected.shape[2] == 2


def weighted_units(ffn: Ffn, projected: torch.Tensor, weights: torch.Tensor,
                   filled: torch.Tensor | None = None) -> torch.Tensor:
    """Return each row's hidden units times its weight, (m, f), from projected
    (m, f, 2) ([..., 0] up, [..., 1] gate) or (m, f, 1) (up) and the rows' weights
    (m,); rows from `filled` on are 0. In projected's dtype (bfloat16, or float32 with
    float32 weights)."""
    require(projected, weights, filled)
    m, f, gated = _gating(projected)
    f32 = _f32(projected, weights)
    h = torch.empty(m, f, dtype=projected.dtype, device=projected.device)
    st = ffn.struct(gated)
    forward = lib().bux_glu_forward_f32 if f32 else lib().bux_glu_forward
    _lib.check(forward(ptr(projected), ptr(weights), ptr(filled), m, f, ctypes.byref(st), ptr(h),
                       stream()))
    return h


def _copies(rows: int, cols: int, height: int, along_rows: bool, along_m: bool,
             dev: torch.device) -> tuple[Tiled | None, Tiled | None]:
    """Buffers for an (rows, cols) matrix's MXFP8 copies (`height` rows of the row copy),
    each only if asked for: along its rows (K = cols) and, transposed, along m."""
    kc, kh = grouped_mxfp8.whole(cols, grouped_mxfp8.K_ALIGN), grouped_mxfp8.whole(height, grouped_mxfp8.K_ALIGN)
    row = col = None
    if along_rows:
        row = Tiled(torch.empty(kc // 64, height, 64, dtype=torch.uint8, device=dev),
                    torch.empty(kc // 128, height, 4, dtype=torch.uint8, device=dev))
    if along_m:
        col = Tiled(torch.empty(kh // 64, cols, 64, dtype=torch.uint8, device=dev),
                    torch.empty(kh // 128, cols, 4, dtype=torch.uint8, device=dev))
    return row, col


def _ptrs(copy: Tiled | None) -> tuple[int | None, int | None]:
    return (None, None) if copy is None else (ptr(copy.values), ptr(copy.scales))


def weighted_units_quantized(ffn: Ffn, projected: torch.Tensor, weights: torch.Tensor,
                             filled: torch.Tensor | None, height: int, keep: bool = False,
                             rows: bool = True, columns: bool = True,
                             ) -> tuple[Tiled | None, Tiled | None, torch.Tensor | None]:
    """Return `weighted_units` in MXFP8 along its rows (if `rows`) and, as h^T, along m
    (if `columns`; both tiled, `height` rows of the copies, None for a copy not asked
    for), computed and quantized in one pass; with `keep`, h itself (projected's dtype
    (m, f)) too, else None. In float32 (projected and weights float32) h is the float32
    result, quantized as it is."""
    require(projected, weights, filled)
    if not (rows or columns):
        raise ValueError("weighted_units_quantized: no copy asked for")
    m, f, gated = _gating(projected)
    dev = projected.device
    row, col = _copies(m, f, height, rows, columns, dev)
    h = torch.empty(m, f, dtype=projected.dtype, device=dev) if keep else None
    st = ffn.struct(gated)
    quantize = lib().bux_glu_quantize_f32 if _f32(projected, weights) else lib().bux_glu_quantize
    _lib.check(quantize(
        ptr(projected), ptr(weights), ptr(filled), m, f, ctypes.byref(st), height, ptr(h),
        *_ptrs(row), *_ptrs(col), stream()))
    return row, col, h


def weighted_units_backward_quantized(
    ffn: Ffn, projected: torch.Tensor, weights: torch.Tensor, dh: torch.Tensor,
    filled: torch.Tensor | None, height: int, keep: bool = False,
    rows: bool = True, columns: bool = True,
) -> tuple[Tiled | None, Tiled | None, torch.Tensor, torch.Tensor | None]:
    """Return the gradient of `weighted_units` to projected in MXFP8 along its rows (p f;
    if `rows`) and, transposed, along m (if `columns`; both tiled, `height` rows of the
    copies, None for a copy not asked for), the gradient to the weights (m,), and with
    `keep` the gradient to projected (m, f, p), in projected's dtype (bfloat16, or
    float32 with weights and dh float32 too)."""
    require(projected, weights, dh, filled)
    if not (rows or columns):
        raise ValueError("weighted_units_backward_quantized: no copy asked for")
    f32 = _f32(projected, weights, dh)
    m, f, gated = _gating(projected)
    p = projected.shape[2]
    dev = projected.device
    row, col = _copies(m, p * f, height, rows, columns, dev)
    dtype = torch.float32 if f32 else torch.bfloat16
    dw = torch.empty(m, dtype=dtype, device=dev)
    dp = torch.empty(m, f, p, dtype=dtype, device=dev) if keep else None
    ws = workspace(lib().bux_glu_backward_quantize_workspace_size(m, f), dev)
    st = ffn.struct(gated)
    backward = lib().bux_glu_backward_quantize_f32 if f32 else lib().bux_glu_backward_quantize
    _lib.check(backward(
        ptr(projected), ptr(weights), ptr(dh), ptr(filled), m, f, ctypes.byref(st), height,
        ptr(dp), *_ptrs(row), *_ptrs(col), ptr(dw), ptr(ws), ws.numel(), stream()))
    return row, col, dw, dp


def weighted_units_backward(ffn: Ffn, projected: torch.Tensor, weights: torch.Tensor,
                            dh: torch.Tensor, filled: torch.Tensor | None = None
                            ) -> tuple[torch.Tensor, torch.Tensor]:
    """Return the gradients of `weighted_units` to projected (m, f, p) and to the
    weights (m,), in projected's dtype (weights and dh the same)."""
    require(projected, weights, dh, filled)
    m, f, gated = _gating(projected)
    f32 = _f32(projected, weights, dh)
    dp = torch.empty(projected.shape, dtype=projected.dtype, device=projected.device)
    dw = torch.empty(m, dtype=projected.dtype, device=projected.device)
    st = ffn.struct(gated)
    backward = lib().bux_glu_backward_f32 if f32 else lib().bux_glu_backward
    _lib.check(backward(ptr(projected), ptr(weights), ptr(dh), ptr(filled), m, f,
                        ctypes.byref(st), ptr(dp), ptr(dw), stream()))
    return dp, dw


# --- The experts' biases ---------------------------------------------------------------


def _experts(offsets: torch.Tensor) -> int:
    if offsets.dtype != torch.int32 or offsets.dim() != 1 or offsets.numel() < 2:
        raise ValueError(f"offsets are int32 (E + 1,), not {offsets.dtype} {tuple(offsets.shape)}")
    return offsets.numel() - 1


def _runs_f32(name: str, x: torch.Tensor, *others: torch.Tensor | None) -> bool:
    """Whether the op runs in float32: x is bfloat16 or float32, and every other tensor
    given (the biases, weights and norm parameters beside it) has x's dtype."""
    if x.dtype not in (torch.bfloat16, torch.float32):
        raise TypeError(f"{name}: bfloat16 or float32 rows, not {x.dtype}")
    for t in others:
        if t is not None and t.dtype != x.dtype:
            raise TypeError(f"{name}: a {t.dtype} tensor beside {x.dtype} rows")
    return x.dtype == torch.float32


def add_expert_bias(x: torch.Tensor, bias: torch.Tensor, offsets: torch.Tensor) -> torch.Tensor:
    """Add each row's expert's row of `bias` (E, width) to x (m, width) in place and
    return x: ``x + by_expert(bias, sizes)`` in x's dtype, bfloat16 or float32 (bias
    the same) (moe.py:848-849,857-861,876-885)."""
    require(x, bias, offsets)
    e = _experts(offsets)
    m, width = x.shape[0], x.numel() // max(x.shape[0], 1)
    f32 = _runs_f32("add_expert_bias", x, bias)
    if bias.numel() != e * width:
        raise ValueError(f"bias {tuple(bias.shape)} for {e} experts of {width}")
    add = lib().bux_expert_bias_add_f32 if f32 else lib().bux_expert_bias_add
    _lib.check(add(ptr(x), m, width, ptr(bias.contiguous()), ptr(offsets), e, stream()))
    return x


def expert_sums(x: torch.Tensor, offsets: torch.Tensor, index: torch.Tensor | None = None,
                index_div: int = 1, weights: torch.Tensor | None = None) -> torch.Tensor:
    """Return each expert's sum of its rows, float32 (E, width): rows ``x[index[r] //
    index_div]`` (or ``x[r]``), each times ``weights[r]`` (rounded to x's dtype) if
    given. The gradient of `add_expert_bias`'s bias, and with the picks' tokens and
    weights of the down bias (moe.py:866-870). x bfloat16 or float32, weights x's
    dtype."""
    require(x, offsets, index, weights)
    e = _experts(offsets)
    m = index.numel() if index is not None else x.shape[0]
    width = x.numel() // x.shape[0] if x.shape[0] else x.shape[-1]
    f32 = _runs_f32("expert_sums", x, weights)
    if weights is not None and weights.numel() != m:
        raise ValueError(f"expert_sums: {weights.numel()} weights for {m} rows")
    out = torch.empty(e, width, dtype=torch.float32, device=x.device)
    sums = lib().bux_expert_sums_f32 if f32 else lib().bux_expert_sums
    _lib.check(sums(ptr(x), ptr(index), index_div, x.shape[0], ptr(weights), m, width,
                    ptr(offsets), e, ptr(out), stream()))
    return out


def sum_by_token_biased(y: torch.Tensor, inverse: torch.Tensor, bias: torch.Tensor,
                        offsets: torch.Tensor, row_weights: torch.Tensor) -> torch.Tensor:
    """Return `sum_by_token` (y) plus each token's sum of its picks' ``bias[e] * w``:
    the down bias's forward, ``y + sums_of_tokens(weighted(by_expert(down_bias),
    weights))`` (moe.py:866-870), in y's dtype (bias and row_weights the same)."""
    require(y, inverse, bias, offsets, row_weights)
    e = _experts(offsets)
    tokens, k = inverse.shape
    width = y.shape[-1]
    f32 = _runs_f32("sum_by_token_biased", y, bias, row_weights)
    if bias.numel() != e * width:
        raise ValueError(f"bias {tuple(bias.shape)} for {e} experts of {width}")
    out = torch.empty(tokens, width, dtype=y.dtype, device=y.device)
    sums = lib().bux_token_sums_biased_f32 if f32 else lib().bux_token_sums_biased
    _lib.check(sums(ptr(y), y.shape[0], ptr(inverse), tokens, k, width, ptr(bias.contiguous()),
                    ptr(offsets), e, ptr(row_weights), ptr(out), stream()))
    return out


def add_bias_weight_grad(d_weights: torch.Tensor, dy: torch.Tensor, order: torch.Tensor, k: int,
                         bias: torch.Tensor, offsets: torch.Tensor) -> torch.Tensor:
    """Add the down bias's share of the row weights' gradient to `d_weights` (m,) in
    place: ``sum_c dy[order[r] // k, c] bias[e(r), c]`` (weighted's VJP,
    moe.py:922-925), in dy's dtype (d_weights and bias the same)."""
    require(d_weights, dy, order, bias, offsets)
    e = _experts(offsets)
    m, width = order.numel(), dy.shape[-1]
    f32 = _runs_f32("add_bias_weight_grad", dy, d_weights, bias)
    grad = lib().bux_expert_bias_weight_grad_f32 if f32 else lib().bux_expert_bias_weight_grad
    _lib.check(grad(ptr(dy), ptr(order), k, dy.shape[0], m, width, ptr(bias.contiguous()),
                    ptr(offsets), e, ptr(d_weights), stream()))
    return d_weights


# --- The experts' output norm ------------------------------------------------------


class ExpertNorm(NamedTuple):
    """The norm of each expert's output rows (MoEConfig.expert_norm, config.py:306): a
    NormalizationConfig (config.py:71-92) of layernorm or rmsnorm, its gain (`scale`)
    and bias given as (d,) tensors of the layer's dtype, as the model casts its
    parameters for the forward (train/trainer.py:129-140)."""

    kind: str = "rmsnorm"  # or "layernorm"
    eps: float = 1e-6
    affine: bool = True
    bias: bool = False
    zero_centered: bool = False
    scale_input: bool = False

    def struct(self) -> _lib.NormStruct:
        kinds = {"layernorm": _lib.LAYERNORM, "rmsnorm": _lib.RMSNORM}
        if self.kind not in kinds:
            raise ValueError(f"no norm {self.kind!r}: layernorm or rmsnorm")
        return _lib.NormStruct(kinds[self.kind], int(self.affine), int(self.zero_centered),
                               int(self.scale_input), int(self.bias), float(self.eps))


def expert_norm_forward(y: torch.Tensor, offsets: torch.Tensor, norm: ExpertNorm,
                        scale: torch.Tensor | None, bias: torch.Tensor | None,
                        row_weights: torch.Tensor, down_bias: torch.Tensor | None = None
                        ) -> torch.Tensor:
    """Return ``weighted(norm(y + down_bias), weights)`` of the down GEMM's rows y
    (m, d) (moe.py:871-872) in y's dtype, bfloat16 or float32 (the other tensors the
    same); rows in no expert 0."""
    require(y, offsets, scale, bias, row_weights, down_bias)
    e = _experts(offsets)
    m, d = y.shape
    f32 = _runs_f32("expert_norm_forward", y, scale, bias, row_weights, down_bias)
    out = torch.empty_like(y)
    st = norm.struct()
    forward = lib().bux_expert_norm_forward_f32 if f32 else lib().bux_expert_norm_forward
    _lib.check(forward(ptr(y), m, d, ptr(down_bias), ptr(offsets), e, ctypes.byref(st), ptr(scale),
                       ptr(bias), ptr(row_weights), ptr(out), stream()))
    return out


def expert_norm_backward(dy: torch.Tensor, order: torch.Tensor, k: int, y: torch.Tensor,
                         offsets: torch.Tensor, norm: ExpertNorm, scale: torch.Tensor | None,
                         bias: torch.Tensor | None, row_weights: torch.Tensor,
                         down_bias: torch.Tensor | None = None
                         ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor | None,
                                    torch.Tensor | None]:
    """Return the VJP of `expert_norm_forward` given the tokens' gradient dy (t, d):
    the gradient to y (m, d) (the down bias's, by expert) and to the row weights (m,)
    in y's dtype, and to the norm's scale and bias (d,) float32 (None where it has
    none). dy and the other tensors in y's dtype, bfloat16 or float32."""
    require(dy, order, y, offsets, scale, bias, row_weights, down_bias)
    e = _experts(offsets)
    m, d = y.shape
    f32 = _runs_f32("expert_norm_backward", y, dy, scale, bias, row_weights, down_bias)
    dev = y.device
    dv = torch.empty_like(y)
    dw = torch.empty(m, dtype=y.dtype, device=dev)
    d_scale = torch.empty(d, dtype=torch.float32, device=dev) if norm.affine else None
    d_bias = torch.empty(d, dtype=torch.float32, device=dev) if norm.bias else None
    ws = workspace(lib().bux_expert_norm_backward_workspace_size(m, d), dev)
    st = norm.struct()
    backward = lib().bux_expert_norm_backward_f32 if f32 else lib().bux_expert_norm_backward
    _lib.check(backward(
        ptr(dy), ptr(order), k, dy.shape[0], ptr(y), m, d, ptr(down_bias), ptr(offsets), e,
        ctypes.byref(st),
        ptr(scale), ptr(bias), ptr(row_weights), ptr(dv), ptr(dw), ptr(d_scale), ptr(d_bias),
        ptr(ws), ws.numel(), stream()))
    return dv, dw, d_scale, d_bias


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
    fmt: str = "mxfp8"  # the recipe they were quantized by
    up_shape: tuple = ()  # the kernels they came from: (E, d, f, p)
    down_shape: tuple = ()  # and (E, f, d)

    def check(self, fmt: str, up: torch.Tensor, down: torch.Tensor) -> None:
        """Raise unless these are `up` and `down` (by shape) quantized by `fmt`'s recipe."""
        if fmt not in MX_FORMATS:
            raise ValueError(f"kernels given in MXFP8, but the GEMMs multiply in {fmt!r}")
        if self.fmt != fmt:
            raise ValueError(f"kernels quantized by the {self.fmt!r} recipe, not {fmt!r}'s")
        if self.up_shape != tuple(up.shape) or self.down_shape != tuple(down.shape):
            raise ValueError(f"kernels quantized from {self.up_shape} and {self.down_shape}, "
                             f"not {tuple(up.shape)} and {tuple(down.shape)}")


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
    return MxWeights(up_n, up_k, down_n, down_k, fmt, tuple(up.shape), tuple(down.shape))


PASSES = ("fprop", "dgrad", "wgrad")


def passes_of(fmt: str, passes=None) -> tuple[bool, bool, bool]:
    """Return whether (fprop, dgrad, wgrad) multiply in MXFP8: none in "compute", else
    those named in `passes` (all by default), the reference's ``matmuls.in_force().
    passes`` (grouped_blockscaled.py:170,189: each GEMM of a pass outside them
    multiplies its operands as they are, in bfloat16)."""
    _check_fmt(fmt)
    if fmt not in MX_FORMATS:
        return False, False, False
    chosen = PASSES if passes is None else tuple(passes)
    unknown = set(chosen) - set(PASSES)
    if unknown:
        raise ValueError(f"passes are among {PASSES}, not {sorted(unknown)}")
    return tuple(q in chosen for q in PASSES)


class Saved(NamedTuple):
    """What the layer's backward takes of its forward (grouped_blockscaled.py:84's Saved
    for each GEMM, and the activation's input, which jax.checkpoint recomputes from)."""

    sorted: Sorted
    k: int
    row_weights: torch.Tensor  # the layer's dtype (m,)
    projected: torch.Tensor  # the layer's dtype (m, p f), with the up bias added
    h: torch.Tensor | None  # (m, f): wgrad in bfloat16, or kept for inspection
    x_m: Tiled | None  # x^T along the rows (wgrad of up in MXFP8)
    up_n: Tiled | None  # each W_up along n (dgrad of up in MXFP8)
    h_m: Tiled | None  # h^T along the rows (wgrad of down in MXFP8)
    down_n: Tiled | None  # each W_down along n (dgrad of down in MXFP8)
    rows: torch.Tensor | None  # the picks' rows (wgrad of up in bfloat16)
    tiles: grouped_mxfp8.TileList | None = None  # the MXFP8 GEMMs' tile list, made once
    passes: tuple[bool, bool, bool] = (True, True, True)  # (fprop, dgrad, wgrad) in MXFP8
    y: torch.Tensor | None = None  # with an expert norm: the down GEMM's rows (m, d)


def _layer_dtype(name: str, x: torch.Tensor) -> torch.dtype:
    """The layer's dtype, x's: bfloat16 or float32."""
    if x.dtype not in (torch.bfloat16, torch.float32):
        raise TypeError(f"{name}: the tokens are bfloat16 or float32, not {x.dtype}")
    return x.dtype


def _cast(dt: torch.dtype, *tensors: torch.Tensor | None) -> tuple[torch.Tensor | None, ...]:
    """The tensors in the layer's dtype (None stays None): the biases as by_expert casts
    them (moe.py:848-849), and the norm's parameters as the model's forward does."""
    return tuple(None if t is None else t.to(dt) for t in tensors)


def experts_forward(
    z: torch.Tensor, idx: torch.Tensor, weights: torch.Tensor, up: torch.Tensor,
    down: torch.Tensor, ffn: Ffn = Ffn(), fmt: str = "mxfp8", intermediates: bool = False,
    fused: bool = False, quantized: MxWeights | None = None, passes=None,
    up_bias: torch.Tensor | None = None, down_bias: torch.Tensor | None = None,
    norm: ExpertNorm | None = None, norm_scale: torch.Tensor | None = None,
    norm_bias: torch.Tensor | None = None,
) -> tuple[torch.Tensor, Saved]:
    """Return the routed experts' output (t, d), in z's dtype, and what the backward
    takes. In MXFP8 the activation goes straight to its quantized copies; with
    `intermediates` it is kept too (Saved.h).

    The layer computes in z's dtype, bfloat16 or float32, as the reference's does in x's
    (the kernels and weights cast to it, experts/moe.py:846; the GEMMs' outputs in it,
    grouped_blockscaled.Dtypes, grouped_blockscaled.py:129): in float32 no value is
    rounded to bfloat16 between the steps (the MXFP8 operands are quantized from the
    float32 values; a pass outside MXFP8 multiplies float32 operands, as ragged_dot of
    float32 does). The biases and the norm's parameters are cast to z's dtype.

    Args:
        z: the tokens, bfloat16 or float32 (t, d).
        idx: each token's k experts, int32 (t, k).
        weights: their weights (t, k), cast to z's dtype.
        up: the experts' up kernels (E, d, f, p), cast to z's dtype: p = 2 for a gated
            FFN (up and gate), 1 for a plain one.
        down: the experts' down kernels (E, f, d), cast to z's dtype.
        ffn: the activation.
        fmt: "mxfp8" (Transformer Engine's recipe: every operand in blocks of 32 along
            what its GEMM contracts), "mxfp8_2d" (the same, but each W with a scale per
            32 x 32 tile, shared by its two copies: blockscaled.MXFP8_2D,
            blockscaled.py:306-309), or "compute" for bfloat16 GEMMs.
        quantized: the kernels already in MXFP8 (`in_mxfp8(up, down, fmt)`), as the
            reference's `quantized` (moe.py:799); None to quantize them here.
        fused: in MXFP8 (without `intermediates`), the activation and h's two copies in
            the up GEMM's epilogue (`grouped_mxfp8.activated`) where it runs them (every
            pass in MXFP8, no bias, `Ffn.fusable`; moe.fused, moe.py:888-895): the same
            bits, in one GEMM kernel instead of the GEMM and the activation's quantizer.
        passes: the GEMMs (of "fprop", "dgrad", "wgrad") that multiply in `fmt`; None
            for all. The others multiply in bfloat16.
        up_bias: the experts' up biases (E, f, p), added to the up GEMM's product;
            None for none (MLPConfig.bias, moe.py:857-861).
        down_bias: the experts' down biases (E, d): each pick adds its expert's, times
            its weight (moe.py:866-870).
        norm: a norm of each expert's output rows (MoEConfig.expert_norm), with its
            gain `norm_scale` and bias `norm_bias` ((d,)): the activation is
            then unweighted and each row is ``weighted(norm(y + down_bias), w)``
            (moe.py:871-872).
    """
    t, k = idx.shape
    e, d, f, p = up.shape
    m = t * k
    dt = _layer_dtype("experts_forward", z)
    # the kernels and the weights take x's dtype (moe.py:846); y, dx and dW then come in
    # it (grouped_blockscaled.py:129)
    up, down, weights = up.to(dt), down.to(dt), weights.to(dt)
    up_bias, down_bias, norm_scale, norm_bias = _cast(dt, up_bias, down_bias, norm_scale, norm_bias)
    fprop, dgrad, wgrad = passes_of(fmt, passes)
    if dt == torch.float32:
        fused = False  # the fused up GEMM's epilogue is bfloat16's
    if quantized is not None:
        quantized.check(fmt, up, down)
    with span("permute"):
        s = sort_by_expert(idx, e)
        filled = s.filled
        row_weights = picked_weights(weights, s.order)
    up2 = up.reshape(e, d, f * p)
    tiles = fmt == "mxfp8_2d"
    # with a norm, the activation is not weighted: the norm's output is (moe.py:871)
    act_weights = row_weights if norm is None else torch.ones_like(row_weights)
    height = grouped_mxfp8.whole(m)
    x_k = x_m = up_n = up_k = h_k = h_m = down_n = down_k = rows = listed = None
    if fprop or dgrad or wgrad:
        with span("tile list"):
            # one tile list for the step's six GEMMs: a of `height` rows, outputs of m
            listed = grouped_mxfp8.tiles_of(s.sizes, height, m)
    if fprop or wgrad:
        with span("quantize x"):
            # the copies its passes take (grouped_blockscaled.py:180-183): x along k for
            # fprop, x^T along m for wgrad
            x_k, x_m = grouped_mxfp8.quantized_twice(z, filled, wgrad, s.order, k, height,
                                                     rows=fprop)
    if not (fprop and wgrad):
        with span("gather x"):
            rows = token_rows(z, s.order, k)
    if fprop or dgrad:
        if quantized is not None:
            up_n, up_k = quantized.up_n, quantized.up_k
        else:
            with span("quantize W_up"):
                # W along n for dgrad, along k for fprop
                up_n, up_k = grouped_mxfp8.quantized_twice(up2, columns=fprop, rows=dgrad,
                                                           tiles=tiles)
    h = None
    if (fused and not intermediates and fprop and dgrad and wgrad and up_bias is None
            and norm is None and ffn.fusable(p == 2)):
        with span("up fprop + activation + quantize h"):
            projected, h_k, h_m = grouped_mxfp8.activated(x_k, up_k, s.sizes, row_weights,
                                                          ffn.struct(True), m)
    else:
        with span("up fprop"):
            if fprop:
                projected = grouped_mxfp8.rows(x_k, up_k, s.sizes, dt, height=m, tiles=listed)
            else:
                projected = grouped.dot(rows, up2, s.sizes)
        if up_bias is not None:
            with span("up bias"):
                add_expert_bias(projected, up_bias.reshape(e, f * p), s.offsets)
        pv = projected.view(m, f, p)
        if fprop or wgrad:
            with span("activation + quantize h"):
                # h along f for the down fprop, h^T along m for the down wgrad
                h_k, h_m, h = weighted_units_quantized(ffn, pv, act_weights, filled, height,
                                                       intermediates or not (fprop and wgrad),
                                                       rows=fprop, columns=wgrad)
        else:
            with span("activation"):
                h = weighted_units(ffn, pv, act_weights, filled)
    if fprop or dgrad:
        if quantized is not None:
            down_n, down_k = quantized.down_n, quantized.down_k
        else:
            with span("quantize W_down"):
                down_n, down_k = grouped_mxfp8.quantized_twice(down, columns=fprop, rows=dgrad,
                                                               tiles=tiles)
    with span("down fprop"):
        if fprop:
            y = grouped_mxfp8.rows(h_k, down_k, s.sizes, dt, height=m, tiles=listed)
        else:
            y = grouped.dot(h, down, s.sizes)
    y_rows = None
    if norm is not None:
        with span("expert norm"):
            y_rows = y
            y = expert_norm_forward(y_rows, s.offsets, norm, norm_scale, norm_bias, row_weights,
                                    None if down_bias is None else down_bias.reshape(e, d))
    with span("combine"):
        if down_bias is None or norm is not None:
            out = sum_by_token(y, s.inverse.view(t, k))
        else:
            out = sum_by_token_biased(y, s.inverse.view(t, k), down_bias.reshape(e, d), s.offsets,
                                      row_weights)
    keep_h = h if (intermediates or not wgrad) else None
    return out, Saved(s, k, row_weights, projected, keep_h, x_m, up_n, h_m, down_n, rows, listed,
                      (fprop, dgrad, wgrad), y_rows)


def experts_backward(saved: Saved, dy: torch.Tensor, up: torch.Tensor, down: torch.Tensor,
                     ffn: Ffn = Ffn(), fmt: str = "mxfp8", intermediates: bool = False,
                     up_bias: torch.Tensor | None = None, down_bias: torch.Tensor | None = None,
                     norm: ExpertNorm | None = None, norm_scale: torch.Tensor | None = None,
                     norm_bias: torch.Tensor | None = None, fused: bool = False,
                     ) -> dict[str, torch.Tensor]:
    """Return the gradients of `experts_forward`'s output, dy (t, d, in the forward's
    dtype), to z and the weights (t, k) in that dtype, to up (E, d, f, p) and down
    (E, f, d) in theirs (computed in the forward's, then cast), and with biases
    to "up_bias" (E, f, p) and "down_bias" (E, d), float32 sums, and with a norm to
    "norm_scale" and "norm_bias" (d,), float32 sums; with `intermediates`,
    also the gradients between the GEMMs: "dh" (m, f) of the down GEMM's input, "dp"
    (m, p f) of the up GEMM's output, "dx" (m, d) of its input, "d_row_weights" (m,),
    and with a norm "dv" (m, d) of the down GEMM's output. With `fused` (and the
    forward's conditions for its fused up GEMM: every pass in MXFP8, no bias or norm,
    `Ffn.fusable`, no `intermediates`), the down dgrad carries the activation's gradient
    and d projected's two copies in its epilogue (`grouped_mxfp8.activation_grad`): the
    same bits. The passes are the forward's (`saved.passes`); `fmt` is checked against
    them."""
    s, k = saved.sorted, saved.k
    t = dy.shape[0]
    dt = saved.projected.dtype  # the forward's x's
    if _layer_dtype("experts_backward", dy) != dt:
        raise TypeError(f"experts_backward: dy is {dy.dtype}, the forward's tokens {dt}")
    up_dtype, down_dtype = up.dtype, down.dtype
    up, down = up.to(dt), down.to(dt)
    up_bias, down_bias, norm_scale, norm_bias = _cast(dt, up_bias, down_bias, norm_scale, norm_bias)
    if dt == torch.float32:
        fused = False
    e, d, f, p = up.shape
    m = t * k
    filled = s.filled
    up2 = up.reshape(e, d, f * p)
    fprop, dgrad, wgrad = saved.passes
    if (fprop or dgrad or wgrad) != (fmt in MX_FORMATS):
        raise ValueError(f"experts_backward: fmt {fmt!r} is not the forward's")
    height = grouped_mxfp8.whole(m)
    dy_n = dy_m = dp_n = dp_m = dy_rows = None
    grads = {}
    if norm is not None:
        if saved.y is None:
            raise ValueError("experts_backward: a norm, but the forward ran without one")
        with span("expert norm backward"):
            db = None if down_bias is None else down_bias.reshape(e, d)
            dv, d_norm_w, d_scale, d_nbias = expert_norm_backward(
                dy, s.order, k, saved.y, s.offsets, norm, norm_scale, norm_bias,
                saved.row_weights, db)
        grads.update({"norm_scale": d_scale, "norm_bias": d_nbias})
        if down_bias is not None:
            with span("down bias grad"):
                grads["down_bias"] = expert_sums(dv, s.offsets)
        # the down GEMM's upstream is dv, a row each (no longer the tokens' dy)
        if dgrad or wgrad:
            with span("quantize dv"):
                dy_n, dy_m = grouped_mxfp8.quantized_twice(dv, filled, wgrad, height=height,
                                                           rows=dgrad)
        dy_rows = dv
    else:
        if dgrad or wgrad:
            with span("quantize dy"):
                # dy along n for dgrad, dy^T along m for wgrad (grouped_blockscaled.py:204-206)
                dy_n, dy_m = grouped_mxfp8.quantized_twice(dy, filled, wgrad, s.order, k, height,
                                                           rows=dgrad)
        if not (dgrad and wgrad):
            with span("gather dy"):
                dy_rows = token_rows(dy, s.order, k)
    pv = saved.projected.view(m, f, p)
    act_weights = saved.row_weights if norm is None else torch.ones_like(saved.row_weights)
    # the activation's gradient in the down dgrad's epilogue: its settings as the forward's
    twin = (fused and not intermediates and dgrad and wgrad and up_bias is None and norm is None
            and ffn.fusable(p == 2))
    dh = None
    if twin:
        with span("down dgrad + activation backward + quantize dp"):
            dp_n, dp_m, d_rows_w, dp = grouped_mxfp8.activation_grad(
                dy_n, saved.down_n, s.sizes, saved.projected, act_weights, ffn.struct(True), m)
    else:
        with span("down dgrad"):
            if dgrad:
                dh = grouped_mxfp8.rows(dy_n, saved.down_n, s.sizes, dt, height=m, tiles=saved.tiles)
            else:
                dh = grouped.dot(dy_rows, down, s.sizes, transposed=True)
    with span("down wgrad"):
        if wgrad:
            d_down = grouped_mxfp8.contract(saved.h_m, dy_m, s.sizes, dt, tiles=saved.tiles)
        else:
            d_down = grouped.weight_grad(saved.h, dy_rows, s.sizes)
    if twin:
        pass
    elif dgrad or wgrad:
        keep = intermediates or up_bias is not None or not (dgrad and wgrad)
        with span("activation backward + quantize dp"):
            dp_n, dp_m, d_rows_w, dp = weighted_units_backward_quantized(
                ffn, pv, act_weights, dh, filled, height, keep, rows=dgrad, columns=wgrad)
    else:
        with span("activation backward"):
            dp, d_rows_w = weighted_units_backward(ffn, pv, act_weights, dh, filled)
    if norm is not None:
        d_rows_w = d_norm_w  # the unweighted activation's is not the weights'
    if dp is not None:
        dp = dp.view(m, f * p)
    with span("up dgrad"):
        if dgrad:
            dx = grouped_mxfp8.rows(dp_n, saved.up_n, s.sizes, dt, height=m, tiles=saved.tiles)
        else:
            dx = grouped.dot(dp, up2, s.sizes, transposed=True)
    with span("up wgrad"):
        if wgrad:
            d_up = grouped_mxfp8.contract(saved.x_m, dp_m, s.sizes, dt, tiles=saved.tiles)
        else:
            d_up = grouped.weight_grad(saved.rows, dp, s.sizes)
    if up_bias is not None:
        with span("up bias grad"):
            grads["up_bias"] = expert_sums(dp, s.offsets).view(e, f, p)
    if down_bias is not None and norm is None:
        with span("down bias grad"):
            db = down_bias.reshape(e, d)
            add_bias_weight_grad(d_rows_w, dy, s.order, k, db, s.offsets)
            grads["down_bias"] = expert_sums(dy, s.offsets, s.order, k, saved.row_weights)
    with span("combine dx"):
        dz = sum_by_token(dx, s.inverse.view(t, k))
        d_weights = token_rows(d_rows_w.view(m, 1), s.inverse, 1).view(t, k)
    # the kernels' gradients back in their own dtypes (the cast's transpose)
    grads.update(z=dz, weights=d_weights, up=d_up.view(e, d, f, p).to(up_dtype),
                 down=d_down.to(down_dtype))
    if intermediates:
        grads.update(dh=dh, dp=dp, dx=dx, d_row_weights=d_rows_w)
        if norm is not None:
            grads["dv"] = dy_rows
    return grads
