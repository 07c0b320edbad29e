"""The MoE expert path of bux off a Blackwell GPU, restated in numpy. TEST
INFRASTRUCTURE ONLY (see `oracle`).

Follows (all paths under ``src/bux/architecture/``):

- `sort_by_expert`: ``experts/moe.py:776-797``;
- `token_rows`, `picked_weights`, `sum_by_token`: ``experts/moe.py:991-1066``,
  ``experts/grouped_blockscaled.py:141-148``;
- `tiles_of`: ``experts/grouped_mxfp8.py:157-182``;
- `rows_mx`, `contract_mx`: ``experts/grouped_blockscaled.py:220-250`` (XLA's
  dequantize, then ``ragged_dot`` / ``ragged_dot_general`` in float32);
- `ragged_dot_bf16`, `weight_grad_bf16`: ``experts/grouped.py:42-146`` off a
  GPU (``jax.lax.ragged_dot`` of bfloat16, float32 sums);
- `activate`, `weighted_units`, `weighted_units_backward`: ``layers/mlp.py:20-35``,
  ``common/functional.py:12-40``, ``experts/moe.py:898-926``;
- `layer_forward`, `layer_backward`: ``experts/moe.py:733-873`` with
  ``grouped_blockscaled.py:167-211`` (``routed`` -> ``experts`` -> two
  ``grouped_product``s, picked rows in, summed rows out).

Pins, run by ``tests/test_oracle.py``:

- `sort_by_expert`: against a brute-force stable sort (Python's ``sorted`` with the
  position as tie-break) and ``np.bincount``; on the reference's size patterns
  ``[70, 0, 100, 3, 77]`` (tests/test_grouped.py:24) and ``[0, 130, 1, 3, 256, 0,
  300, 100]`` (tests/test_grouped_mxfp8.py:23); out-of-range picks sort last;
- `tiles_of`: the reference's own invariant (tests/test_grouped_mxfp8.py:31-41):
  every group row covered once, inside one tile, count ``ceil(m/t) + g - 1``;
- `sum_by_token`: the transpose identity ``<token_rows(z), y> == <z, sum_by_token(y)>``
  in float64, and brute-force loops;
- `rows_mx`, `contract_mx`: brute-force float64 triple loops on small shapes; empty
  groups and rows past the groups are 0; garbage past ``filled`` changes no dW
  (tests/test_grouped.py:89-95);
- `weighted_units_backward`: against torch.autograd of the same forward in float64,
  for bfloat16 inputs and (to 1e-6) for a float32 layer's;
- `_act`: each activation and its derivative against torch in float64 over [-30, 30],
  and to 1e-12 relative of the textbook functions in 400-digit arithmetic (mpmath)
  from x = -700 to 300, where e^x-sized values must not cancel to 0.

Bit-level parity of float sums is unpinned: XLA:CPU's summation order inside
``ragged_dot`` and its bfloat16 excess-precision choices are not observable without
jax. The oracle sums in float32 (numpy's BLAS) and rounds once to bfloat16; GPU
results are compared to it within tolerances stated in each test.
"""

from typing import NamedTuple

import numpy as np
from scipy import special

from oracle import bf16, mxfp8
from oracle.mxfp8 import Blocks


class Sorted(NamedTuple):
    """`sort_by_expert`'s result (moe.py:776-791), plus the group offsets that the
    kernels take (``cumsum(sizes) - sizes``, grouped_mxfp8.py:142)."""

    order: np.ndarray  # int32 [M]
    inverse: np.ndarray  # int32 [M]
    sizes: np.ndarray  # int32 [E]
    offsets: np.ndarray  # int32 [E]


def sort_by_expert(idx: np.ndarray, num_experts: int) -> Sorted:
    """Return the flat picks sorted by expert, stably; picks outside [0, E) sort
    last and count for none (moe.py:776-797)."""
    flat = np.asarray(idx).reshape(-1).astype(np.int64)
    flat = np.where((flat >= 0) & (flat < num_experts), flat, num_experts)
    order = np.argsort(flat, kind="stable").astype(np.int32)
    sizes = np.bincount(flat, minlength=num_experts + 1)[:num_experts].astype(np.int32)
    inverse = np.empty_like(order)
    inverse[order] = np.arange(order.size, dtype=np.int32)
    offsets = (np.cumsum(sizes) - sizes).astype(np.int32)
    return Sorted(order, inverse, sizes, offsets)


def token_rows(z: np.ndarray, order: np.ndarray, k: int) -> np.ndarray:
    """Return ``z[order // k]`` (moe.py:991-1016)."""
    return z[np.asarray(order) // k]


def picked_weights(weights: np.ndarray, order: np.ndarray) -> np.ndarray:
    """Return each sorted pick's weight, ``weights.reshape(-1)[order]``
    (moe.py:1027-1032)."""
    return np.asarray(weights).reshape(-1)[np.asarray(order)]


def sum_by_token(y: np.ndarray, inverse: np.ndarray, out_bf16: bool = True,
                 exact: bool = False) -> np.ndarray:
    """Return each token's sum of its k rows of y at ``inverse`` (t, k), added in
    float32 in pick order; an index outside y's rows adds 0
    (grouped_blockscaled.py:141-148). y is bfloat16 bits or float32; the result is
    bfloat16 bits if `out_bf16`, else float32. `exact`: float64 sums, one rounding."""
    t_ = _sums(exact)
    values = (bf16.to_f32(y) if y.dtype == np.uint16 else np.asarray(y, np.float32)).astype(t_)
    inverse = np.asarray(inverse)
    m = values.shape[0]
    inside = (inverse >= 0) & (inverse < m)
    total = np.zeros((inverse.shape[0], values.shape[1]), t_)
    for j in range(inverse.shape[1]):
        rows = values[np.where(inside[:, j], inverse[:, j], 0)]
        total += np.where(inside[:, j, None], rows, t_(0))
    if not out_bf16:
        return total.astype(np.float32)
    return bf16.from_f64(total) if exact else bf16.to_bf16(total)


def tiles_of(sizes: np.ndarray, m: int, tile: int, starts: np.ndarray | None = None) -> np.ndarray:
    """Return, for each tile of `tile` rows of m that a group has rows in, the group
    and where its rows there start and end, then (0, 0, 0) rows up to
    ``ceil(m / tile) + g - 1`` (grouped_mxfp8.py:157-182)."""
    sizes = np.asarray(sizes, np.int64)
    g = sizes.shape[0]
    starts = np.cumsum(sizes) - sizes if starts is None else np.asarray(starts, np.int64)
    ends = starts + sizes
    first = starts // tile
    count = np.where(sizes > 0, -(-ends // tile) - first, 0)
    before = np.cumsum(count) - count
    at = np.arange(-(-m // tile) + g - 1)
    group = np.searchsorted(before + count, at, side="right")
    group = np.minimum(group, g - 1)
    index = first[group] + at - before[group]
    lo = np.maximum(starts[group], index * tile)
    hi = np.minimum(ends[group], (index + 1) * tile)
    real = at < count.sum()
    return np.stack([group, np.where(real, lo, 0), np.where(real, hi, 0)], -1).astype(np.int32)


def whole(rows: int, tile: int = 128) -> int:
    """Return `rows` rounded up to whole tiles, as ragged_dot pads its rows
    (grouped_blockscaled.py:122-124, grouped_mxfp8.LANES)."""
    return -(-rows // tile) * tile


def _cast(y: np.ndarray, out: str) -> np.ndarray:
    """The GEMMs' output: "bf16" bits (rounded once), "f32", or "f64" (exact sums
    unrounded, for tests that model another summation's error before the rounding)."""
    if out == "f64":
        return y.astype(np.float64)
    if y.dtype == np.float64:  # exact sums: one rounding
        return bf16.from_f64(y) if out == "bf16" else y.astype(np.float32)
    return bf16.to_bf16(y) if out == "bf16" else y.astype(np.float32)


def _sums(exact: bool):
    """The dtype the GEMMs multiply and add in: float32 (XLA:CPU's, the oracle's), or
    float64 with `exact` (products of dequantized E4M3 or bfloat16 values are exact
    there, and sums of up to 2^20 of them lose at most a few float64 ulps): the exact
    restatement that tells how far from the exact result a float32 order lands."""
    return np.float64 if exact else np.float32


def rows_mx(a: Blocks, b: Blocks, sizes: np.ndarray, out: str = "bf16", height: int | None = None,
            starts: np.ndarray | None = None, exact: bool = False) -> np.ndarray:
    """Return each group's rows of a times its matrix b[g]^T: a (m, k) and b
    (g, n, k) in MXFP8 along k, dequantized and multiplied in float32; rows past the
    groups are 0 (grouped_blockscaled.py:220-233, grouped_mxfp8.py:116-154). With
    `starts`, group g's rows of a start at starts[g], y's stay packed. `exact`: sums in
    float64, one rounding (`_sums`)."""
    t = _sums(exact)
    x = mxfp8.dequantized(a).astype(t)
    w = mxfp8.dequantized(b).astype(t)
    m = x.shape[0] if height is None else height
    y = np.zeros((m, w.shape[1]), t)
    start = 0
    for g, size in enumerate(np.asarray(sizes).tolist()):
        at = start if starts is None else int(starts[g])
        if size:
            y[start:start + size] = x[at:at + size] @ w[g].T
        start += size
    return _cast(y, out)


def contract_mx(a: Blocks, b: Blocks, sizes: np.ndarray, out: str = "bf16",
                exact: bool = False) -> np.ndarray:
    """Return dW[g] = a[:, rows of g] b[:, rows of g]^T: a (d, m) and b (f, m) in
    MXFP8 along m, dequantized and multiplied in float32 (grouped_blockscaled.py:
    236-250). `exact`: sums in float64, one rounding (`_sums`)."""
    t = _sums(exact)
    x = mxfp8.dequantized(a).astype(t)
    y = mxfp8.dequantized(b).astype(t)
    sizes = np.asarray(sizes).tolist()
    dw = np.zeros((len(sizes), x.shape[0], y.shape[0]), t)
    start = 0
    for g, size in enumerate(sizes):
        if size:
            dw[g] = x[:, start:start + size] @ y[:, start:start + size].T
        start += size
    return _cast(dw, out)


def ragged_dot_bf16(x: np.ndarray, w: np.ndarray, sizes: np.ndarray, out: str | None = None,
                    exact: bool = False) -> np.ndarray:
    """Return ``jax.lax.ragged_dot`` of x (m, k) and w (g, k, n), bfloat16 bits or (a
    layer in float32) float32 values: float32 sums rounded to x's dtype (`out` None;
    else as `_cast`), rows past the groups 0 (grouped.py:42-62,90-102). `exact`: sums in
    float64, one rounding (`_sums`)."""
    t = _sums(exact)
    out = out or ("f32" if _is_f32(x) else "bf16")
    xf, wf = _values(x).astype(t), _values(w).astype(t)
    y = np.zeros((xf.shape[0], wf.shape[2]), t)
    start = 0
    for g, size in enumerate(np.asarray(sizes).tolist()):
        if size:
            y[start:start + size] = xf[start:start + size] @ wf[g]
        start += size
    return _cast(y, out)


def weight_grad_bf16(x: np.ndarray, dy: np.ndarray, sizes: np.ndarray, out: str | None = None,
                     exact: bool = False) -> np.ndarray:
    """Return x^T dy per group (grouped.py:105-146) of bfloat16 bits or float32 values,
    float32 sums (`exact`: float64, one rounding) in x's dtype (`out` None)."""
    t = _sums(exact)
    out = out or ("f32" if _is_f32(x) else "bf16")
    xf, gf = _values(x).astype(t), _values(dy).astype(t)
    sizes = np.asarray(sizes).tolist()
    dw = np.zeros((len(sizes), xf.shape[1], gf.shape[1]), t)
    start = 0
    for g, size in enumerate(sizes):
        if size:
            dw[g] = xf[start:start + size].T @ gf[start:start + size]
        start += size
    return _cast(dw, out)


# --- The expert FFN's activation ---------------------------------------------------


QUICK_GELU_ALPHA = float(bf16.round_f32(np.array([1.702], np.float32))[0])  # 1.703125

ACTIVATIONS = ("swish", "quick_gelu", "relu", "relu2", "gelu", "gelu_tanh", "sigmoid", "tanh",
               "softplus", "situ")


class Ffn(NamedTuple):
    """An expert FFN's activation settings (config.py:204-221): the activation, the
    clamp, the up branch's offset and soft cap. Gated or plain follows the projection's
    last axis, 2 or 1 (moe.py:913-919)."""

    activation: str = "swish"  # one of ACTIVATIONS
    limit: float | None = None
    up_offset: float = 0.0
    up_softcap: float | None = None


def _sigmoid(x: np.ndarray) -> np.ndarray:
    """1 / (1 + e^-x), to a few float64 ulps of itself everywhere (``(1 + tanh(x/2)) / 2``
    is 0 from x = -37 on, where the true value is e^x, still a float32 down to -87)."""
    return special.expit(x)


def _act(name: str, x: np.ndarray, f32: bool = False) -> tuple[np.ndarray, np.ndarray]:
    """Return act(x) and act'(x) in float64 (functional.py:12-40; relu's gradient 0 at
    0, as jax.nn.relu's); `f32`: of a layer in float32."""
    if name in ("swish", "quick_gelu"):
        # functional.py:29 writes ``x * jax.nn.sigmoid(1.702 * x)``: jax casts the weakly
        # typed 1.702 to x's dtype, bfloat16, whose nearest value is 1.703125 (in
        # float32, 1.702's nearest float32).
        alpha = 1.0 if name == "swish" else (
            float(np.float32(1.702)) if f32 else QUICK_GELU_ALPHA)
        s, sc = _sigmoid(alpha * x), _sigmoid(-alpha * x)  # sc = 1 - s, without cancelling
        return x * s, s + alpha * x * s * sc
    if name == "relu":
        return np.maximum(x, 0.0), (x > 0).astype(np.float64)
    if name == "relu2":
        r = np.maximum(x, 0.0)
        return r * r, 2.0 * r
    # below, 1 + tanh(z) = 2 sigmoid(2 z), 1 - tanh(z)^2 = 1 / cosh(z)^2 and
    # 1 + erf(z) = erfc(-z): the same values, with no cancellation where tanh(z) nears -1
    if name == "gelu":
        phi = 0.5 * special.erfc(-x / np.sqrt(2.0))
        return x * phi, phi + x * np.exp(-0.5 * x * x) / np.sqrt(2.0 * np.pi)
    if name == "gelu_tanh":
        c = np.sqrt(2.0 / np.pi)
        z = c * (x + 0.044715 * x ** 3)
        s, sc = _sigmoid(2.0 * z), _sigmoid(-2.0 * z)
        return x * s, s + 2.0 * x * s * sc * c * (1.0 + 3 * 0.044715 * x * x)
    if name == "sigmoid":
        s = _sigmoid(x)
        return s, s * _sigmoid(-x)
    if name == "tanh":
        with np.errstate(over="ignore"):
            return np.tanh(x), 1.0 / np.cosh(x) ** 2
    if name == "softplus":
        return np.logaddexp(x, 0.0), _sigmoid(x)
    if name == "situ":
        t, s, sc = np.tanh(x / 4.0), _sigmoid(x), _sigmoid(-x)
        with np.errstate(over="ignore"):
            sech2 = 1.0 / np.cosh(x / 4.0) ** 2
        return 4.0 * t * s, sech2 * s + 4.0 * t * s * sc
    raise ValueError(name)


def _up_branch(ffn: Ffn, up: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Return the up branch clipped and capped (mlp.py:28-30), and its derivative (jnp.clip
    is maximum then minimum, whose gradients split 0.5 / 0.5 at a tie: at a limit of 0
    an up of 0 ties both, 0.25)."""
    d = np.ones_like(up)
    if ffn.limit is not None:
        tie = 0.25 if ffn.limit == 0 else 0.5
        d = np.where(np.abs(up) < ffn.limit, 1.0, np.where(np.abs(up) == ffn.limit, tie, 0.0))
        up = np.clip(up, -ffn.limit, ffn.limit)
    if ffn.up_softcap is not None:
        t = np.tanh(up / ffn.up_softcap)
        d = d * (1.0 - t * t)
        up = ffn.up_softcap * t
    return up, d


def _wide(x: np.ndarray) -> np.ndarray:
    """bfloat16 bits (uint16) or float32 values as float64, exactly."""
    x = np.asarray(x)
    return (bf16.to_f32(x) if x.dtype == np.uint16 else x.astype(np.float32)).astype(np.float64)


def _narrow(v: np.ndarray, f32: bool) -> np.ndarray:
    """float64 values rounded once: to float32 (`f32`), else to bfloat16 bits (through
    float32, as the activation's float32 result is rounded)."""
    return v.astype(np.float32) if f32 else bf16.to_bf16(v.astype(np.float32))


def weighted_units(ffn: Ffn, projected: np.ndarray, weights: np.ndarray) -> np.ndarray:
    """Return ``act(gate) * (up + offset) * w`` for projected (m, f, 2) [up, gate], or
    ``act(up) * w`` for (m, f, 1) or (m, f), and row weights (m,), computed in float64
    and rounded once (mlp.py:20-35, moe.py:898-926): bfloat16 bits of bfloat16 bits, or
    float32 of float32 (a layer in float32)."""
    f32 = np.asarray(projected).dtype == np.float32
    p = _wide(projected)
    if p.ndim == 2:
        p = p[..., None]
    w = _wide(weights)[:, None]
    up, _ = _up_branch(ffn, p[..., 0])
    if p.shape[-1] == 1:
        a, _ = _act(ffn.activation, up, f32)
        return _narrow(a * w, f32)
    gate = p[..., 1]
    if ffn.limit is not None:
        gate = np.minimum(gate, ffn.limit)
    a, _ = _act(ffn.activation, gate, f32)
    return _narrow(a * (up + ffn.up_offset) * w, f32)


def weighted_units_backward(
    ffn: Ffn, projected: np.ndarray, weights: np.ndarray, dh: np.ndarray
) -> tuple[np.ndarray, np.ndarray]:
    """Return the gradients of `weighted_units` to projected (its shape) and to the row
    weights (m,), as bfloat16 bits (float32 for float32 inputs) (the VJP jax takes of it,
    moe.py:898-910, with jax's gradients of clip and minimum: 1 strictly inside, 0.5 at
    the limit, 0 outside)."""
    f32 = np.asarray(projected).dtype == np.float32
    p = _wide(projected)
    plain2d = p.ndim == 2
    if plain2d:
        p = p[..., None]
    w = _wide(weights)[:, None]
    g_ = _wide(dh)
    up, up_pass = _up_branch(ffn, p[..., 0])
    if p.shape[-1] == 1:
        a, da = _act(ffn.activation, up, f32)
        dp = (g_ * w * da * up_pass)[..., None]
        d_w = (g_ * a).sum(-1)
    else:
        gate = p[..., 1]
        gate_pass = np.ones_like(gate)
        if ffn.limit is not None:
            gate_pass = np.where(gate < ffn.limit, 1.0, np.where(gate == ffn.limit, 0.5, 0.0))
            gate = np.minimum(gate, ffn.limit)
        a, da = _act(ffn.activation, gate, f32)
        u = up + ffn.up_offset
        dp = np.stack([g_ * w * a * up_pass, g_ * w * u * da * gate_pass], -1)
        d_w = (g_ * a * u).sum(-1)
    if plain2d:
        dp = dp[..., 0]
    return _narrow(dp, f32), _narrow(d_w, f32)


# --- The experts' biases ----------------------------------------------------------------


def _expert_of_rows(sizes: np.ndarray, m: int) -> np.ndarray:
    """Each of m sorted rows' expert, -1 past the groups."""
    sizes = np.asarray(sizes, np.int64)
    ends = np.cumsum(sizes)
    r = np.arange(m)
    e = np.searchsorted(ends, r, side="right")
    return np.where(r < ends[-1] if ends.size else False, e, -1)


def _values(x: np.ndarray) -> np.ndarray:
    """bfloat16 bits (uint16) or float32 values as float32, exactly."""
    x = np.asarray(x)
    return bf16.to_f32(x) if x.dtype == np.uint16 else x.astype(np.float32)


def _is_f32(x: np.ndarray) -> bool:
    """Whether x holds a float32 layer's values (float32), not bfloat16 bits."""
    return np.asarray(x).dtype == np.float32


def by_expert(bias: np.ndarray, sizes: np.ndarray, m: int) -> np.ndarray:
    """Return each row's expert's row of `bias` (E, c; bfloat16 bits or float32), 0
    past the groups, float32 (moe.by_expert, moe.py:876-885: a one-hot product, exact
    here)."""
    b = _values(bias).reshape(len(sizes), -1)
    e = _expert_of_rows(sizes, m)
    return np.where((e >= 0)[:, None], b[np.maximum(e, 0)], np.float32(0))


def add_expert_bias(x: np.ndarray, bias: np.ndarray, sizes: np.ndarray) -> np.ndarray:
    """Return ``x + by_expert(bias)`` in x's dtype (moe.py:848-849,857-861): bfloat16
    bits, or float32 values for a float32 layer's x."""
    xf = _values(x).reshape(x.shape[0], -1)
    total = xf + by_expert(bias, sizes, x.shape[0])  # one float32 rounding
    return (total if _is_f32(x) else bf16.to_bf16(total)).reshape(x.shape)


def expert_sums(v: np.ndarray, sizes: np.ndarray) -> np.ndarray:
    """Return each expert's sum of its rows of v (float32 values, (m, c)), in float64:
    by_expert's gradient, the one-hot product's transpose (moe.py:876-885)."""
    e = _expert_of_rows(sizes, v.shape[0])
    out = np.zeros((len(sizes), v.shape[1]), np.float64)
    np.add.at(out, e[e >= 0], v[e >= 0].astype(np.float64))
    return out


def weighted_bias_rows(bias: np.ndarray, sizes: np.ndarray, row_weights: np.ndarray, m: int) -> np.ndarray:
    """Return ``weighted(by_expert(down_bias), weights)`` in the row weights' dtype
    (bfloat16 bits, or float32) (moe.py:869,922-925): each row's expert's bias times the
    row's weight, rounded."""
    w = _values(row_weights)[:, None]
    b = by_expert(bias, sizes, m) * w  # a float32 product
    return b if _is_f32(row_weights) else bf16.to_bf16(b)


# --- The experts' output norm -------------------------------------------------------


class Norm(NamedTuple):
    """The norm of each expert's output (MoEConfig.expert_norm, config.py:306): a
    NormalizationConfig (config.py:71-92)."""

    kind: str = "rmsnorm"  # or "layernorm"
    eps: float = 1e-6
    affine: bool = True
    bias: bool = False
    zero_centered: bool = False
    scale_input: bool = False


def _rounding(f32: bool):
    """The rounding of each of the norm's ops: to float32 (a float32 layer), else to
    bfloat16 (through float32, as the float32 result of a bfloat16 op is rounded)."""
    return (lambda a: np.asarray(a, np.float64).astype(np.float32)) if f32 else bf16.round_f32


def _norm_parts(norm: Norm, v: np.ndarray, scale, nbias, f32: bool = False):
    """The forward's pieces in float64 with the reference's roundings (layers/norm.py:
    55-78 in bfloat16 compute, or float32 with `f32`): gain, x (the normalization's
    input), u, rs, xn (its rounded output) and n (the norm's output)."""
    r = _rounding(f32)
    d = v.shape[-1]
    gain = np.ones(d)
    if norm.affine:
        s_ = _values(scale).astype(np.float64)
        gain = r(1.0 + s_).astype(np.float64) if norm.zero_centered else s_
    x = r(v * gain).astype(np.float64) if norm.affine and norm.scale_input else v
    u = x - x.mean(-1, keepdims=True) if norm.kind == "layernorm" else x
    rs = 1.0 / np.sqrt((u * u).mean(-1, keepdims=True) + norm.eps)
    xn = r(u * rs).astype(np.float64)
    n = xn
    if norm.affine and not norm.scale_input:
        n = r(n * gain).astype(np.float64)
    if norm.bias:
        n = r(n + _values(nbias).astype(np.float64)).astype(np.float64)
    return gain, x, u, rs, xn, n


def _norm_input(y: np.ndarray, sizes: np.ndarray, down_bias) -> np.ndarray:
    v = _values(y).astype(np.float64)
    if down_bias is not None:
        v = _rounding(_is_f32(y))(v + by_expert(down_bias, sizes, y.shape[0])).astype(np.float64)
    return v


def expert_norm_forward(norm: Norm, y: np.ndarray, sizes: np.ndarray, row_weights: np.ndarray,
                        scale=None, nbias=None, down_bias=None) -> np.ndarray:
    """Return ``weighted(norm(y + down_bias), weights)`` of the down GEMM's rows y (m, d)
    (moe.py:871-872) in y's dtype (bfloat16 bits, or float32 values: then every rounding
    float32's); rows past the groups 0."""
    f32 = _is_f32(y)
    v = _norm_input(y, sizes, down_bias)
    *_, n = _norm_parts(norm, v, scale, nbias, f32)
    w = _values(row_weights).astype(np.float64)[:, None]
    live = (_expert_of_rows(sizes, y.shape[0]) >= 0)[:, None]
    out = np.where(live, n * w, 0.0).astype(np.float32)
    return out if f32 else bf16.to_bf16(out)


def expert_norm_backward(norm: Norm, g: np.ndarray, y: np.ndarray, sizes: np.ndarray,
                         row_weights: np.ndarray, scale=None, nbias=None, down_bias=None):
    """Return the VJP of `expert_norm_forward` given each row's upstream gradient g
    (m, d) (its token's dy), in y's dtype: dv (m, d) and d weights (m,) as bfloat16 bits
    (float32 values for a float32 y), d scale and d bias (d,) as float64 sums (None
    where the norm has none); jax's VJP of the chain, the normalization's in float32
    (here float64)."""
    f32 = _is_f32(y)
    r = _rounding(f32)
    v = _norm_input(y, sizes, down_bias)
    gain, x, u, rs, xn, n = _norm_parts(norm, v, scale, nbias, f32)
    gf = _values(g).astype(np.float64)
    w = _values(row_weights).astype(np.float64)[:, None]
    live = (_expert_of_rows(sizes, y.shape[0]) >= 0)[:, None]
    gf = np.where(live, gf, 0.0)
    d_w = r(r(gf * n).sum(-1)).astype(np.float64)
    dn = r(gf * w).astype(np.float64)
    d_bias = dn.sum(0) if norm.bias else None
    d_scale = None
    dxn = dn
    if norm.affine and not norm.scale_input:
        d_scale = r(dn * xn).sum(0)
        dxn = r(dn * gain).astype(np.float64)
    mean_dx = dxn.mean(-1, keepdims=True) if norm.kind == "layernorm" else 0.0
    mean_dxu = (dxn * u).mean(-1, keepdims=True)
    dx = r(rs * (dxn - mean_dx - u * rs * rs * mean_dxu)).astype(np.float64)
    if norm.affine and norm.scale_input:
        d_scale = r(dx * v).sum(0)
        dx = r(dx * gain).astype(np.float64)
    dv = np.where(live, dx, 0.0).astype(np.float32)
    d_w = np.where(live[:, 0], d_w, 0.0).astype(np.float32)
    if f32:
        return dv, d_w, d_scale, d_bias
    return bf16.to_bf16(dv), bf16.to_bf16(d_w), d_scale, d_bias


# --- The layer: routed -> experts, forward and backward ----------------------------


PASSES = ("fprop", "dgrad", "wgrad")


class Saved(NamedTuple):
    """What the layer's backward takes of its forward (grouped_blockscaled.py:84)."""

    sorted: Sorted
    row_weights: np.ndarray
    projected: np.ndarray  # bf16 bits (m, p f), the up bias added
    h: np.ndarray  # bf16 bits (m, f)
    x_m: Blocks | None
    up_n: Blocks | None
    h_m: Blocks | None
    down_n: Blocks | None
    passes: tuple[bool, bool, bool] = (True, True, True)
    y: np.ndarray | None = None  # with a norm: the down GEMM's rows, bf16 bits (m, d)


def _ones(m: int, f32: bool) -> np.ndarray:
    """Weights of 1 in the layer's dtype (the unweighted activation before a norm)."""
    ones = np.ones(m, np.float32)
    return ones if f32 else bf16.to_bf16(ones)


def _passes(fmt: str, passes) -> tuple[bool, bool, bool]:
    if fmt not in ("mxfp8", "mxfp8_2d"):
        return False, False, False
    chosen = PASSES if passes is None else tuple(passes)
    return tuple(q in chosen for q in PASSES)


def layer_forward(
    z: np.ndarray,
    idx: np.ndarray,
    weights: np.ndarray,
    up: np.ndarray,
    down: np.ndarray,
    ffn: Ffn = Ffn(),
    fmt: str = "mxfp8",
    passes=None,
    up_bias: np.ndarray | None = None,
    down_bias: np.ndarray | None = None,
    norm: Norm | None = None,
    norm_scale: np.ndarray | None = None,
    norm_bias: np.ndarray | None = None,
    exact: bool = False,
) -> tuple[np.ndarray, Saved]:
    """Return the MoE's routed experts' output (t, d) as bfloat16 bits, and what the
    backward takes: ``routed`` (moe.py:733-773) on one device with picked rows in and
    summed rows out, each grouped GEMM in MXFP8 (`fmt` "mxfp8") or bfloat16
    ("compute"); with `passes`, only those GEMMs in MXFP8 (grouped_blockscaled.py:
    167-211); with biases, moe.py:857-870.

    Args:
        z: tokens, bfloat16 bits (t, d).
        idx: each token's k experts, int (t, k).
        weights: their weights, bfloat16 bits (t, k).
        up: the experts' up kernels, bfloat16 bits (E, d, f, p): p = 2 gated, 1 plain.
        down: the experts' down kernels, bfloat16 bits (E, f, d).
        ffn: the activation.
        fmt: "mxfp8", "mxfp8_2d" (each W with a scale per 32 x 32 tile shared by its
            copies, blockscaled.MXFP8_2D, blockscaled.py:306-309) or "compute".
        passes: the GEMMs in `fmt`, of PASSES; None for all.
        up_bias: bfloat16 bits (E, f, p) or None; down_bias: (E, d) or None.
        norm: the experts' output norm (moe.py:871-872), with its scale and bias
            (bfloat16 bits (d,)); the activation is then unweighted.
        exact: every GEMM and token sum in float64, rounded once (the quantization and
            rounding points unchanged): the exact restatement float32 orders are
            measured against.
    """
    t, k = idx.shape
    e, d, f, p = up.shape
    f32 = np.asarray(z).dtype == np.float32
    gemm_out = "f32" if f32 else "bf16"
    s = sort_by_expert(idx, e)
    m = t * k
    filled = int(s.sizes.sum())
    tokens = s.order // k
    inside = (idx.reshape(-1) >= 0) & (idx.reshape(-1) < e)
    w_flat = np.asarray(weights).reshape(-1)
    kept = np.where(inside, w_flat, w_flat.dtype.type(0)).astype(w_flat.dtype)
    row_weights = kept[s.order]
    up2 = np.asarray(up).reshape(e, d, f * p)
    x_m = up_n = h_m = down_n = None
    fprop, dgrad, wgrad = _passes(fmt, passes)
    tiles = fmt == "mxfp8_2d"
    # rows padded by 0 to whole tiles of 128 (grouped_blockscaled.py:122-128)
    if fprop or wgrad:
        x_k, x_m = mxfp8.quantized_twice(z, filled, True, index=tokens, height=whole(m))
    if fprop or dgrad:
        up_n, up_k = mxfp8.quantized_twice(up2, d, tiles=tiles)
        down_n, down_k = mxfp8.quantized_twice(down, f, tiles=tiles)
    if fprop:
        projected = rows_mx(x_k, up_k, s.sizes, out=gemm_out, height=m, exact=exact)
    else:
        projected = ragged_dot_bf16(z[tokens], up2, s.sizes, exact=exact)
    if up_bias is not None:
        projected = add_expert_bias(projected, up_bias, s.sizes)
    act_weights = row_weights if norm is None else _ones(m, f32)
    h = weighted_units(ffn, projected.reshape(m, f, p), act_weights)
    if fprop or wgrad:
        h_k, h_m = mxfp8.quantized_twice(h, filled, True, height=whole(m))
    if fprop:
        y = rows_mx(h_k, down_k, s.sizes, out=gemm_out, height=m, exact=exact)
    else:
        y = ragged_dot_bf16(h, down, s.sizes, exact=exact)
    y_rows = None
    if norm is not None:
        y_rows = y
        y = expert_norm_forward(norm, y_rows, s.sizes, row_weights, norm_scale, norm_bias, down_bias)
    out = sum_by_token(y, s.inverse.reshape(t, k), out_bf16=not f32, exact=exact)
    if down_bias is not None and norm is None:
        b = weighted_bias_rows(down_bias, s.sizes, row_weights, m)
        bsum = sum_by_token(b, s.inverse.reshape(t, k), out_bf16=not f32, exact=exact)
        total = _values(out) + _values(bsum)
        out = total if f32 else bf16.to_bf16(total)
    return out, Saved(s, row_weights, projected, h, x_m, up_n, h_m, down_n, (fprop, dgrad, wgrad),
                      y_rows)


def layer_backward(
    saved: Saved, dy: np.ndarray, z: np.ndarray, up: np.ndarray, down: np.ndarray,
    k: int, ffn: Ffn = Ffn(), fmt: str = "mxfp8",
    up_bias: np.ndarray | None = None, down_bias: np.ndarray | None = None,
    norm: Norm | None = None, norm_scale: np.ndarray | None = None,
    norm_bias: np.ndarray | None = None, exact: bool = False,
) -> dict[str, np.ndarray]:
    """Return the gradients of `layer_forward`'s output, dy (t, d) bfloat16 bits, to
    z, the weights, up and down (bfloat16 bits), to the biases (float64 sums), and
    between the GEMMs "dh" (m, f) and "dp" (m, p f) (bfloat16 bits):
    grouped_blockscaled._backward (:191-211) for each GEMM, weighted_units' VJP between
    them, and the gathers' and biases' VJPs (moe.py:857-870,1018-1021,1060-1063). The
    passes are the forward's; `exact` as `layer_forward`'s."""
    s = saved.sorted
    t = dy.shape[0]
    e, d, f, p = up.shape
    m = t * k
    f32 = np.asarray(dy).dtype == np.float32
    gemm_out = "f32" if f32 else "bf16"
    filled = int(s.sizes.sum())
    tokens = s.order // k
    up2 = np.asarray(up).reshape(e, d, f * p)
    fprop, dgrad, wgrad = saved.passes
    grads = {}
    if norm is not None:
        dv, d_norm_w, d_scale, d_nbias = expert_norm_backward(
            norm, dy[tokens], saved.y, s.sizes, saved.row_weights, norm_scale, norm_bias, down_bias)
        grads.update(norm_scale=d_scale, norm_bias=d_nbias)
        if down_bias is not None:
            grads["down_bias"] = expert_sums(_values(dv), s.sizes)
        dy_rows = dv
        if dgrad or wgrad:
            dy_n, dy_m = mxfp8.quantized_twice(dv, filled, True, height=whole(m))
    else:
        if dgrad or wgrad:
            dy_n, dy_m = mxfp8.quantized_twice(dy, filled, True, index=tokens, height=whole(m))
        dy_rows = dy[tokens]
    if dgrad:
        dh = rows_mx(dy_n, saved.down_n, s.sizes, out=gemm_out, height=m, exact=exact)
    else:
        dh = ragged_dot_bf16(dy_rows, np.ascontiguousarray(np.swapaxes(down, 1, 2)), s.sizes,
                             exact=exact)
    if wgrad:
        d_down = contract_mx(saved.h_m, dy_m, s.sizes, out=gemm_out, exact=exact)
    else:
        d_down = weight_grad_bf16(saved.h, dy_rows, s.sizes, exact=exact)
    act_weights = saved.row_weights if norm is None else _ones(m, f32)
    dp, d_rows_w = weighted_units_backward(ffn, saved.projected.reshape(m, f, p), act_weights, dh)
    if norm is not None:
        d_rows_w = d_norm_w
    dp = dp.reshape(m, f * p)
    if dgrad or wgrad:
        dp_n, dp_m = mxfp8.quantized_twice(dp, filled, True, height=whole(m))
    if dgrad:
        dx = rows_mx(dp_n, saved.up_n, s.sizes, out=gemm_out, height=m, exact=exact)
    else:
        dx = ragged_dot_bf16(dp, np.ascontiguousarray(np.swapaxes(up2, 1, 2)), s.sizes,
                             exact=exact)
    if wgrad:
        d_up = contract_mx(saved.x_m, dp_m, s.sizes, out=gemm_out, exact=exact)
    else:
        d_up = weight_grad_bf16(z[tokens], dp, s.sizes, exact=exact)
    if up_bias is not None:
        grads["up_bias"] = expert_sums(_values(dp), s.sizes).reshape(e, f, p)
    if down_bias is not None and norm is None:
        # weighted(b_rows, w)'s VJP: to b_rows ct * w, to w sum_c ct * b_rows (products
        # in the layer's dtype, summed in float32); ct = dy at each row's token
        rd = (lambda a: np.asarray(a, np.float32)) if f32 else bf16.round_f32
        g = _values(dy_rows)
        w = _values(saved.row_weights)[:, None]
        b_rows = by_expert(down_bias, s.sizes, m)
        live = (_expert_of_rows(s.sizes, m) >= 0)[:, None]
        grads["down_bias"] = expert_sums(np.where(live, rd(g * w), 0), s.sizes)
        extra = rd(rd(g * b_rows).sum(-1, dtype=np.float32))
        total = _values(d_rows_w) + extra
        d_rows_w = total if f32 else bf16.to_bf16(total)
    dz = sum_by_token(dx, s.inverse.reshape(t, k), out_bf16=not f32, exact=exact)
    d_weights = d_rows_w[s.inverse].reshape(t, k)
    grads.update(z=dz, weights=d_weights, up=d_up.reshape(e, d, f, p), down=d_down, dh=dh, dp=dp)
    return grads
