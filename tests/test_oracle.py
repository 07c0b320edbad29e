"""Pins of the CPU oracle (``oracle/``), independent of this repository's kernels:
torch's own float8/bfloat16 casts, exact rational arithmetic, brute force on tiny
inputs, and the invariants bux's own tests hold for this path
(tests/test_grouped.py, tests/test_grouped_mxfp8.py, tests/test_precision.py in the
reference). Each check is chosen so that a plausible slip in the oracle (a dropped
term, a wrong sign, an off-by-one exponent, a transposed operand) fails it."""

import math
from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import bf16, moe, mxfp8

ALL_BF16 = np.arange(65536, dtype=np.uint32).astype(np.uint16)
FINITE = ALL_BF16[np.isfinite(bf16.to_f32(ALL_BF16))]


# --- bfloat16 ---------------------------------------------------------------------


def test_bf16_widening_is_torchs_for_every_pattern():
    want = torch.from_numpy(ALL_BF16.view(np.int16)).view(torch.bfloat16).float().numpy()
    got = bf16.to_f32(ALL_BF16)
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


def test_bf16_rounding_is_torchs():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        (rng.standard_normal(200000) * 10.0 ** rng.integers(-40, 38, 200000)).astype(np.float32),
        # ties: exactly halfway between two bfloat16 values, both parities
        ((np.arange(1, 4000, dtype=np.uint32) << 16) | 0x8000).view(np.float32),
        np.array([3.4e38, -3.4e38, 1e-45, -1e-45, 0.0, -0.0], np.float32),
    ])
    x = x[np.isfinite(x)].astype(np.float32)
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(bf16.to_bf16(x), want)


# --- E4M3 and the quantizer -----------------------------------------------------------


def _in_range_bf16() -> np.ndarray:
    v = bf16.to_f32(FINITE)
    return v[np.abs(v) <= 448]


def test_e4m3_rounding_is_torchs_for_every_bf16_in_range():
    """torch's float32 -> float8_e4m3fn cast is an independent RNE implementation;
    the quantizer only ever casts values already clipped to [-448, 448]."""
    v = _in_range_bf16()
    want = torch.from_numpy(v).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    np.testing.assert_array_equal(mxfp8.to_e4m3fn(v), want)
    # negatives that round to zero keep their sign: 0x80
    assert mxfp8.to_e4m3fn(np.array([-1e-4, -0.0], np.float32)).tolist() == [0x80, 0x80]


def test_e4m3_rounding_is_the_nearest_even_code():
    """Brute force: the nearest of the 254 finite codes' values, ties to an even code."""
    codes = np.arange(256)
    values = mxfp8.e4m3_values()
    finite = codes[~np.isnan(values) & (codes < 128)]
    rng = np.random.default_rng(1)
    v = _in_range_bf16()
    v = v[rng.choice(v.size, 3000, replace=False)]
    for x in v:
        d = np.abs(values[finite].astype(np.float64) - abs(float(x)))
        best = finite[d == d.min()]
        code = int(best[best % 2 == 0][0]) if best.size > 1 else int(best[0])
        code |= 0x80 if math.copysign(1, x) < 0 else 0
        assert mxfp8.to_e4m3fn(np.array([x], np.float32))[0] == code, x


def test_e4m3_values_are_torchs():
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    want = codes.view(torch.float8_e4m3fn).float().numpy()
    got = mxfp8.e4m3_values()
    np.testing.assert_array_equal(np.isnan(got), np.isnan(want))
    ok = ~np.isnan(want)
    np.testing.assert_array_equal(got[ok], want[ok])


def test_a_tile_takes_the_least_power_of_two_that_fits_it():
    """mx_tiles_twice: brute force over exponents for each 32 x 32 tile; both copies
    hold the same codes, transposed, and their scale bytes repeat the tile's."""
    rng = np.random.default_rng(10)
    w = (rng.standard_normal((96, 64)) * rng.choice([1e-3, 1.0, 50.0], (96, 64))).astype(np.float32)
    rows, cols = mxfp8.mx_tiles_twice(w)
    assert (cols.values == rows.values.T).all()
    for i in range(3):
        for j in range(2):
            tile = w[32 * i:32 * i + 32, 32 * j:32 * j + 32]
            amax = float(np.abs(tile).max())
            e = min(e for e in range(-126, 127) if amax <= 448.0 * 2.0**e)
            assert (rows.scales[32 * i:32 * i + 32, j] == e + 127).all()
            assert (cols.scales[32 * j:32 * j + 32, i] == e + 127).all()
    deq = mxfp8.dequantized(rows).astype(np.float64)
    assert np.allclose(deq, w, rtol=2.0**-4, atol=2.0**-9 * np.abs(w).max())


def test_tiles_of_one_magnitude_quantize_as_row_blocks_do():
    """Where every row block of a tile holds the tile's largest magnitude, the tile's
    scale is each block's: the codes equal the 1 x 32 copies'."""
    rng = np.random.default_rng(11)
    w = rng.standard_normal((64, 96)).astype(np.float32)
    w[:, ::32] = np.abs(w).reshape(64, 3, 32).max(-1).reshape(2, 32, 3).max(1).repeat(32, 0)
    rows, _ = mxfp8.mx_tiles_twice(w)
    plain = mxfp8.mx_quantize(w)
    assert (rows.values == plain.values).all() and (rows.scales == plain.scales).all()


def test_e8m0_values_are_torchs():
    """Every E8M0 byte (byte 0: 2^-127, 255: NaN) as torch's float8_e8m0fnu widens it."""
    want = torch.arange(256, dtype=torch.uint8).view(torch.float8_e8m0fnu).float().numpy()
    got = mxfp8.e8m0_values()
    assert np.array_equal(got[:255], want[:255]) and np.isnan(got[255]) and np.isnan(want[255])


def test_mxfp8_rows_pack_into_bytes_and_back():
    """The reference's round trip (tests/test_precision.py:344-352): 8 rows of 64 pack
    into 66 bytes each, codes then scale bytes, and unpack to the same values."""
    x = (np.random.default_rng(8).standard_normal((8, 64)) * 3).astype(np.float32)
    blocks = mxfp8.mx_quantize(x)
    packed = mxfp8.mx_packed(blocks)
    assert packed.dtype == np.uint8 and packed.shape == (8, 64 + 2)
    assert (packed[:, :64] == blocks.values).all() and (packed[:, 64:] == blocks.scales).all()
    back = mxfp8.mx_unpacked(packed, 64)
    assert np.array_equal(mxfp8.dequantized(back), mxfp8.dequantized(blocks))


def test_tokens_from_mxfp8_are_exact_bfloat16():
    """from_mxfp8: each code (torch's float8_e4m3fn cast) times its scale is a bfloat16
    exactly wherever the product is a normal bfloat16 (4 significant bits), for every
    byte pattern of a row and every scale byte 0..255; below that, bfloat16's
    subnormals round it, as the reference's astype does."""
    rng = np.random.default_rng(9)
    packed = rng.integers(0, 256, (256, 64 + 2), dtype=np.uint8)
    packed[:, 64] = np.arange(256, dtype=np.uint8)  # every scale byte
    got = bf16.to_f32(mxfp8.from_mxfp8(packed, 64)).astype(np.float64)
    codes = torch.from_numpy(packed[:, :64].copy()).view(torch.float8_e4m3fn).double().numpy()
    scale = np.repeat(torch.from_numpy(packed[:, 64:].copy()).view(torch.float8_e8m0fnu)
                      .double().numpy(), 32, axis=-1)
    want = codes * scale
    normal = np.isfinite(want) & (np.abs(want) < 3e38) & ((want == 0) | (np.abs(want) >= 2.0**-126))
    assert np.array_equal(got[normal], want[normal])  # exact: no rounding happened
    assert np.isnan(got[~np.isfinite(want) & np.isnan(want)]).all()


def test_ceil_log2_is_exact_for_every_bf16_block_maximum():
    """e = the least integer with 2^e >= fl32(amax / 448), clipped to [-126, 126],
    computed from the quotient's exact rational value (not from its bits)."""
    amax = bf16.to_f32(FINITE)
    amax = amax[~np.signbit(amax)]  # |b|'s max is never -0
    q = amax / np.float32(448.0)
    got = mxfp8.ceil_log2(q)
    for qi, gi in zip(q.tolist(), got.tolist()):
        if qi == 0:
            want = -126
        else:
            r = Fraction(qi)
            e = math.floor(math.log2(qi)) - 2
            while Fraction(2) ** e < r:
                e += 1
            want = min(max(e, -126), 126)
        assert gi == want, (qi, gi, want)


def test_a_block_takes_the_least_power_of_two_that_fits_it():
    rng = np.random.default_rng(2)
    x = (rng.standard_normal((64, 256)) * 10.0 ** rng.integers(-30, 30, (64, 1))).astype(np.float32)
    x = bf16.round_f32(x)
    values, scales = mxfp8.in_e4m3(x, "rows")
    blocks = x.reshape(64, 8, 32)
    amax = np.abs(blocks).max(-1).astype(np.float64)
    e = scales.astype(np.int64) - 127
    assert (amax <= 448 * 2.0 ** e).all()
    assert ((amax > 448 * 2.0 ** (e - 1)) | (e == -126)).all()
    # dequantized is within half an E4M3 step (3 mantissa bits) of each value
    deq = mxfp8.dequantized(mxfp8.Blocks(values, scales)).astype(np.float64)
    step = np.maximum(2.0 ** (np.floor(np.log2(np.maximum(np.abs(x), 1e-300))) - 3),
                      2.0 ** -9 * np.repeat(2.0 ** e, 32, axis=-1))
    assert (np.abs(deq - x) <= step / 2 + 1e-300).all()


def test_a_block_of_zeros_gets_byte_1():
    """E8M0 has no 0: a zero block's scale is 2^-126 (test_grouped_mxfp8.py:62-68)."""
    values, scales = mxfp8.in_e4m3(np.zeros((2, 64), np.float32))
    assert (scales == 1).all() and (values == 0).all()


def test_the_column_copy_is_the_transposes_row_copy():
    rng = np.random.default_rng(3)
    x = bf16.round_f32(rng.standard_normal((64, 96)).astype(np.float32))
    v_cols, e_cols = mxfp8.in_e4m3(x, "columns")
    v_t, e_t = mxfp8.in_e4m3(np.ascontiguousarray(x.T), "rows")
    np.testing.assert_array_equal(v_cols.T, v_t)
    np.testing.assert_array_equal(e_cols.T, e_t)


def test_rows_past_filled_quantize_as_zero_and_picked_rows_as_their_copy():
    rng = np.random.default_rng(4)
    tokens = bf16.to_bf16(rng.standard_normal((40, 64)).astype(np.float32))
    index = rng.integers(0, 40, 256)
    got = mxfp8.quantized_twice(tokens, 200, True, index=index)
    want = mxfp8.quantized_twice(tokens[index], 200, True)
    for a, b in zip(got, want):
        np.testing.assert_array_equal(a.values, b.values)
        np.testing.assert_array_equal(a.scales, b.scales)
    rows, cols = got
    assert (rows.values[200:] == 0).all() and (rows.scales[200:] == 1).all()
    assert (cols.values[:, 200:] == 0).all()


# --- The token path ------------------------------------------------------------------


def _brute_sort(idx, e):
    flat = [int(v) if 0 <= v < e else e for v in np.asarray(idx).reshape(-1)]
    order = sorted(range(len(flat)), key=lambda i: (flat[i], i))
    sizes = [sum(1 for v in flat if v == g) for g in range(e)]
    return order, sizes


@pytest.mark.parametrize("sizes", [[70, 0, 100, 3, 77], [0, 130, 1, 3, 256, 0, 300, 100]])
def test_sort_by_expert_on_the_references_size_patterns(sizes):
    rng = np.random.default_rng(5)
    flat = np.repeat(np.arange(len(sizes)), sizes)
    rng.shuffle(flat)
    idx = flat.reshape(-1, 1)
    s = moe.sort_by_expert(idx, len(sizes))
    order, want_sizes = _brute_sort(idx, len(sizes))
    assert s.order.tolist() == order
    assert s.sizes.tolist() == want_sizes == sizes
    assert (s.order[s.inverse] == np.arange(flat.size)).all()
    assert s.offsets.tolist() == (np.cumsum(sizes) - sizes).tolist()


def test_sort_by_expert_puts_out_of_range_picks_last():
    idx = np.array([[3, -1], [0, 7], [2, 3], [5, 0]])
    s = moe.sort_by_expert(idx, 4)
    order, sizes = _brute_sort(idx, 4)
    assert s.order.tolist() == order and s.sizes.tolist() == sizes
    assert set(s.order[-3:].tolist()) == {1, 3, 6}


def test_the_tiles_of_rows_cover_each_groups_rows_once():
    """tests/test_grouped_mxfp8.py:31-41, on the oracle's tile list."""
    sizes = np.array([0, 130, 1, 3, 256, 0, 300, 100])
    m = 1024
    tiles = moe.tiles_of(sizes, m, 128)
    group_of = np.searchsorted(np.cumsum(sizes), np.arange(m), side="right")
    covered = np.full(m, -1)
    for group, lo, hi in tiles:
        assert lo == hi or lo // 128 == (hi - 1) // 128
        assert (covered[lo:hi] == -1).all() and (group_of[lo:hi] == group).all()
        covered[lo:hi] = group
    assert (covered >= 0).sum() == sizes.sum()
    assert len(tiles) == -(-m // 128) + len(sizes) - 1


def test_sum_by_token_is_the_transpose_of_token_rows():
    rng = np.random.default_rng(6)
    t, k, d, e = 50, 4, 16, 7
    idx = rng.integers(0, e, (t, k))
    s = moe.sort_by_expert(idx, e)
    z = rng.standard_normal((t, d))
    y = bf16.round_f32(rng.standard_normal((t * k, d)).astype(np.float32))
    rows = moe.token_rows(z, s.order, k)
    sums = moe.sum_by_token(y, s.inverse.reshape(t, k), out_bf16=False).astype(np.float64)
    np.testing.assert_allclose((rows * y).sum(), (z * sums).sum(), rtol=1e-6)
    # brute force
    for tok in range(t):
        want = sum(y[s.inverse[tok * k + j]].astype(np.float64) for j in range(k))
        np.testing.assert_allclose(sums[tok], want, rtol=1e-6, atol=1e-6)


def _blocks(rng, shape):
    x = rng.standard_normal(shape).astype(np.float32)
    if len(shape) == 3:
        parts = [mxfp8.mx_quantize(m) for m in x]
        return mxfp8.Blocks(np.stack([p.values for p in parts]), np.stack([p.scales for p in parts]))
    return mxfp8.mx_quantize(x)


def test_rows_multiply_each_groups_rows_by_its_matrix():
    """Brute force in float64 over dequantized codes, with the reference's sizes
    (empty groups, a group of one row, rows past the groups)."""
    rng = np.random.default_rng(7)
    sizes = np.array([0, 13, 1, 3, 25, 0, 30, 10])
    m, k, n = 100, 64, 24
    a, b = _blocks(rng, (m, k)), _blocks(rng, (8, n, k))
    got = moe.rows_mx(a, b, sizes, out="f32")
    ea = mxfp8.e4m3_values()[a.values].astype(np.float64) * np.repeat(2.0 ** (a.scales - 127.0), 32, -1)
    eb = mxfp8.e4m3_values()[b.values].astype(np.float64) * np.repeat(2.0 ** (b.scales - 127.0), 32, -1)
    ends = np.cumsum(sizes)
    for i in range(m):
        g = int(np.searchsorted(ends, i, side="right"))
        for j in range(n):
            want = 0.0 if g >= 8 else sum(ea[i, c] * eb[g, j, c] for c in range(k))
            assert abs(got[i, j] - want) <= 1e-5 * max(1.0, abs(want)), (i, j)
    assert (got[sizes.sum():] == 0).all()


def test_contract_sums_each_groups_rows_and_ignores_rows_past_them():
    rng = np.random.default_rng(8)
    sizes = np.array([70, 0, 100, 3, 77])
    m, d, f = 320, 32, 64
    a, b = _blocks(rng, (d, m)), _blocks(rng, (f, m))
    got = moe.contract_mx(a, b, sizes, out="f32")
    ea, eb = mxfp8.dequantized(a).astype(np.float64), mxfp8.dequantized(b).astype(np.float64)
    start = 0
    for g, size in enumerate(sizes):
        want = sum(np.outer(ea[:, i], eb[:, i]) for i in range(start, start + size)) if size else 0
        np.testing.assert_allclose(got[g], want, rtol=1e-5, atol=1e-4)
        start += size
    assert (got[1] == 0).all()
    # garbage past the groups changes nothing (tests/test_grouped.py:89-95)
    junk = a.values.copy()
    junk[:, sizes.sum():] = 0x7E
    np.testing.assert_array_equal(moe.contract_mx(mxfp8.Blocks(junk, a.scales), b, sizes, "f32"), got)


# torch's own activations (library routines, differentiated by autograd): the oracle's
# closed forms and hand-derived derivatives are checked against them.
TORCH_ACTS = {
    "swish": torch.nn.functional.silu,
    "quick_gelu": lambda x: x * torch.sigmoid(moe.QUICK_GELU_ALPHA * x),
    "relu": torch.relu,
    "relu2": lambda x: torch.relu(x) ** 2,
    "gelu": torch.nn.functional.gelu,
    "gelu_tanh": lambda x: torch.nn.functional.gelu(x, approximate="tanh"),
    "sigmoid": torch.sigmoid,
    "tanh": torch.tanh,
    # jax.nn.softplus is logaddexp(x, 0) everywhere; torch's turns linear past its
    # threshold (20 by default), so the threshold is raised past the range tested
    "softplus": lambda x: torch.nn.functional.softplus(x, threshold=100.0),
    "situ": lambda x: 4.0 * torch.tanh(x / 4.0) * torch.sigmoid(x),
}


@pytest.mark.parametrize("name", moe.ACTIVATIONS)
def test_each_activation_and_its_derivative_are_torchs(name):
    """functional.py:12-40's activations: the oracle's values and derivatives against
    torch's functions and autograd in float64, over [-30, 30], at 0 (relu's gradient
    0 there, as jax.nn.relu's) and at tiny magnitudes."""
    x = np.concatenate([np.linspace(-30.0, 30.0, 6001), [0.0, 1e-30, -1e-30, 1e-8, -1e-8]])
    a, da = moe._act(name, x)
    xt = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    y = TORCH_ACTS[name](xt)
    y.sum().backward()
    np.testing.assert_allclose(a, y.detach().numpy(), rtol=1e-10, atol=1e-14)
    np.testing.assert_allclose(da, xt.grad.numpy(), rtol=1e-8, atol=1e-14)


def _textbook(name, alpha):
    """functional.py:12-40's activations as written there, in mpmath."""
    import mpmath as mp
    sig = lambda v: 1 / (1 + mp.exp(-v))  # noqa: E731
    return {
        "swish": lambda v: v * sig(v),
        "quick_gelu": lambda v: v * sig(alpha * v),
        "relu": lambda v: mp.mpf(max(v, 0)),
        "relu2": lambda v: mp.mpf(max(v, 0)) ** 2,
        "gelu": lambda v: v * (1 + mp.erf(v / mp.sqrt(2))) / 2,
        "gelu_tanh": lambda v: v * (1 + mp.tanh(mp.sqrt(2 / mp.pi) * (v + mp.mpf("0.044715") * v ** 3))) / 2,
        "sigmoid": sig,
        "tanh": mp.tanh,
        "softplus": lambda v: mp.log(1 + mp.exp(v)),
        "situ": lambda v: 4 * mp.tanh(v / 4) * sig(v),
    }[name]


@pytest.mark.parametrize("f32", [False, True])
@pytest.mark.parametrize("name", moe.ACTIVATIONS)
def test_each_activation_holds_its_relative_precision_in_the_tails(name, f32):
    """The oracle's values and derivatives to 1e-12 relative of the textbook functions
    evaluated in 400-digit arithmetic (derivatives by mpmath's numerical differentiation),
    from x = -700 to 300: e^x-sized values far in the negative tail, where a
    (1 + tanh) / 2 or 1 + erf form cancels to 0 (values below float64's range, 1e-300,
    are taken as 0)."""
    import mpmath as mp
    alpha = float(np.float32(1.702)) if f32 else moe.QUICK_GELU_ALPHA
    lo = {"gelu_tanh": -12.0, "gelu": -30.0}.get(name, -700.0)
    x = np.array([v for v in (-700, -300, -120, -87, -60, -40, -30, -20, -12, -9, -6, -3, -0.5,
                              0.3, 2.5, 7, 15, 40, 90, 300) if v >= lo], np.float64)
    a, da = moe._act(name, x, f32)
    f = _textbook(name, mp.mpf(alpha))
    with mp.workdps(400):
        want = np.array([float(f(mp.mpf(v))) for v in x])
        dwant = np.array([float(mp.diff(f, mp.mpf(v))) for v in x])
    np.testing.assert_allclose(a, want, rtol=1e-12, atol=1e-300)
    np.testing.assert_allclose(da, dwant, rtol=1e-12, atol=1e-300)


FFNS = [
    # (ffn, p): p = 2 gated (gated_mlp), 1 plain (mlp)
    (moe.Ffn(), 2),
    (moe.Ffn("quick_gelu", 7.0, 1.0), 2),  # gpt-oss
    (moe.Ffn("situ", None, 0.0, 6.0), 2),  # SiTU-GLU with its soft cap
    (moe.Ffn("gelu_tanh", 3.0, 0.5, 5.0), 2),
    (moe.Ffn("sigmoid", 0.0), 2),  # a clamp at 0: every up at the limit or beyond
    (moe.Ffn("relu2"), 1),
    (moe.Ffn("gelu", 4.0, 0.0, 3.0), 1),
    (moe.Ffn("softplus"), 1),
    (moe.Ffn("tanh", None, 0.0, 2.0), 1),
    (moe.Ffn("relu", 2.0), 1),
]


def _torch_units(ffn, pt, wt, alpha=None):
    """weighted_units in torch float64: mlp.activate (layers/mlp.py:20-35), with
    maximum/minimum for the clip (their gradients 0.5 at a tie, as jax's); `alpha`
    replaces quick_gelu's."""
    up = pt[..., 0]
    if ffn.limit is not None:
        lim = torch.tensor(ffn.limit, dtype=torch.float64)
        up = torch.minimum(torch.maximum(up, -lim), lim)
    if ffn.up_softcap is not None:
        up = ffn.up_softcap * torch.tanh(up / ffn.up_softcap)
    act = TORCH_ACTS[ffn.activation]
    if alpha is not None and ffn.activation == "quick_gelu":
        act = lambda x: x * torch.sigmoid(alpha * x)  # noqa: E731
    if pt.shape[-1] == 1:
        return act(up) * wt[:, None]
    gate = pt[..., 1]
    if ffn.limit is not None:
        gate = torch.minimum(gate, torch.tensor(ffn.limit, dtype=torch.float64))
    return act(gate) * (up + ffn.up_offset) * wt[:, None]


@pytest.mark.parametrize("ffn,p", FFNS)
def test_the_activations_gradient_is_autograds(ffn, p):
    rng = np.random.default_rng(9)
    m, f = 64, 48
    pr = bf16.to_bf16((rng.standard_normal((m, f, p)) * 4).astype(np.float32))
    if ffn.limit is not None:  # ties with the clamp, both signs
        pr.reshape(-1)[:8] = bf16.to_bf16(np.array([1, -1, 1, -1, 2, -2, 0.5, 0], np.float32) * ffn.limit)
    w = bf16.to_bf16(rng.random(m).astype(np.float32))
    dh = bf16.to_bf16(rng.standard_normal((m, f)).astype(np.float32))
    dp, dw = moe.weighted_units_backward(ffn, pr, w, dh)
    pt = torch.tensor(bf16.to_f32(pr), dtype=torch.float64, requires_grad=True)
    wt = torch.tensor(bf16.to_f32(w), dtype=torch.float64, requires_grad=True)
    h = _torch_units(ffn, pt, wt)
    np.testing.assert_allclose(bf16.to_f32(moe.weighted_units(ffn, pr, w)), h.detach().numpy(),
                               rtol=8e-3, atol=1e-6)
    h.backward(torch.tensor(bf16.to_f32(dh), dtype=torch.float64))
    np.testing.assert_allclose(bf16.to_f32(dp), pt.grad.numpy(), rtol=8e-3, atol=1e-5)
    np.testing.assert_allclose(bf16.to_f32(dw), wt.grad.numpy(), rtol=8e-3, atol=1e-4)


@pytest.mark.parametrize("ffn,p", FFNS)
def test_a_float32_layers_activation_rounds_once_to_float32(ffn, p):
    """In float32 the activation and its gradients come from float32 inputs, each
    rounded once to float32 (quick_gelu's 1.702 its float32 value, functional.py:29):
    within float32's rounding of torch's float64 autograd, far inside bfloat16's."""
    rng = np.random.default_rng(19)
    m, f = 64, 48
    pr = (rng.standard_normal((m, f, p)) * 4).astype(np.float32)
    if ffn.limit is not None:  # ties with the clamp, both signs
        pr.reshape(-1)[:8] = np.array([1, -1, 1, -1, 2, -2, 0.5, 0], np.float32) * ffn.limit
    w = rng.random(m).astype(np.float32)
    dh = rng.standard_normal((m, f)).astype(np.float32)
    h = moe.weighted_units(ffn, pr, w)
    dp, dw = moe.weighted_units_backward(ffn, pr, w, dh)
    assert h.dtype == dp.dtype == dw.dtype == np.float32
    pt = torch.tensor(pr, dtype=torch.float64, requires_grad=True)
    wt = torch.tensor(w, dtype=torch.float64, requires_grad=True)
    ht = _torch_units(ffn, pt, wt, alpha=float(np.float32(1.702)))
    np.testing.assert_allclose(h, ht.detach().numpy(), rtol=1e-6, atol=1e-12)
    ht.backward(torch.tensor(dh, dtype=torch.float64))
    np.testing.assert_allclose(dp, pt.grad.numpy(), rtol=1e-6, atol=1e-12)
    np.testing.assert_allclose(dw, wt.grad.numpy(), rtol=1e-6, atol=1e-9)


def test_a_plain_ffn_takes_its_projection_with_or_without_the_last_axis():
    rng = np.random.default_rng(11)
    pr = bf16.to_bf16(rng.standard_normal((16, 32, 1)).astype(np.float32))
    w = bf16.to_bf16(rng.random(16).astype(np.float32))
    dh = bf16.to_bf16(rng.standard_normal((16, 32)).astype(np.float32))
    ffn = moe.Ffn("relu2")
    np.testing.assert_array_equal(moe.weighted_units(ffn, pr, w), moe.weighted_units(ffn, pr[..., 0], w))
    a, b = moe.weighted_units_backward(ffn, pr, w, dh), moe.weighted_units_backward(ffn, pr[..., 0], w, dh)
    np.testing.assert_array_equal(a[0][..., 0], b[0])
    np.testing.assert_array_equal(a[1], b[1])


NORMS = [
    moe.Norm("rmsnorm"),
    moe.Norm("layernorm", 1e-5, True, True),
    moe.Norm("rmsnorm", 1e-6, True, False, True),  # zero-centered gain (Qwen3-Next)
    moe.Norm("layernorm", 1e-6, True, True, False, True),  # scale_input
    moe.Norm("layernorm", 1e-6, False, False),  # no gain, no bias
]


def _torch_norm(norm, x, scale, bias):
    """layers/norm.py:55-78 in torch float64, from torch's own layer_norm / rms_norm."""
    gain = None
    if norm.affine:
        gain = 1 + scale if norm.zero_centered else scale
    if gain is not None and norm.scale_input:
        x = x * gain
    d = x.shape[-1]
    if norm.kind == "layernorm":
        x = torch.nn.functional.layer_norm(x, (d,), eps=norm.eps)
    else:
        x = torch.nn.functional.rms_norm(x, (d,), eps=norm.eps)
    if gain is not None and not norm.scale_input:
        x = x * gain
    if norm.bias:
        x = x + bias
    return x


@pytest.mark.parametrize("norm", NORMS)
def test_the_expert_norm_and_its_gradient_are_torchs(norm):
    """The oracle's norm (with its bfloat16 roundings) against torch's layer_norm and
    rms_norm and autograd in float64, with a down bias by expert and row weights; rows
    past the groups give 0."""
    rng = np.random.default_rng(13)
    m, d, sizes = 96, 64, np.array([30, 0, 50, 6])
    filled = int(sizes.sum())
    y = bf16.to_bf16((rng.standard_normal((m, d)) * 3 + 0.5).astype(np.float32))
    db = bf16.to_bf16(rng.standard_normal((4, d)).astype(np.float32))
    scale = bf16.to_bf16((1 + 0.3 * rng.standard_normal(d)).astype(np.float32))
    nb = bf16.to_bf16((0.2 * rng.standard_normal(d)).astype(np.float32))
    w = bf16.to_bf16(rng.random(m).astype(np.float32))
    g = bf16.to_bf16(rng.standard_normal((m, d)).astype(np.float32))
    out = moe.expert_norm_forward(norm, y, sizes, w, scale, nb, db)
    dv, dw, dscale, dbias = moe.expert_norm_backward(norm, g, y, sizes, w, scale, nb, db)

    def t(a, grad=False):
        return torch.tensor(bf16.to_f32(a), dtype=torch.float64, requires_grad=grad)

    yt, wt, st, bt = t(y[:filled], True), t(w[:filled], True), t(scale, True), t(nb, True)
    rows = torch.tensor(np.repeat(np.arange(4), sizes))
    x = yt + t(db)[rows]
    want = _torch_norm(norm, x, st, bt) * wt[:, None]
    want.backward(t(g[:filled]))

    def close(got, ref, tol):
        ref = ref.detach().numpy()
        err = np.linalg.norm(got - ref) / np.linalg.norm(ref)
        assert err < tol, err

    close(bf16.to_f32(out[:filled]), want, 1e-2)
    assert (out[filled:] == 0).all() and (dv[filled:] == 0).all() and (dw[filled:] == 0).all()
    close(bf16.to_f32(dv[:filled]), yt.grad, 2e-2)
    close(bf16.to_f32(dw[:filled]), wt.grad, 2e-2)
    if norm.affine:
        close(dscale, st.grad, 2e-2)
    if norm.bias:
        close(dbias, bt.grad, 2e-2)


@pytest.mark.parametrize("norm", NORMS)
def test_a_float32_expert_norm_rounds_only_to_float32(norm):
    """The oracle's norm of a float32 layer (float32 y, weights, biases and parameters)
    against torch's layer_norm / rms_norm and autograd in float64: within float32's
    rounding (each op rounded once to float32, not to bfloat16), rows past the groups 0,
    the results float32."""
    rng = np.random.default_rng(14)
    m, d, sizes = 96, 64, np.array([30, 0, 50, 6])
    filled = int(sizes.sum())
    f32 = np.float32
    y = (rng.standard_normal((m, d)) * 3 + 0.5).astype(f32)
    db = rng.standard_normal((4, d)).astype(f32)
    scale = (1 + 0.3 * rng.standard_normal(d)).astype(f32)
    nb = (0.2 * rng.standard_normal(d)).astype(f32)
    w = rng.random(m).astype(f32)
    g = rng.standard_normal((m, d)).astype(f32)
    out = moe.expert_norm_forward(norm, y, sizes, w, scale, nb, db)
    dv, dw, dscale, dbias = moe.expert_norm_backward(norm, g, y, sizes, w, scale, nb, db)
    assert out.dtype == dv.dtype == dw.dtype == np.float32

    def t(a, grad=False):
        return torch.tensor(a, dtype=torch.float64, requires_grad=grad)

    yt, wt, st, bt = t(y[:filled], True), t(w[:filled], True), t(scale, True), t(nb, True)
    rows = torch.tensor(np.repeat(np.arange(4), sizes))
    want = _torch_norm(norm, yt + t(db)[rows], st, bt) * wt[:, None]
    want.backward(t(g[:filled]))

    def close(got, ref, tol):
        ref = ref.detach().numpy()
        err = np.linalg.norm(got - ref) / np.linalg.norm(ref)
        assert err < tol, err

    # bfloat16 roundings anywhere would put these near 1e-3
    close(out[:filled], want, 2e-6)
    assert (out[filled:] == 0).all() and (dv[filled:] == 0).all() and (dw[filled:] == 0).all()
    close(dv[:filled], yt.grad, 2e-5)
    close(dw[:filled], wt.grad, 2e-5)
    if norm.affine:
        close(dscale, st.grad, 2e-5)
    if norm.bias:
        close(dbias, bt.grad, 2e-5)


def test_a_float32_layers_down_bias_adds_each_picks_weighted_bias():
    """The down bias of a float32 MXFP8 layer (moe.py:866-870): the output with it less
    the output without it is each token's sum of w b[e] over its picks, in float32; its
    gradient each expert's sum of dy w over its picks, and the weights' gradient gains
    dy . b[e] (float64 sums here, float32 there); the up bias's gradient each expert's
    sum of the layer's own d projected."""
    rng = np.random.default_rng(15)
    t, k, e, d, f = 64, 2, 4, 64, 64
    f32 = np.float32
    z = rng.standard_normal((t, d)).astype(f32)
    idx = np.stack([rng.choice(e, k, replace=False) for _ in range(t)])
    w = rng.random((t, k)).astype(f32)
    up = (rng.standard_normal((e, d, f, 2)) * 0.1).astype(f32)
    down = (rng.standard_normal((e, f, d)) * 0.1).astype(f32)
    dy = rng.standard_normal((t, d)).astype(f32)
    ub = rng.standard_normal((e, f, 2)).astype(f32)
    db = rng.standard_normal((e, d)).astype(f32)
    ffn = moe.Ffn()
    y0, s0 = moe.layer_forward(z, idx, w, up, down, ffn, up_bias=ub)
    y1, s1 = moe.layer_forward(z, idx, w, up, down, ffn, up_bias=ub, down_bias=db)
    g0 = moe.layer_backward(s0, dy, z, up, down, k, ffn, up_bias=ub)
    g1 = moe.layer_backward(s1, dy, z, up, down, k, ffn, up_bias=ub, down_bias=db)
    assert y1.dtype == np.float32 and g1["down_bias"].dtype == np.float64
    picks = (w.astype(np.float64)[:, :, None] * db.astype(np.float64)[idx]).sum(1)
    np.testing.assert_allclose(y1.astype(np.float64) - y0, picks, rtol=1e-5, atol=1e-5)
    want_db = np.zeros((e, d))
    np.add.at(want_db, idx.reshape(-1), np.repeat(dy.astype(np.float64), k, 0) * w.reshape(-1, 1))
    np.testing.assert_allclose(g1["down_bias"], want_db, rtol=1e-5, atol=1e-5)
    dots = (dy.astype(np.float64)[:, None, :] * db.astype(np.float64)[idx]).sum(-1)
    np.testing.assert_allclose(g1["weights"].astype(np.float64) - g0["weights"], dots,
                               rtol=1e-4, atol=1e-4)
    sorted_experts = np.sort(idx.reshape(-1), kind="stable")
    want_ub = np.zeros((e, f * 2))
    np.add.at(want_ub, sorted_experts, g1["dp"].astype(np.float64))
    np.testing.assert_allclose(g1["up_bias"].reshape(e, -1), want_ub, rtol=1e-6, atol=1e-9)


DENSE = [
    # (ffn, p, biased, norm)
    (moe.Ffn("quick_gelu", 7.0, 1.0), 2, False, None),
    (moe.Ffn("quick_gelu", 7.0, 1.0), 2, True, None),  # gpt-oss: clamped, with biases
    (moe.Ffn("relu2"), 1, False, None),
    (moe.Ffn("gelu", None, 0.0, 3.0), 1, True, None),
    (moe.Ffn(), 2, False, moe.Norm("rmsnorm")),
    (moe.Ffn("quick_gelu", 7.0, 1.0), 2, True, moe.Norm("layernorm", 1e-5, True, True)),
]


@pytest.mark.parametrize("f32", [False, True], ids=["bf16", "f32"])
@pytest.mark.parametrize("ffn,p,biased,norm", DENSE)
def test_the_sorted_layer_is_the_dense_one_with_gradients(ffn, p, biased, norm, f32):
    """``sorted`` equals ``dense`` with gradients (tests/test_moe.py:475-484): the
    oracle's layer, in the compute format (bfloat16, or float32 for float32 inputs),
    against every token through each of its experts one by one, differentiated by
    torch.autograd in float64; gated or plain, with the experts' up and down biases
    (moe.py:857-870) or without, with an expert norm or without. In float32 the layer
    is within float32's rounding (a bfloat16 rounding anywhere would show at 1e-3)."""
    rng = np.random.default_rng(10)
    t, k, e, d, f = 48, 2, 5, 32, 24
    cast = (lambda a: a.astype(np.float32)) if f32 else (lambda a: bf16.to_bf16(a.astype(np.float32)))
    z = cast(rng.standard_normal((t, d)))
    idx = np.stack([rng.choice(e, k, replace=False) for _ in range(t)])
    w = cast(rng.random((t, k)))
    up = cast(rng.standard_normal((e, d, f, p)) * 0.3)
    down = cast(rng.standard_normal((e, f, d)) * 0.3)
    dy = cast(rng.standard_normal((t, d)))
    ub = cast(rng.standard_normal((e, f, p))) if biased else None
    db = cast(rng.standard_normal((e, d))) if biased else None
    ns = cast(1 + 0.3 * rng.standard_normal(d)) if norm else None
    nb = cast(0.2 * rng.standard_normal(d)) if norm else None
    y, saved = moe.layer_forward(z, idx, w, up, down, ffn, fmt="compute", up_bias=ub, down_bias=db,
                                 norm=norm, norm_scale=ns, norm_bias=nb)
    grads = moe.layer_backward(saved, dy, z, up, down, k, ffn, fmt="compute", up_bias=ub,
                               down_bias=db, norm=norm, norm_scale=ns, norm_bias=nb)

    def tensor(a):
        return torch.tensor(moe._values(a), dtype=torch.float64, requires_grad=True)

    zt, wt, upt, downt = tensor(z), tensor(w), tensor(up), tensor(down)
    # quick_gelu's 1.702: a float32 constant times a float32 gate, 1.703125 for bfloat16
    alpha = float(np.float32(1.702)) if f32 else None
    ubt, dbt = (tensor(ub), tensor(db)) if biased else (None, None)
    nst, nbt = (tensor(ns), tensor(nb)) if norm else (None, None)
    out = torch.zeros(t, d, dtype=torch.float64)
    for tok in range(t):
        for j in range(k):
            g = int(idx[tok, j])
            pr = zt[tok] @ upt[g].reshape(d, p * f)
            if biased:
                pr = pr + ubt[g].reshape(p * f)
            if norm is None:
                h = _torch_units(ffn, pr.reshape(1, f, p), wt[tok, j].reshape(1), alpha)[0]
                row = h @ downt[g]
                if biased:
                    row = row + dbt[g] * wt[tok, j]
            else:  # moe.py:871-872: unweighted, biased, normed, then weighted
                h = _torch_units(ffn, pr.reshape(1, f, p), torch.ones(1, dtype=torch.float64),
                                 alpha)[0]
                row = h @ downt[g]
                if biased:
                    row = row + dbt[g]
                row = _torch_norm(norm, row, nst, nbt) * wt[tok, j]
            out = out.index_add(0, torch.tensor([tok]), row[None])
    out.backward(torch.tensor(moe._values(dy), dtype=torch.float64))
    if f32:
        assert y.dtype == grads["z"].dtype == grads["up"].dtype == np.float32
    fwd, bwd = (2e-6, 2e-5) if f32 else (1e-2, 2e-2)

    def close(got, want, rtol):
        got = bf16.to_f32(got).astype(np.float64) if got.dtype == np.uint16 else got
        want = want.detach().numpy()
        err = np.linalg.norm(got - want) / np.linalg.norm(want)
        assert err < rtol, err

    close(y, out, fwd)
    close(grads["z"], zt.grad, bwd)
    close(grads["weights"], wt.grad, bwd)
    close(grads["up"], upt.grad, bwd)
    close(grads["down"], downt.grad, bwd)
    if biased:
        close(grads["up_bias"], ubt.grad, bwd)
        close(grads["down_bias"], dbt.grad, bwd)
    if norm is not None:
        close(grads["norm_scale"], nst.grad, bwd)
        if norm.bias:
            close(grads["norm_bias"], nbt.grad, bwd)
        else:
            assert grads["norm_bias"] is None


def test_the_layer_with_no_pass_in_mxfp8_is_the_compute_layer_and_all_passes_the_default():
    """passes=() multiplies everything in bfloat16: fmt "compute", bit for bit; all
    three passes are the default (grouped_blockscaled.py:167-211)."""
    rng = np.random.default_rng(12)
    t, k, e, d, f = 40, 2, 4, 64, 32
    z = bf16.to_bf16(rng.standard_normal((t, d)).astype(np.float32))
    idx = np.stack([rng.choice(e, k, replace=False) for _ in range(t)])
    w = bf16.to_bf16(rng.random((t, k)).astype(np.float32))
    up = bf16.to_bf16((rng.standard_normal((e, d, f, 2)) * 0.3).astype(np.float32))
    down = bf16.to_bf16((rng.standard_normal((e, f, d)) * 0.3).astype(np.float32))
    dy = bf16.to_bf16(rng.standard_normal((t, d)).astype(np.float32))
    runs = {}
    for name, fmt, passes in (("compute", "compute", None), ("none", "mxfp8", ()),
                              ("all", "mxfp8", moe.PASSES), ("default", "mxfp8", None)):
        y, saved = moe.layer_forward(z, idx, w, up, down, fmt=fmt, passes=passes)
        runs[name] = (y, moe.layer_backward(saved, dy, z, up, down, k, fmt=fmt))
    for a, b in (("compute", "none"), ("all", "default")):
        np.testing.assert_array_equal(runs[a][0], runs[b][0])
        for key in runs[a][1]:
            np.testing.assert_array_equal(runs[a][1][key], runs[b][1][key])
    assert not np.array_equal(runs["none"][0], runs["all"][0])




def test_the_quantizers_halves_read_is_the_inverse_of_halves_of():
    """grouped_triton's `read` (which pair column each column in halves takes) and
    grouped_cudnn.halves_of (where each pair column goes) are inverse permutations: a
    GLU's halves quantized from pairs are the pairs quantized, permuted by halves_of."""
    c = 256
    read = mxfp8.read_as_halves(c)
    assert sorted(read.tolist()) == list(range(c))
    np.testing.assert_array_equal(mxfp8.halves_of(read), np.arange(c))
    # in each 64: the 32 gates (odd pair columns), then the 32 ups
    np.testing.assert_array_equal(read[:32], np.arange(1, 64, 2))
    np.testing.assert_array_equal(read[32:64], np.arange(0, 64, 2))
    rng = np.random.default_rng(14)
    x = bf16.to_bf16(rng.standard_normal((64, c)).astype(np.float32))
    a, at = mxfp8.quantized_twice(x, 64, True, halves=True)
    b, bt = mxfp8.quantized_twice(x[:, read], 64, True)
    np.testing.assert_array_equal(a.values, b.values)
    np.testing.assert_array_equal(at.values, bt.values)
