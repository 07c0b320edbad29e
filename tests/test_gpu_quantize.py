"""The HIP MXFP8 quantizer against the oracle, bit for bit: E4M3 codes and E8M0 scale
bytes (read back from the tiled layout row-major, its K padding checked), for both
copies (along the rows, and x^T along its rows), every bfloat16 value at every scale
exponent, gathered rows, rows past `filled`, padding, stacks, and the benchmark's
full-size activations."""

import numpy as np
import pytest
import torch

from oracle import bf16, mxfp8
from tests._util import announce, normal_bf16, to_gpu, to_gpu_bf16, untiled, with_outliers

pytestmark = pytest.mark.gpu

ALL = np.arange(65536, dtype=np.uint32).astype(np.uint16)
FINITE = ALL[np.isfinite(bf16.to_f32(ALL))]


def _equal(got, want, what):
    got_v, got_s = untiled(got, want.values.shape[-1])
    assert got_v.shape == want.values.shape, (what, got_v.shape, want.values.shape)
    bad = np.flatnonzero(got_v.reshape(-1) != want.values.reshape(-1))
    assert bad.size == 0, f"{what}: {bad.size} codes differ, first at {bad[:5]}: " \
        f"{got_v.reshape(-1)[bad[:5]]} vs {want.values.reshape(-1)[bad[:5]]}"
    bad = np.flatnonzero(got_s.reshape(-1) != want.scales.reshape(-1))
    assert bad.size == 0, f"{what}: {bad.size} scales differ, first at {bad[:5]}"


def _every_value_at_every_exponent() -> np.ndarray:
    """Blocks of 32 whose first entry, 448 * 2^e, sets the block's exponent to e, and
    whose other 31 are every finite bfloat16 of magnitude at most it, for e from -126
    to 119 (448 * 2^120 overflows bfloat16): (rows, 32) bfloat16 bits."""
    v = bf16.to_f32(FINITE)
    blocks = []
    for e in range(-126, 120):
        anchor = np.float32(448.0 * 2.0 ** e)
        values = FINITE[np.abs(v) <= anchor]
        pad = -values.size % 31
        values = np.concatenate([values, np.zeros(pad, np.uint16)]).reshape(-1, 31)
        head = np.full((values.shape[0], 1), bf16.to_bf16(np.array([anchor]))[0], np.uint16)
        blocks.append(np.concatenate([head, values], 1))
    return np.concatenate(blocks)


def test_every_bf16_value_at_every_exponent_rows_and_columns(lib):
    x = _every_value_at_every_exponent()
    x = x[: x.shape[0] // 32 * 32]
    announce("quantize every value x exponent", x.shape)
    got_rows, got_cols = _quantize(to_gpu_bf16(x))
    want_rows, want_cols = mxfp8.mx_twice(bf16.to_f32(x))
    _equal(got_rows, want_rows, "rows")
    _equal(got_cols, want_cols, "columns")


def _quantize(x, **kw):
    from bux_amd import grouped_mxfp8
    out = grouped_mxfp8.quantized_twice(x, **kw)
    torch.cuda.synchronize()
    return out


def test_every_bf16_magnitude_as_a_blocks_largest(lib):
    """Each block's scale from its largest magnitude, for every finite bfloat16 of
    either sign as that largest (its other 31 values 0 or smaller), along the rows and
    down the columns: the kernels derive the exponent from the maximum's bits, which
    must agree with the reference's float32 division for every pattern."""
    mags = FINITE[(FINITE & 0x7FFF) != 0]
    mags = mags[: mags.size // 32 * 32]
    rng = np.random.default_rng(16)
    x = np.zeros((mags.size, 32), np.uint16)
    x[:, 0] = mags
    small = bf16.to_bf16((bf16.to_f32(mags) * np.float32(0.5)).astype(np.float32))
    x[:, 1 + rng.integers(0, 31, mags.size)] = small  # a smaller value beside it
    announce("quantize every magnitude as the largest", x.shape)
    got_rows, got_cols = _quantize(to_gpu_bf16(x))
    want_rows, want_cols = mxfp8.mx_twice(bf16.to_f32(x))
    _equal(got_rows, want_rows, "rows")
    _equal(got_cols, want_cols, "columns")


def test_every_bf16_pattern_shuffled(lib):
    rng = np.random.default_rng(11)
    x = np.where(np.isfinite(bf16.to_f32(ALL)), ALL, 0).astype(np.uint16)
    x = rng.permutation(x).reshape(2048, 32)
    announce("quantize shuffled patterns", x.shape)
    got_rows, got_cols = _quantize(to_gpu_bf16(x))
    want_rows, want_cols = mxfp8.mx_twice(bf16.to_f32(x))
    _equal(got_rows, want_rows, "rows")
    _equal(got_cols, want_cols, "columns")


@pytest.mark.parametrize("cols", [32, 96, 2048])
def test_gathered_rows_past_filled_and_padding(lib, cols):
    """Picked rows ``tokens[order // k]`` (a -1 reads 0, and so does an entry whose
    token lies past the tokens: no read leaves them), rows from `filled` on and the
    padding up to whole tiles of 128 as 0 (grouped_blockscaled.py:122-128, 314)."""
    rng = np.random.default_rng(12)
    tokens, k, m = 300, 4, 1000
    z = with_outliers(rng, normal_bf16(rng, (tokens, cols)), 0.01)
    order = rng.permutation(tokens * k)[:m].astype(np.int32)
    order[rng.choice(m, 7, replace=False)] = -1
    past = rng.choice(m, 5, replace=False)
    order[past] = tokens * k + np.array([0, 1, k, 1000, 2**31 - 1 - tokens * k])[:5]
    filled = 937
    height = 1024
    announce("quantize gathered", tokens, cols, m, filled, height)
    got_rows, got_cols = _quantize(
        to_gpu_bf16(z), filled=to_gpu(np.array([filled], np.int32)), columns=True,
        index=to_gpu(order), index_div=k, height=height)
    index = np.where((order >= 0) & (order // k < tokens), order // k, -1)
    want_rows, want_cols = mxfp8.quantized_twice(z, filled, True, index=index, height=height)
    _equal(got_rows, want_rows, "rows")
    _equal(got_cols, want_cols, "columns")


def test_a_stack_of_matrices_one_at_a_time(lib):
    """Each expert's W quantizes on its own (grouped_blockscaled.py:315-317)."""
    rng = np.random.default_rng(13)
    w = normal_bf16(rng, (5, 96, 160), 0.02)
    announce("quantize stack", w.shape)
    got_rows, got_cols = _quantize(to_gpu_bf16(w))
    want_rows, want_cols = mxfp8.quantized_twice(w, 96, True)
    _equal(got_rows, want_rows, "rows")
    _equal(got_cols, want_cols, "columns")


@pytest.mark.parametrize("shape", [(5, 96, 160), (2, 2048, 1536), (3, 768, 2048), (1, 32, 32)])
def test_weights_with_a_scale_per_32x32_tile(lib, shape):
    """The mxfp8_2d recipe's W (blockscaled.mx_tiles_twice): each expert's matrix with a
    scale per 32 x 32 tile, both copies the tile's; c3's W_up and W_down shapes
    included (two experts of W_up, three of W_down), with outliers that set a tile's
    scale apart from its row blocks'."""
    rng = np.random.default_rng(15)
    w = with_outliers(rng, normal_bf16(rng, shape, 0.02), 1e-3, 1e3)
    announce("quantize tiles", shape)
    got_rows, got_cols = _quantize(to_gpu_bf16(w), tiles=True)
    want_rows, want_cols = mxfp8.quantized_twice(w, shape[1], True, tiles=True)
    _equal(got_rows, want_rows, "rows")
    _equal(got_cols, want_cols, "columns")
    v_rows, _ = untiled(got_rows, shape[2])
    v_cols, _ = untiled(got_cols, shape[1])
    assert (v_cols == np.swapaxes(v_rows, -1, -2)).all()  # the same codes, transposed


def test_only_the_rows_copy_or_only_the_columns_copy(lib):
    rng = np.random.default_rng(14)
    x = normal_bf16(rng, (64, 128))
    from bux_amd import grouped_mxfp8
    announce("quantize rows only / columns only")
    r, none = grouped_mxfp8.quantized_twice(to_gpu_bf16(x), columns=False)
    none2, c = grouped_mxfp8.quantized_twice(to_gpu_bf16(x), rows=False)
    torch.cuda.synchronize()
    assert none is None and none2 is None
    want_rows, want_cols = mxfp8.mx_twice(bf16.to_f32(x))
    _equal(r, want_rows, "rows")
    _equal(c, want_cols, "columns")


def test_config2_activations_full_size(lib):
    """Config 2's x: 16384 tokens of 2048, 0.1% outliers x100, read by index into
    131072 rows (top-8 picks). The oracle checks a seeded sample of 4096 rows of the
    row copy and 64 blocks of 32 rows of the column copy; the rest is pinned by
    size-independent properties: a second run is bitwise identical, and reading the
    rows by index gives the same bytes as quantizing the gathered rows."""
    rng = np.random.default_rng(1)
    t, d, k = 16384, 2048, 8
    z = with_outliers(rng, normal_bf16(rng, (t, d)))
    order = rng.permutation(t * k).astype(np.int32)
    m = t * k
    announce("quantize config2 full size", t, d, k)
    zg, og = to_gpu_bf16(z), to_gpu(order)
    rows1, cols1 = _quantize(zg, index=og, index_div=k, height=m)
    rows2, cols2 = _quantize(zg, index=og, index_div=k, height=m)
    assert torch.equal(rows1.values, rows2.values) and torch.equal(cols1.values, cols2.values)
    assert torch.equal(rows1.scales, rows2.scales) and torch.equal(cols1.scales, cols2.scales)
    from bux_amd import moe
    gathered = moe.token_rows(zg, og, k)
    rows3, cols3 = _quantize(gathered)
    assert torch.equal(rows1.values, rows3.values) and torch.equal(cols1.scales, cols3.scales)
    assert torch.equal(cols1.values, cols3.values)
    from bux_amd import grouped_mxfp8
    sample = rng.choice(m, 4096, replace=False)
    want = mxfp8.mx_quantize(z[order[sample] // k])
    at = torch.from_numpy(sample).cuda()
    rows_v, rows_s = grouped_mxfp8.canonical(rows1, d)
    np.testing.assert_array_equal(rows_v[at].cpu().numpy(), want.values)
    np.testing.assert_array_equal(rows_s[at].cpu().numpy(), want.scales)
    cols_v, cols_s = grouped_mxfp8.canonical(cols1, m)
    for b in rng.choice(m // 32, 64, replace=False):
        block = z[order[32 * b:32 * b + 32] // k]  # 32 rows, all columns
        want = mxfp8.mx_quantize(np.ascontiguousarray(bf16.to_f32(block).T))
        np.testing.assert_array_equal(cols_v[:, 32 * b:32 * b + 32].cpu().numpy(), want.values)
        np.testing.assert_array_equal(cols_s[:, b].cpu().numpy(), want.scales[:, 0])


@pytest.mark.parametrize("index", [False, True])
def test_halves_read_a_glus_pairs_as_its_halves(lib, index):
    """BUX_MX_HALVES (the reference's `halves`, grouped_triton.py:49): the columns of
    (up, gate) pairs quantized as a GLU's halves, bit for bit the oracle's, for a stack
    of kernels and for rows read by index."""
    from bux_amd import grouped_mxfp8 as gm
    from oracle import mxfp8 as omx
    rng = np.random.default_rng(90)
    announce("quantize halves", index)
    if index:
        x = normal_bf16(rng, (300, 384))
        idx = rng.integers(0, 300 * 4, 1000).astype(np.int32)
        idx[::17] = -1
        got_k, got_m = gm.quantized_twice(to_gpu_bf16(x), None, True, to_gpu(idx), 4, 1024,
                                          halves=True)
        want_k, want_m = omx.quantized_twice(x, 1000, True, index=np.where(idx >= 0, idx // 4, -1),
                                             height=1024, halves=True)
        pairs = [(got_k, want_k, 384), (got_m, want_m, 1024)]
    else:
        x = normal_bf16(rng, (3, 256, 512), 0.05)
        got_k, got_m = gm.quantized_twice(to_gpu_bf16(x), halves=True)
        want_k, want_m = omx.quantized_twice(x, 256, True, halves=True)
        pairs = [(got_k, want_k, 512), (got_m, want_m, 256)]
    torch.cuda.synchronize()
    for got, want, cols in pairs:
        v, sc = untiled(got, cols)
        np.testing.assert_array_equal(v, want.values)
        np.testing.assert_array_equal(sc, want.scales)
