"""The HIP grouped GEMMs against the oracle (the reference's XLA path off Blackwell:
dequantize, then GEMMs per group), here summed in float64.

Bars: float32 outputs within MAX_OF_MAX of the largest |value| and NORM in norm (set
from the block-scaled MFMA's measured summation error, below; the reference's
kernel-vs-XLA bar, scripts/gpu_smoke/grouped_mxfp8.py:45, is 1e-5 of the max between
two float32 summations on Blackwell); bfloat16 outputs within ||y - y_ref|| / ||y_ref||
<= 1e-3 (the north star's bar); empty groups and rows past the groups exactly 0; a
wgrad ignores whatever lies past the groups (tests/test_grouped.py:89-95)."""

import numpy as np
import pytest
import torch

from oracle import bf16, moe as omoe, mxfp8
from tests._util import announce, bf16_bits, normal_bf16, rel_err, to_gpu, to_gpu_bf16, to_gpu_tiled

pytestmark = pytest.mark.gpu


def _codes(rng, shape, scale=1.0):
    """Random MXFP8 blocks of bfloat16 N(0, scale^2) draws, with outliers."""
    x = bf16.to_f32(normal_bf16(rng, shape, scale))
    x.reshape(-1)[rng.choice(x.size, max(1, x.size // 500), replace=False)] *= 100
    if len(shape) == 3:
        parts = [mxfp8.mx_quantize(a) for a in x]
        return mxfp8.Blocks(np.stack([p.values for p in parts]), np.stack([p.scales for p in parts]))
    return mxfp8.mx_quantize(x)


def _gpu(blocks):
    return to_gpu_tiled(blocks)


# The block-scaled MFMA does not sum a block's products in IEEE float32 (its error bound,
# SUM_ERROR, is measured by test_the_block_scaled_mfma_sum_is_within_its_error_bound):
# against float64 sums of the same products its float32 outputs deviate by 1.5e-5 in
# norm on Gaussian data, and by up to 8.5e-5 in norm (1.3e-4 of the largest |value|)
# where x100 outliers share a block with ordinary values; an IEEE float32 sum would be
# near 1e-7. The bars hold those with margin, against a float64 reference: a wrong
# block, scale, row or group gives errors of order 1.
MAX_OF_MAX = 5e-4  # |y - y_ref| <= this x max |y_ref|
NORM = 2e-4  # ||y - y_ref|| / ||y_ref||


def _close_f32(got, want, what=""):
    got = got.astype(np.float64)
    want = np.asarray(want, np.float64)
    top = max(float(np.abs(want).max()), 1e-30)
    err = np.abs(got - want)
    print(f"[err] {what} max/max {err.max() / top:.3e} norm {rel_err(got, want):.3e}", flush=True)
    assert err.max() <= MAX_OF_MAX * top, (err.max() / top, np.unravel_index(err.argmax(), err.shape))
    assert rel_err(got, want) <= NORM


def _rows64(a, b, sizes, height):
    """The oracle's rows (dequantize, GEMM per group), summed in float64."""
    x, w = mxfp8.dequantized(a).astype(np.float64), mxfp8.dequantized(b).astype(np.float64)
    y = np.zeros((height, w.shape[1]))
    start = 0
    for g, size in enumerate(sizes.tolist()):
        y[start:start + size] = x[start:start + size] @ w[g].T
        start += size
    return y


def _contract64(a, b, sizes):
    """The oracle's contract, summed in float64."""
    x, y = mxfp8.dequantized(a).astype(np.float64), mxfp8.dequantized(b).astype(np.float64)
    dw = np.zeros((len(sizes), x.shape[0], y.shape[0]))
    start = 0
    for g, size in enumerate(sizes.tolist()):
        dw[g] = x[:, start:start + size] @ y[:, start:start + size].T
        start += size
    return dw


ROW_CASES = [
    # sizes, k, n, height (None: m)
    ([0, 130, 1, 3, 256, 0, 300, 100], 256, 384, None),
    ([70, 0, 100, 3, 77], 2880, 2880, 384),  # k and n not whole tiles of 128; padding rows
    ([128, 128, 256], 128, 128, None),  # groups on tile edges
    ([5], 64, 96, 64),
    ([0, 0, 0], 128, 128, 128),  # no rows at all: every row 0
    ([700, 0, 1, 300, 513, 2000], 512, 640, 3712),  # tiles of 256 from each group's start
    ([0, 300, 1, 0, 250, 49], 7168, 256, None),  # config 5's d as K: a 112-step K loop
    ([100, 0, 37], 256, 7168, 160),  # config 5's d as N: 28 column tiles
    # n a whole number of 384s: the last column tile of 256 half full
    ([0, 130, 1, 3, 256, 0, 300, 100], 256, 768, None),
    ([700, 0, 1, 300, 513, 2000], 512, 1152, 3712),
    ([0, 300, 1, 0, 250, 49], 2048, 1536, None),  # config 3's up fprop shape, ragged
    ([70, 0, 100, 3, 77], 128, 384, 192),  # rows of the groups past the output's
]


@pytest.mark.parametrize("sizes,k,n,height", ROW_CASES)
def test_rows(lib, sizes, k, n, height):
    from bux_amd import grouped_mxfp8
    rng = np.random.default_rng(30)
    sizes = np.array(sizes, np.int32)
    m = max(int(sizes.sum()), 32)
    m = -(-m // 32) * 32
    a = _codes(rng, (m, k))
    b = _codes(rng, (len(sizes), n, k), 0.02)
    h = m if height is None else height
    announce("rows", sizes.tolist(), m, k, n, h)
    ga, gb, gs = _gpu(a), _gpu(b), to_gpu(sizes)
    y32 = grouped_mxfp8.rows(ga, gb, gs, torch.float32, height=h)
    y16 = grouped_mxfp8.rows(ga, gb, gs, torch.bfloat16, height=h)
    torch.cuda.synchronize()
    want = _rows64(a, b, sizes, max(h, m))[:h]
    got = y32.cpu().numpy()
    _close_f32(got, want, f"rows {sizes.tolist()} k={k}")
    filled = int(sizes.sum())
    assert (got[filled:] == 0).all()
    # bfloat16 out against the reference's own bfloat16 rounding of its sums
    got16 = bf16.to_f32(bf16_bits(y16)).astype(np.float64)
    assert rel_err(got16, bf16.round_f32(want.astype(np.float32))) <= 1e-3 or np.abs(want).max() == 0
    assert (got16[filled:] == 0).all()


@pytest.mark.parametrize("sizes", [[100, -7, 150, 400, 90], [100, 2**31 - 1, 5], [-(2**31), 64]])
def test_rows_take_a_negative_size_as_none_and_stop_at_the_rows(lib, sizes):
    """Sizes are device data the host cannot check: a negative one counts as 0, and sizes
    summing past the rows there are (512) give the last groups fewer rows, so that no
    tile starts before row 0 or stores past y. The result is the oracle's on the sizes
    so taken ([100, 0, 150, 262, 0], [100, 412, 0], [0, 64])."""
    from bux_amd import grouped_mxfp8
    rng = np.random.default_rng(36)
    m = h = 512
    k, n = 256, 384
    sizes = np.array(sizes, np.int64)
    taken, start = [], 0
    for size in np.maximum(sizes, 0).tolist():
        taken.append(min(size, m - start))
        start += taken[-1]
    taken = np.array(taken, np.int32)
    a = _codes(rng, (m, k))
    b = _codes(rng, (len(sizes), n, k), 0.02)
    announce("rows with sizes outside the rows", sizes.tolist())
    y32 = grouped_mxfp8.rows(_gpu(a), _gpu(b), to_gpu(sizes.astype(np.int32)), torch.float32,
                             height=h)
    torch.cuda.synchronize()
    got = y32.cpu().numpy()
    want = _rows64(a, b, taken, h)
    _close_f32(got, want, f"rows {sizes.tolist()} taken as {taken.tolist()}")
    assert (got[int(taken.sum()):] == 0).all()
    # the contract takes the same sizes the same way, its K (m) as the rows: the wgrad of
    # a group agrees with its forward
    at, bt = _codes(rng, (k, m)), _codes(rng, (128, m))
    announce("contract with sizes outside the rows", sizes.tolist())
    dw = grouped_mxfp8.contract(_gpu(at), _gpu(bt), to_gpu(sizes.astype(np.int32)), torch.float32)
    torch.cuda.synchronize()
    _close_f32(dw.cpu().numpy(), _contract64(at, bt, taken),
               f"contract {sizes.tolist()} taken as {taken.tolist()}")


CONTRACT_CASES = [
    ([70, 0, 100, 3, 77], 256, 192, 256),
    ([0, 130, 1, 3, 256, 0, 300, 100], 2880, 160, 800),  # d not whole tiles, blocks across groups
    ([128, 0, 384], 128, 256, 512),  # groups on tile edges
    ([0, 0], 64, 64, 64),  # nothing: dW 0
    ([700, 0, 1, 300, 513, 2000], 640, 384, 3584),  # 256-wide tiles, a partial one
    ([300, 0, 212, 0], 7168, 256, 512),  # config 5's d as the wgrad's rows
    # d or f a whole number of 384s: the last row or column tile of 256 half full
    ([70, 0, 100, 3, 77], 256, 768, 256),
    ([0, 130, 1, 3, 256, 0, 300, 100], 2048, 1536, 896),  # config 3's up wgrad shape
    ([70, 0, 100, 3, 77], 768, 256, 256),
    ([700, 0, 1, 300, 513, 2000], 768, 512, 3584),
    ([128, 0, 384], 384, 2048, 512),  # config 3's down wgrad shape
]


@pytest.mark.parametrize("sizes,d,f,m", CONTRACT_CASES)
def test_contract(lib, sizes, d, f, m):
    from bux_amd import grouped_mxfp8
    rng = np.random.default_rng(31)
    sizes = np.array(sizes, np.int32)
    a = _codes(rng, (d, m))
    b = _codes(rng, (f, m), 0.01)
    filled = int(sizes.sum())
    # garbage past the groups (tests/test_grouped.py:89-95): it must add nothing
    junk = a.values.copy()
    junk[:, filled:] = 0x7E
    a = mxfp8.Blocks(junk, a.scales)
    announce("contract", sizes.tolist(), d, f, m)
    ga, gb, gs = _gpu(a), _gpu(b), to_gpu(sizes)
    dw32 = grouped_mxfp8.contract(ga, gb, gs, torch.float32)
    dw16 = grouped_mxfp8.contract(ga, gb, gs, torch.bfloat16)
    torch.cuda.synchronize()
    want = _contract64(a, b, sizes)
    got = dw32.cpu().numpy()
    for g in range(len(sizes)):
        if sizes[g] == 0:
            assert (got[g] == 0).all()
        else:
            _close_f32(got[g], want[g], f"contract group {g} of {sizes.tolist()}")
    got16 = bf16.to_f32(bf16_bits(dw16))
    assert rel_err(got16, bf16.round_f32(want.astype(np.float32))) <= 1e-3 or np.abs(want).max() == 0


def test_rows_at_config3_up_shape(lib):
    """Config 3's gate/up fprop shape, 131072 rows of 2048 by 128 experts' (1536, 2048),
    near-uniform loads: a seeded sample of 512 rows against the oracle; the whole
    output against the same GEMM in float32 out (bfloat16 is its rounding)."""
    from bux_amd import grouped_mxfp8
    rng = np.random.default_rng(32)
    e, m, k, n = 128, 131072, 2048, 1536
    sizes = np.bincount(rng.integers(0, e, m), minlength=e).astype(np.int32)
    announce("rows config3 up")
    x = torch.randn(m, k, device="cuda", dtype=torch.bfloat16)
    w = (torch.randn(e, n, k, device="cuda") * 0.02).to(torch.bfloat16)
    xa, _ = grouped_mxfp8.quantized_twice(x, columns=False)
    wb, _ = grouped_mxfp8.quantized_twice(w, columns=False)
    gs = to_gpu(sizes)
    y16 = grouped_mxfp8.rows(xa, wb, gs)
    y32 = grouped_mxfp8.rows(xa, wb, gs, torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(y16, y32.to(torch.bfloat16))
    sample = np.sort(rng.choice(m, 512, replace=False))
    starts = np.cumsum(sizes) - sizes
    xa_v, xa_s = grouped_mxfp8.canonical(xa, k)
    at = torch.from_numpy(sample).cuda()
    a = mxfp8.Blocks(xa_v[at].cpu().numpy(), xa_s[at].cpu().numpy())
    wb_v, wb_s = grouped_mxfp8.canonical(wb, k)
    deq_a = mxfp8.dequantized(a).astype(np.float64)
    groups = np.searchsorted(starts + sizes, sample, side="right")
    got = y32[torch.from_numpy(sample).cuda()].cpu().numpy()
    for g in np.unique(groups):
        rows = groups == g
        wg = mxfp8.Blocks(wb_v[int(g)].cpu().numpy(), wb_s[int(g)].cpu().numpy())
        want = deq_a[rows] @ mxfp8.dequantized(wg).astype(np.float64).T
        _close_f32(got[rows], want, f"config3 up rows of group {g}")


def test_contract_at_config3_down_shape(lib):
    """Config 3's down wgrad shape: h^T (768, 131072) and dy^T (2048, 131072), 128
    experts; a seeded sample of 4 experts' dW against the oracle in float64."""
    from bux_amd import grouped_mxfp8
    rng = np.random.default_rng(33)
    e, m, d, f = 128, 131072, 768, 2048
    sizes = np.bincount(rng.integers(0, e, m), minlength=e).astype(np.int32)
    announce("contract config3 down")
    h = torch.randn(m, d, device="cuda", dtype=torch.bfloat16)
    dy = (torch.randn(m, f, device="cuda") * 0.01).to(torch.bfloat16)
    _, hm = grouped_mxfp8.quantized_twice(h, rows=False)
    _, dym = grouped_mxfp8.quantized_twice(dy, rows=False)
    gs = to_gpu(sizes)
    dw = grouped_mxfp8.contract(hm, dym, gs, torch.float32)
    torch.cuda.synchronize()
    starts = np.cumsum(sizes) - sizes
    hm_v, hm_s = grouped_mxfp8.canonical(hm, m)
    dym_v, dym_s = grouped_mxfp8.canonical(dym, m)
    for g in rng.choice(e, 4, replace=False):
        lo, hi = int(starts[g]), int(starts[g] + sizes[g])
        b0, b1 = lo // 32, -(-hi // 32)
        a = mxfp8.Blocks(hm_v[:, 32 * b0:32 * b1].cpu().numpy(), hm_s[:, b0:b1].cpu().numpy())
        b = mxfp8.Blocks(dym_v[:, 32 * b0:32 * b1].cpu().numpy(), dym_s[:, b0:b1].cpu().numpy())
        da = mxfp8.dequantized(a).astype(np.float64)[:, lo - 32 * b0:hi - 32 * b0]
        db = mxfp8.dequantized(b).astype(np.float64)[:, lo - 32 * b0:hi - 32 * b0]
        want = da @ db.T
        got = dw[int(g)].cpu().numpy()
        _close_f32(got, want, f"config3 down dW group {g}")


# bfloat16 rows GEMM cases: (sizes, m, k, n). Rows past the groups hold NaN in x (they
# must not reach any output: those rows are 0). k = 200 is not a whole number of the
# kernel's K steps of 32 (its last step masked); n = 264 leaves a partial column tile.
BF16_ROWS = {
    "five groups": ([1000, 0, 1500, 3, 1589], 4200, 256, 1024),
    "k tail, partial tiles": ([300, 77, 0, 500], 900, 200, 264),
    "one group, whole tiles": ([512], 512, 64, 256),
    "64 small groups": (None, 1500, 128, 128),
    "k under one step, n of 8": ([5, 0, 7], 20, 8, 8),
    "one row": ([1], 1, 64, 64),
    "all groups empty": ([0, 0, 0], 300, 64, 64),
    # rows off 16-byte chunks: the any-shape kernels (element loads)
    "n and k off multiples of 8": ([300, 0, 41, 500], 900, 45, 37),
    "k off 8, n whole tiles": ([700, 3, 297], 1000, 100, 264),
    "k and n of 1": ([5, 0, 3], 10, 1, 1),
    "n off 8, 64 small groups": (None, 1500, 64, 70),
}


def _bf16_sizes(rng, sizes, m):
    if sizes is None:  # 64 groups of 0 .. 40 rows, some empty
        sizes = rng.integers(0, 41, 64)
        sizes[rng.choice(64, 8, replace=False)] = 0
    sizes = np.asarray(sizes, np.int32)
    assert sizes.sum() <= m
    return sizes


@pytest.mark.parametrize("transposed", [False, True])
@pytest.mark.parametrize("case", list(BF16_ROWS))
def test_bf16_rows(lib, case, transposed):
    from bux_amd import grouped
    rng = np.random.default_rng(34)
    sizes, m, k, n = BF16_ROWS[case]
    sizes = _bf16_sizes(rng, sizes, m)
    filled = int(sizes.sum())
    x = normal_bf16(rng, (m, k))
    x[filled:] = 0x7FC0  # NaN
    w = normal_bf16(rng, (len(sizes), k, n), 0.02)
    announce("bf16 rows", case, transposed)
    wt = np.ascontiguousarray(np.swapaxes(w, 1, 2)) if transposed else w
    y = grouped.dot(to_gpu_bf16(x), to_gpu_bf16(wt), to_gpu(sizes), transposed=transposed)
    torch.cuda.synchronize()
    want = omoe.ragged_dot_bf16(x[:filled], w, sizes, out="bf16")
    got = bf16.to_f32(bf16_bits(y))
    assert (got[filled:] == 0).all()
    err = rel_err(got[:filled], bf16.to_f32(want)) if filled else 0.0
    print(f"[err] bf16 rows {case} {err:.3e}", flush=True)
    assert err <= 1e-3  # both float32 sums rounded to bfloat16: the north star's bar


# bfloat16 wgrad cases: (sizes, m, k, n). Group boundaries off the kernel's K step of 32
# rows; the rows past the groups hold NaN in x and dy (a wgrad ignores them); k = 136
# and n = 264 leave partial tiles.
BF16_CONTRACT = {
    "five groups": ([70, 0, 100, 3, 77], 256, 256, 512),
    "unaligned groups, NaN past them": ([33, 0, 95, 1, 200], 400, 136, 264),
    "64 small groups": (None, 1500, 128, 256),
    "k and n of 8, rows under one step": ([3, 0, 9], 16, 8, 8),
    "all groups empty": ([0, 0], 100, 64, 64),
    # rows off 16-byte chunks: the any-shape kernel
    "k and n off multiples of 8": ([33, 0, 95, 1, 200], 400, 45, 37),
    "k of 300, n of 3": ([70, 0, 100, 3, 77], 256, 300, 3),
    "all groups empty, n off 8": ([0, 0], 100, 5, 9),
}


@pytest.mark.parametrize("case", list(BF16_CONTRACT))
def test_bf16_weight_grad(lib, case):
    from bux_amd import grouped
    rng = np.random.default_rng(35)
    sizes, m, k, n = BF16_CONTRACT[case]
    sizes = _bf16_sizes(rng, sizes, m)
    filled = int(sizes.sum())
    x = normal_bf16(rng, (m, k))
    dy = normal_bf16(rng, (m, n), 0.01)
    x[filled:] = 0x7FC0
    dy[filled:] = 0x7FC0
    announce("bf16 weight_grad", case)
    dw = grouped.weight_grad(to_gpu_bf16(x), to_gpu_bf16(dy), to_gpu(sizes))
    torch.cuda.synchronize()
    want = omoe.weight_grad_bf16(x[:filled], dy[:filled], sizes, out="bf16")
    got = bf16.to_f32(bf16_bits(dw))
    assert (got[sizes == 0] == 0).all()
    err = rel_err(got, bf16.to_f32(want)) if filled else float(np.abs(got).max())
    print(f"[err] bf16 weight_grad {case} {err:.3e}", flush=True)
    assert err <= 1e-3


def test_a_tile_list_made_once_serves_every_gemm(lib):
    """rows and contract on one `tiles_of` list give the bytes they give on their own
    prologue (the reference's rows/contract taking `tiles` and `starts`)."""
    from bux_amd import grouped_mxfp8 as gm
    rng = np.random.default_rng(31)
    sizes = np.array([0, 130, 1, 3, 256, 0, 300, 100], np.int32)
    m, height, k, n = 900, 896, 256, 384
    a = _gpu(_codes(rng, (m, k)))
    b = _gpu(_codes(rng, (len(sizes), n, k), 0.05))
    gs = to_gpu(sizes)
    announce("gemm tile list", m, height, k, n)
    tiles = gm.tiles_of(gs, a.height, height)
    for out in (torch.bfloat16, torch.float32):
        y0 = gm.rows(a, b, gs, out, height=height)
        y1 = gm.rows(a, b, gs, out, height=height, tiles=tiles)
        torch.cuda.synchronize()
        assert torch.equal(y0.view(torch.uint8), y1.view(torch.uint8))
    xt = _gpu(_codes(rng, (192, 1024)))
    dt = _gpu(_codes(rng, (128, 1024)))
    dw0 = gm.contract(xt, dt, gs)
    dw1 = gm.contract(xt, dt, gs, tiles=tiles)
    torch.cuda.synchronize()
    assert torch.equal(dw0.view(torch.uint8), dw1.view(torch.uint8))


def _c3_like_sizes():
    rng = np.random.default_rng(33)
    sizes = rng.integers(990, 1060, 128)
    return sizes.tolist(), int(sizes.sum()), int((sizes.sum() + 127) // 128 * 128)


TILE_LIST_CASES = {
    "reference sizes": ([0, 130, 1, 3, 256, 0, 300, 100], 1024, 1024),
    "rows past the groups": ([0, 130, 1, 3, 256, 0, 300, 100], 900, 896),
    "every group empty": ([0, 0, 0], 256, 256),
    "one row": ([0, 1], 1, 32),
    "config 3 like": _c3_like_sizes(),
}


@pytest.mark.parametrize("case", list(TILE_LIST_CASES))
def test_the_device_tile_list_covers_each_groups_rows_once(lib, case):
    """The invariant of the reference's tiles_of (tests/test_grouped_mxfp8.py:31-41), on
    the list the device prologue builds (tiles of 256 rows from each group's first row):
    every row of group g, [starts[g], starts[g + 1]), is held by exactly one tile of g, a
    tile (g, lo, hi) holding rows [max(lo, starts[g]), hi) inside [lo, lo + 256); the
    rows from the groups' end to `height` are held once by tiles of group `groups`; a
    group of s rows has ceil(s / 256) tiles, in group order; the list holds starts[groups
    + 1] tiles and (0, 0, 0) past them; its header names the dimensions."""
    from bux_amd import _lib, grouped_mxfp8 as gm
    sizes, m, height = TILE_LIST_CASES[case]
    groups = len(sizes)
    announce("device tile list", case, groups, m, height)
    tl = gm.tiles_of(to_gpu(np.array(sizes, np.int32)), m, height)
    torch.cuda.synchronize()
    buf = tl.buffer.cpu().numpy()
    header = buf[:64].view(np.int32)
    assert list(header[:5]) == [_lib.LIST_MAGIC, groups, m, height, 0]
    starts = buf[64:64 + 4 * (groups + 2)].view(np.int32)
    filled = int(np.sum(sizes))
    assert starts[:groups + 1].tolist() == [0] + np.cumsum(sizes).tolist()
    slots = -(-max(m, height) // 256) + groups + 1
    first = (64 + 4 * (groups + 2) + 255) // 256 * 256
    tiles = buf[first:first + 12 * slots].view(np.int32).reshape(slots, 3)
    count = int(starts[groups + 1])
    lo_of = list(starts[:groups]) + [filled]  # where each group's rows begin
    rows_of = list(sizes) + [max(height - filled, 0)]
    assert count == sum(-(-s // 256) for s in rows_of)
    assert (tiles[count:] == 0).all()
    covered = np.full(max(m, height, filled), -1)
    last = -1
    for g, lo, hi in tiles[:count]:
        assert last <= g <= groups
        last = g
        held = max(lo, lo_of[g])
        assert lo_of[g] <= lo and held < hi <= lo + 256 and hi <= lo_of[g] + rows_of[g]
        assert (covered[held:hi] == -1).all()
        covered[held:hi] = g
    for g in range(groups + 1):
        assert (covered[lo_of[g]:lo_of[g] + rows_of[g]] == g).all()
    assert (covered >= 0).sum() == filled + max(height - filled, 0)


def test_a_tile_list_made_for_other_dimensions_is_refused_on_the_device(lib):
    """A list whose header names other dimensions than the call's (but long enough for
    them, so the host lets it by) is refused by the GEMM kernel as it starts: its status
    word becomes BUX_LIST_REFUSED and nothing is written (the output keeps what it
    held); a matching list's status stays 0."""
    from bux_amd import _lib, grouped_mxfp8 as gm
    from bux_amd.kernels import ptr, stream
    rng = np.random.default_rng(32)
    sizes = np.array([0, 130, 1, 3, 256, 0, 300, 100], np.int32)
    m, height, k, n = 900, 896, 256, 384
    a = _gpu(_codes(rng, (m, k)))
    b = _gpu(_codes(rng, (len(sizes), n, k), 0.05))
    gs = to_gpu(sizes)
    announce("gemm tile list refused", m, height, k, n)
    good = gm.tiles_of(gs, a.height, height)
    y = gm.rows(a, b, gs, height=height, tiles=good)
    torch.cuda.synchronize()
    header = good.buffer[:20].view(torch.int32).cpu().numpy()
    assert list(header) == [_lib.LIST_MAGIC, len(sizes), a.height, height, 0]
    # made for 896 output rows, called for 768: the list is longer than 768 rows need
    other = gm.tiles_of(gs, a.height, height)
    kept = torch.full((768, n), 7.0, dtype=torch.bfloat16, device="cuda")
    _lib.check(lib.bux_mx_grouped_rows_listed(
        ptr(a.values), ptr(a.scales), ptr(b.values), ptr(b.scales), ptr(other.buffer),
        other.buffer.numel(), len(sizes), a.height, n, k, 768, _lib.BF16, ptr(kept), stream()))
    torch.cuda.synchronize()
    assert int(other.buffer[16:20].view(torch.int32).item()) == _lib.LIST_REFUSED
    assert (kept.float() == 7.0).all()
    # the contract, called for 4 groups on an 8-group list
    third = gm.tiles_of(gs, a.height, height)
    xt = _gpu(_codes(rng, (192, 1024)))
    dt = _gpu(_codes(rng, (128, 1024)))
    dw = torch.full((4, 192, 128), 7.0, dtype=torch.bfloat16, device="cuda")
    _lib.check(lib.bux_mx_grouped_contract_listed(
        ptr(xt.values), ptr(xt.scales), ptr(dt.values), ptr(dt.scales), ptr(third.buffer),
        third.buffer.numel(), 4, 192, 128, 1024, _lib.BF16, ptr(dw), stream()))
    torch.cuda.synchronize()
    assert int(third.buffer[16:20].view(torch.int32).item()) == _lib.LIST_REFUSED
    assert (dw.float() == 7.0).all()
    # the good list still serves, its status 0
    y2 = gm.rows(a, b, gs, height=height, tiles=good)
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int16), y2.view(torch.int16))
    assert int(good.buffer[16:20].view(torch.int32).item()) == 0


def _crafted(rng, rows, k, kind):
    """MXFP8 blocks of N(0, 1) bfloat16 draws; with "outliers", every block of 32 holds
    one value x100 at a random place (the large product beside 31 ordinary ones)."""
    x = bf16.to_f32(normal_bf16(rng, (rows, k)))
    if kind == "outliers":
        blocks = x.reshape(rows, k // 32, 32)
        at = rng.integers(0, 32, (rows, k // 32))
        np.put_along_axis(blocks, at[..., None], np.take_along_axis(blocks, at[..., None], -1) * 100, -1)
    return mxfp8.mx_quantize(x)


# The block-scaled MFMA's float32 output against the exact sum of the same products:
# |y - y_exact| <= SUM_ERROR x sum_i |a_i b_i|, elementwise, measured by the test below
# on the MI355X: at worst 2^-15.5 of that sum on Gaussian blocks (K = 128; less as K
# grows) and 2^-11.4 where every block of 32 holds a x100 value. An IEEE float32 sum of K
# products keeps within K 2^-24 of it, near sqrt(K) 2^-24 in practice; the MFMA keeps
# fewer low bits of the products it adds beside a large one. The bounds hold those
# measurements with a margin of 2.6x-2.8x. MAX_OF_MAX and NORM follow from them: on
# these inputs sum_i |a_i b_i| is 1.3x (outliers) to 13x (Gaussian, K = 7168) max |y|,
# and the measured elementwise error stays under 1e-4 of max |y|.
SUM_ERROR = {"gaussian": 2.0 ** -14, "outliers": 2.0 ** -10}


@pytest.mark.parametrize("kind", ["gaussian", "outliers"])
@pytest.mark.parametrize("k", [128, 2048, 7168])
def test_the_block_scaled_mfma_sum_is_within_its_error_bound(lib, kind, k):
    """The bound that the float32 bars rest on, measured on crafted blocks: one group, a
    float32 output, against float64 sums of the dequantized products."""
    from bux_amd import grouped_mxfp8 as gm
    rng = np.random.default_rng(36 + k)
    m, n = 512, 256
    a, b = _crafted(rng, m, k, kind), _crafted(rng, n, k, kind)
    announce("mfma error bound", kind, k)
    y = gm.rows(_gpu(a), _gpu(mxfp8.Blocks(b.values[None], b.scales[None])),
                to_gpu(np.array([m], np.int32)), torch.float32)
    torch.cuda.synchronize()
    x64, w64 = mxfp8.dequantized(a).astype(np.float64), mxfp8.dequantized(b).astype(np.float64)
    exact = x64 @ w64.T
    scale = np.abs(x64) @ np.abs(w64).T
    ratio = np.abs(y.cpu().numpy().astype(np.float64) - exact) / scale
    top = float(np.abs(exact).max())
    print(f"[mfma] {kind} k={k} max |err|/sum|ab| {ratio.max():.3e} (2^{np.log2(ratio.max()):.1f}) "
          f"mean {ratio.mean():.3e} max|err|/max|y| "
          f"{float((ratio * scale).max()) / top:.3e} sum|ab|/max|y| {float(scale.max()) / top:.1f}",
          flush=True)
    assert ratio.max() <= SUM_ERROR[kind]
    assert float((ratio * scale).max()) <= MAX_OF_MAX * top


@pytest.mark.parametrize("align", [256, 128])
def test_rows_with_groups_apart_in_a(lib, align):
    """`starts` (the reference's, grouped_mxfp8.py:116-154): each group's rows of a
    laid out apart, at whole tiles as grouped_glu.padded lays them, with garbage
    between; y packed. Against the oracle (float32 out, the GEMM bars) and bit for bit
    against the packed GEMM on the packed rows (each row's tile position is the same)."""
    from bux_amd import grouped_mxfp8 as gm
    rng = np.random.default_rng(37 + align)
    sizes = np.array([0, 130, 1, 3, 256, 0, 300, 100, 29], np.int32)
    k, n = 256, 384
    starts = np.zeros_like(sizes)
    at = 0
    for g, size in enumerate(sizes):
        starts[g] = at
        at += -(-int(size) // align) * align + align  # a spare tile between groups too
    m = at
    packed = _codes(rng, (int(sizes.sum()), k))
    a_vals = rng.integers(0, 255, (m, k), dtype=np.uint8)  # garbage between the groups
    a_scales = rng.integers(100, 140, (m, k // 32), dtype=np.uint8)
    src = 0
    for g, size in enumerate(sizes):
        a_vals[starts[g]:starts[g] + size] = packed.values[src:src + size]
        a_scales[starts[g]:starts[g] + size] = packed.scales[src:src + size]
        src += size
    a = mxfp8.Blocks(a_vals, a_scales)
    b = _codes(rng, (len(sizes), n, k), 0.05)
    height = int(sizes.sum()) + 60
    announce("gemm rows with starts", align)
    gs = to_gpu(sizes)
    y = gm.rows(_gpu(a), _gpu(b), gs, torch.float32, height=height, starts=to_gpu(starts))
    packed_pad = mxfp8.Blocks(np.concatenate([packed.values, np.zeros((60, k), np.uint8)]),
                              np.concatenate([packed.scales, np.ones((60, k // 32), np.uint8)]))
    y0 = gm.rows(_gpu(packed_pad), _gpu(b), gs, torch.float32, height=height)
    torch.cuda.synchronize()
    want = omoe.rows_mx(a, b, sizes, out="f32", height=height, starts=starts)
    _close_f32(y.cpu().numpy(), want, f"rows with starts, align {align}")
    assert torch.equal(y, y0)
    assert (y[int(sizes.sum()):] == 0).all()
