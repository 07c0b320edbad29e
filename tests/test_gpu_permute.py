"""The HIP sort of picks by expert, and the token path's gathers and sums, against the
oracle: integer outputs bit-exact; the float32 sums of `sum_by_token` too, as both add
a token's picks in order."""

import numpy as np
import pytest
import torch

from oracle import bf16, moe as omoe
from tests._util import announce, bf16_bits, normal_bf16, to_gpu, to_gpu_bf16

pytestmark = pytest.mark.gpu


def _sort(idx: np.ndarray, e: int):
    from bux_amd import moe
    s = moe.sort_by_expert(to_gpu(idx.astype(np.int32)), e)
    torch.cuda.synchronize()
    return [a.cpu().numpy() for a in s]


def _check(idx: np.ndarray, e: int):
    order, inverse, sizes, offsets = _sort(idx, e)
    want = omoe.sort_by_expert(idx, e)
    np.testing.assert_array_equal(order, want.order)
    np.testing.assert_array_equal(inverse, want.inverse)
    np.testing.assert_array_equal(sizes, want.sizes)
    np.testing.assert_array_equal(offsets[:e], want.offsets)
    assert offsets[e] == want.sizes.sum()


@pytest.mark.parametrize("sizes", [[70, 0, 100, 3, 77], [0, 130, 1, 3, 256, 0, 300, 100]])
def test_the_references_size_patterns(lib, sizes):
    rng = np.random.default_rng(20)
    flat = np.repeat(np.arange(len(sizes)), sizes)
    rng.shuffle(flat)
    announce("permute sizes", sizes)
    _check(flat.reshape(-1, 1), len(sizes))


@pytest.mark.parametrize("t,k,e", [(4096, 2, 8), (16384, 8, 128), (8192, 4, 128), (8192, 8, 256),
                                   (1000, 3, 1), (77, 5, 300), (1, 1, 4)])
def test_random_picks(lib, t, k, e):
    rng = np.random.default_rng(21)
    idx = np.stack([rng.choice(e, k, replace=e < k) for _ in range(t)])
    announce("permute random", t, k, e)
    _check(idx, e)


def test_out_of_range_picks_sort_last(lib):
    rng = np.random.default_rng(22)
    idx = rng.integers(-3, 70, (3000, 6))
    announce("permute out of range")
    _check(idx, 64)


def test_skewed_loads_with_empty_experts(lib):
    """Config 5's loads: Zipf(1.2) shares, a fifth of the experts empty."""
    rng = np.random.default_rng(23)
    e, t, k = 256, 8192, 8
    p = 1.0 / np.arange(1, e + 1) ** 1.2
    p[int(e * 0.8):] = 0
    p = rng.permutation(p / p.sum())
    idx = np.stack([rng.choice(e, k, replace=False, p=p) for _ in range(t)])
    announce("permute zipf")
    _check(idx, e)


def test_no_picks(lib):
    from bux_amd import moe
    announce("permute empty")
    s = moe.sort_by_expert(torch.empty(0, 2, dtype=torch.int32, device="cuda"), 4)
    torch.cuda.synchronize()
    assert s.sizes.cpu().tolist() == [0, 0, 0, 0] and s.offsets.cpu().tolist() == [0] * 5


def test_token_rows_and_picked_weights(lib):
    from bux_amd import moe
    rng = np.random.default_rng(24)
    t, k, d, e = 500, 4, 264, 16
    z = normal_bf16(rng, (t, d))
    w = normal_bf16(rng, (t, k))
    idx = rng.integers(0, e, (t, k)).astype(np.int32)
    s = omoe.sort_by_expert(idx, e)
    announce("token_rows")
    order = to_gpu(s.order)
    rows = moe.token_rows(to_gpu_bf16(z), order, k)
    pw = moe.picked_weights(to_gpu_bf16(w), order)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bf16_bits(rows), omoe.token_rows(z, s.order, k))
    np.testing.assert_array_equal(bf16_bits(pw), omoe.picked_weights(w, s.order))


@pytest.mark.parametrize("d", [264, 1])
def test_token_rows_read_zeros_where_an_order_entry_leaves_the_tokens(lib, d):
    """An order entry whose token lies outside z (past its rows, or negative) gives a row
    of 0 rather than a read outside z; the others are z[order // k]. (The reference's
    orders, the sort's, always lie inside.) Width 1 is picked_weights' kernel."""
    from bux_amd import moe
    rng = np.random.default_rng(26)
    t, k, m = 200, 4, 700
    z = normal_bf16(rng, (t, d))
    order = rng.permutation(t * k)[:m].astype(np.int32)
    order[:6] = [-1, -k, t * k, t * k + k - 1, 2**31 - 1, -(2**31)]
    announce("token_rows out of range", d)
    rows = moe.token_rows(to_gpu_bf16(z), to_gpu(order), k)
    torch.cuda.synchronize()
    inside = (order >= 0) & (order // k < t)
    want = np.where(inside[:, None], z[np.where(inside, order // k, 0)], 0).astype(np.uint16)
    np.testing.assert_array_equal(bf16_bits(rows), want)


@pytest.mark.parametrize("t,k,d", [(300, 8, 2048), (64, 2, 256), (50, 4, 2880)])
def test_sum_by_token_adds_in_float32_in_pick_order(lib, t, k, d):
    """Bit-exact: each token's k rows added in float32, in order, rounded once; an index
    past y's rows adds 0 (mode="fill")."""
    from bux_amd import moe
    rng = np.random.default_rng(25)
    m = t * k
    y = normal_bf16(rng, (m - 5, d))
    inverse = rng.permutation(m).astype(np.int32).reshape(t, k)  # m - 5.. fall outside y
    announce("sum_by_token", t, k, d)
    got = moe.sum_by_token(to_gpu_bf16(y), to_gpu(inverse))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bf16_bits(got), omoe.sum_by_token(y, inverse))
