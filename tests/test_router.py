"""The router's oracle (oracle.router) against what fixes it without jax: closed forms,
brute force over small cases, and the reference's own all-ties case."""

import itertools

import numpy as np
import pytest
import torch

from oracle import bf16, router as orouter


def test_softmax_rows_sum_to_one_and_keep_the_logits_order():
    rng = np.random.default_rng(0)
    z = (rng.standard_normal((50, 40)) * 3).astype(np.float32)
    s = orouter.scores_of(z, orouter.SOFTMAX)
    assert np.allclose(s.sum(-1), 1.0, atol=1e-6)
    assert (np.argsort(s, -1, kind="stable") == np.argsort(z, -1, kind="stable")).all()
    # shift invariance: softmax(z + c) == softmax(z)
    assert np.allclose(orouter.scores_of(z + 5.0, orouter.SOFTMAX), s, rtol=1e-6, atol=1e-7)


def test_sigmoid_and_sqrt_softplus_at_exact_points():
    z = np.array([[0.0, 1.0, -1.0, 30.0, -30.0]], np.float32)
    sg = orouter.scores_of(z, orouter.SIGMOID)
    assert sg[0, 0] == 0.5
    assert np.isclose(sg[0, 1] + sg[0, 2], 1.0, atol=1e-7)  # sigmoid(x) + sigmoid(-x) = 1
    sp = orouter.scores_of(z, orouter.SQRTSOFTPLUS)
    assert np.isclose(sp[0, 0], np.sqrt(np.log(2.0)), rtol=1e-7)
    assert np.isclose(sp[0, 3], np.sqrt(30.0), rtol=1e-6)  # softplus(x) -> x
    assert 0 < sp[0, 4] < 1e-6


def _brute_top_k(row, k):
    return [i for _, i in sorted(((-float(v), i) for i, v in enumerate(row)))[:k]]


def test_top_k_is_the_largest_first_ties_to_the_lower_index():
    rng = np.random.default_rng(1)
    choice = rng.integers(-3, 4, (200, 12)).astype(np.float32)  # many ties
    choice[0] = -np.inf
    choice[1, 5:] = -np.inf
    got = orouter.top_k(choice, 5)
    for row, g in zip(choice, got):
        assert list(g) == _brute_top_k(row, 5)


def test_every_tie_picks_the_first_experts():
    """The reference's case: a zero router kernel ties every score; each token picks
    experts 0 .. k-1 (tests/test_moe.py:469-476)."""
    x = bf16.to_bf16(np.random.default_rng(2).standard_normal((10, 16)).astype(np.float32))
    kernel = np.zeros((16, 8), np.uint16)
    idx, w, _, _ = orouter.route(orouter.logits(x, kernel), 8, 2)
    assert (idx == np.array([0, 1])).all()
    assert (bf16.to_f32(w) == 0.5).all()


def test_group_limit_against_every_choice_of_groups():
    rng = np.random.default_rng(3)
    t, groups, per, keep = 30, 4, 3, 2
    choice = rng.standard_normal((t, groups * per)).astype(np.float32)
    got = orouter.limit_groups(choice, groups, keep)
    for r in range(t):
        g = choice[r].reshape(groups, per)
        score = [np.float32(np.sort(gg)[-1]) + np.float32(np.sort(gg)[-2]) for gg in g]
        best = max(itertools.combinations(range(groups), keep),
                   key=lambda c: (sorted((score[i] for i in c), reverse=True), [-i for i in c]))
        # the kept set is the `keep` largest scores; with distinct scores it is unique
        want = np.full((groups, per), -np.inf, np.float32)
        for i in best:
            want[i] = g[i]
        assert (got[r].reshape(groups, per) == want).all()


def test_one_expert_a_group_scores_by_itself():
    choice = np.array([[0.1, 0.9, 0.3, 0.5]], np.float32)
    got = orouter.limit_groups(choice, 4, 2)
    assert (got == np.array([[-np.inf, 0.9, -np.inf, 0.5]], np.float32)).all()


def test_normalized_weights_sum_to_one_and_sinks_share_the_total():
    rng = np.random.default_rng(4)
    z = rng.standard_normal((40, 10)).astype(np.float32)
    idx, w, sinks, scores = orouter.route(z, 8, 3, router=orouter.SIGMOID)
    wf, sf = bf16.to_f32(w), bf16.to_f32(sinks)
    # before the bfloat16 rounding the picks and the sinks sum to 1
    assert np.allclose(wf.sum(-1) + sf.sum(-1), 1.0, atol=3e-2)
    picked = np.take_along_axis(scores, idx, -1)
    total = picked.sum(-1) + orouter.scores_of(z, orouter.SIGMOID)[:, 8:].sum(-1)
    assert np.allclose(wf, picked / total[:, None], rtol=8e-3)


def test_scaling_is_a_bfloat16_product():
    """jax turns a python float into the array's dtype before the product (weak typing):
    a product of two bfloat16 values, rounded to bfloat16 (torch's bfloat16 x bfloat16
    here). 2.827 is not a bfloat16: its rounding shows."""
    rng = np.random.default_rng(5)
    w = rng.random(1000).astype(np.float32)
    for factor in (2.5, 2.827, 1.0):
        got = orouter.times_in_bf16(w, factor)
        f = torch.tensor(factor, dtype=torch.bfloat16)
        want = (torch.from_numpy(w).to(torch.bfloat16) * f).view(torch.int16).numpy()
        assert (got == want.view(np.uint16)).all(), factor


def test_logits_are_the_float32_product_plus_bias_times_scale():
    rng = np.random.default_rng(6)
    x = rng.integers(-4, 5, (5, 32)).astype(np.float32)
    k = rng.integers(-4, 5, (32, 6)).astype(np.float32)
    bias = np.arange(6, dtype=np.float32) / 4
    got = orouter.logits(bf16.to_bf16(x), bf16.to_bf16(k), bias, 2.0)
    assert (got == (x @ k + bias) * 2).all()


def test_unnormalized_weights_are_the_scores():
    rng = np.random.default_rng(7)
    z = rng.standard_normal((20, 16)).astype(np.float32)
    idx, w, sinks, scores = orouter.route(z, 16, 4, router=orouter.SQRTSOFTPLUS,
                                          normalize=False, scaling=2.5)
    assert sinks is None
    want = orouter.times_in_bf16(np.take_along_axis(scores, idx, -1), 2.5)
    assert (w == want).all()
