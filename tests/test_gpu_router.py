"""The HIP router (bux_route) against the oracle (oracle.router): the picks exactly
wherever the oracle's choices are apart by more than the float32 sums' rounding (and,
where they are not, picks whose choices equal the oracle's to within it); weights to a
bfloat16 rounding; logits and scores to float32 sums' rounding (the tolerances below).
Exact ties (equal logits) pick as the reference does, the lower index first."""

import numpy as np
import pytest
import torch

from oracle import bf16, router as orouter
from tests._util import announce, bf16_bits, normal_bf16, to_gpu, to_gpu_bf16

pytestmark = pytest.mark.gpu

LOGIT_ATOL = 3e-5  # float32 sums of d bfloat16 products, in another order
CHOICE_RTOL = 2e-4  # the scores' error after exp and the division


def _run(x, kernel, **kw):
    from bux_amd import router
    out = router.route(to_gpu_bf16(x), to_gpu_bf16(kernel), with_scores=True, with_logits=True,
                       **{k: (to_gpu(v) if isinstance(v, np.ndarray) else v) for k, v in kw.items()})
    torch.cuda.synchronize()
    return out


def _choice(logit, scored, router, choice_bias, groups, keep):
    scores = orouter.scores_of(logit, router)[:, :scored]
    c = scores if choice_bias is None else (scores + choice_bias).astype(np.float32)
    return orouter.limit_groups(c, groups, keep) if groups > 1 else c


def _check(x, kernel, *, k, scored=None, router="softmax", bias=None, scale=1.0,
           choice_bias=None, groups=1, keep=1, normalize=True, scaling=1.0, min_exact=0.99):
    n = kernel.shape[1]
    scored = n if scored is None else scored
    r = {"softmax": orouter.SOFTMAX, "sigmoid": orouter.SIGMOID,
         "sqrtsoftplus": orouter.SQRTSOFTPLUS}[router]
    got = _run(x, kernel, top_k=k, scored=scored, router=router, bias=bias,
               router_logit_scale=scale, router_bias=choice_bias, num_groups=groups,
               top_k_groups=keep, normalize_top_k=normalize, routed_scaling_factor=scaling)
    logit = orouter.logits(x, kernel, bias, scale)
    np.testing.assert_allclose(got.logits.cpu().numpy(), logit, rtol=0, atol=LOGIT_ATOL * max(1, scale))
    idx, w, sinks, scores = orouter.route(logit, scored, k, r, choice_bias, groups, keep, normalize,
                                          scaling)
    np.testing.assert_allclose(got.scores.cpu().numpy(), scores, rtol=CHOICE_RTOL, atol=1e-7)
    gi = got.idx.cpu().numpy()
    choice = _choice(logit, scored, r, choice_bias, groups, keep)
    rows = np.arange(len(gi))[:, None]
    # every pick's choice is the oracle's pick's at that place, to within the rounding
    cg, cw = choice[rows, gi], choice[rows, idx]
    close = (cg == cw) | (np.abs(cg - cw) <= CHOICE_RTOL * np.maximum(np.abs(cw), 1e-3))
    assert close.all(), np.argwhere(~close)[:5]
    assert all(len(set(row)) == k for row in gi)
    exact = (gi == idx).all(-1)
    assert exact.mean() >= min_exact, exact.mean()
    # weights where the picks agree: a bfloat16 rounding apart at most
    gw = bf16.to_f32(bf16_bits(got.weights))[exact]
    ww = bf16.to_f32(w)[exact]
    assert (np.abs(gw - ww) <= np.abs(ww) * 2.0 ** -7 + 1e-30).all()
    if sinks is not None:
        gs = bf16.to_f32(bf16_bits(got.sinks))[exact]
        ws = bf16.to_f32(sinks)[exact]
        assert (np.abs(gs - ws) <= np.abs(ws) * 2.0 ** -7 + 1e-30).all()
    else:
        assert got.sinks is None
    return got, idx


def test_qwen3_router_at_config_3():
    """Qwen3-30B-A3B: 128 experts, top-8 of a softmax, normalized; c3's 16384 tokens."""
    rng = np.random.default_rng(40)
    x = normal_bf16(rng, (16384, 2048))
    kernel = normal_bf16(rng, (2048, 128), 0.02)
    announce("route qwen3 c3")
    _check(x, kernel, k=8)


def test_every_tie_picks_the_first_experts():
    """A zero kernel ties every score: every token picks experts 0 and 1, each weighing
    1/2 (tests/test_moe.py:469-476)."""
    rng = np.random.default_rng(41)
    x = normal_bf16(rng, (100, 64))
    announce("route all ties")
    got = _run(x, np.zeros((64, 8), np.uint16), top_k=2)
    assert (got.idx.cpu().numpy() == np.array([0, 1])).all()
    assert (got.weights.float().cpu().numpy() == 0.5).all()


@pytest.mark.parametrize("router", ["softmax", "sigmoid", "sqrtsoftplus"])
def test_exact_logits_with_ties_pick_exactly(router):
    """Small-integer operands: every logit exact, half the experts copies of the other
    half (equal logits, equal scores): the picks equal the oracle's everywhere."""
    rng = np.random.default_rng(42)
    x = bf16.to_bf16(rng.integers(-3, 4, (300, 64)).astype(np.float32))
    half = rng.integers(-2, 3, (64, 16)).astype(np.float32) / 16
    kernel = bf16.to_bf16(np.repeat(half, 2, axis=1))
    announce("route exact ties", router)
    _check(x, kernel, k=6, router=router, min_exact=1.0)


def test_deepseek_groups_bias_and_scaling():
    """DeepSeek-V3's router: sigmoid scores, the aux-free bias on the choice, 4 of 8
    groups, top-8 of 256, normalized, times 2.5."""
    rng = np.random.default_rng(43)
    x = normal_bf16(rng, (4096, 1024))
    kernel = normal_bf16(rng, (1024, 256), 0.03)
    choice_bias = (rng.standard_normal(256) * 0.01).astype(np.float32)
    announce("route deepseek groups")
    _check(x, kernel, k=8, router="sigmoid", choice_bias=choice_bias, groups=8, keep=4,
           scaling=2.5)


def test_shared_expert_sinks():
    """shared_expert_sink: 2 sink columns past 64 experts share the normalization; a
    width that is not a multiple of 64 (the K loop's tail)."""
    rng = np.random.default_rng(44)
    x = normal_bf16(rng, (1000, 272))
    kernel = normal_bf16(rng, (272, 66), 0.05)
    announce("route sinks")
    _check(x, kernel, k=6, scored=64, router="sigmoid")


def test_scaled_sqrt_softplus_unnormalized_with_a_logit_bias():
    """The reference's "scaled" option (sqrtsoftplus, logit scale 2, weights times 2.5,
    not normalized) with gpt-oss's bias on the logits."""
    rng = np.random.default_rng(45)
    x = normal_bf16(rng, (2000, 512))
    kernel = normal_bf16(rng, (512, 32), 0.05)
    bias = (rng.standard_normal(32) * 0.1).astype(np.float32)
    announce("route scaled")
    _check(x, kernel, k=4, router="sqrtsoftplus", bias=bias, scale=2.0, normalize=False,
           scaling=2.5)


@pytest.mark.parametrize("t", [1, 77])
def test_wide_router_and_ragged_tokens(t):
    """768 scored experts (512 routed, 256 zero experts: LongCat-Flash's), top-12; token
    counts that leave a workgroup part-full."""
    rng = np.random.default_rng(46 + t)
    x = normal_bf16(rng, (t, 512))
    kernel = normal_bf16(rng, (512, 768), 0.05)
    announce("route wide", t)
    _check(x, kernel, k=12, min_exact=0.9)


def test_no_tokens():
    from bux_amd import router
    announce("route no tokens")
    got = router.route(torch.empty(0, 64, dtype=torch.bfloat16, device="cuda"),
                       torch.zeros(64, 8, dtype=torch.bfloat16, device="cuda"), top_k=2)
    torch.cuda.synchronize()
    assert got.idx.shape == (0, 2) and got.weights.shape == (0, 2)
