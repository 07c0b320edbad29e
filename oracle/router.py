"""The MoE router of bux, restated in numpy. TEST INFRASTRUCTURE ONLY (see `oracle`).

Follows ``src/bux/architecture/experts/moe.py``:

- `logits`: ``MoE._logits`` (moe.py:275-284) times ``router_logit_scale``
  (moe.py:249): ``x @ kernel`` of bfloat16 operands with float32 sums, plus the
  router's float32 bias, then the scale;
- `scores_of`: the ``match config.router`` of ``MoE._route`` (moe.py:251-257):
  ``jax.nn.softmax`` over every logit (the sinks' too), ``jax.nn.sigmoid`` or
  ``sqrt(jax.nn.softplus)`` of each, in float32;
- `limit_groups`: ``_limit_groups`` (moe.py:474-483): each of `groups` groups of
  experts scored by the sum of its best two choices (one if a group holds one), the
  `keep` best groups kept (ties to the lower group), the rest -inf;
- `route`: ``MoE._route`` (moe.py:236-273) off training (no random logits, no balance
  taps): scores split into the scored experts' and the sinks' (moe.py:258), the choice
  = scores + the aux-free bias (moe.py:259), group-limited, ``jax.lax.top_k`` (ties to
  the lower index), the weights = the picked scores, normalized by their sum plus the
  sinks' sum if ``normalize_top_k`` (moe.py:266-268), then cast to bfloat16 and
  multiplied by ``routed_scaling_factor`` in bfloat16 (moe.py:269-270: a python float
  times a bfloat16 array is a bfloat16 product of the bfloat16-rounded factor).

Pins, run by ``tests/test_router.py``: softmax rows sum to 1 and preserve the order of
the logits; sigmoid and sqrt-softplus against their closed forms at exact points
(sigmoid(0) = 1/2, softplus(0) = log 2); top-k against a brute-force loop over
``sorted`` with the index as tie-break; the reference's all-ties case (a zero kernel:
every token picks experts 0..k-1, tests/test_moe.py:469-476); group limiting against a
brute-force enumeration of the groups; normalized weights summing to 1 with no sinks;
the bfloat16 product against ``torch``'s bfloat16 multiply.

Float sums (the logits' dot, the softmax's denominator, the weights' total) follow
XLA's results only to rounding: the order XLA:CPU adds in is not observable without
jax. The oracle adds in float64 and rounds once to float32 where the reference adds in
float32; GPU results are compared to it within tolerances stated in each test, and the
picks exactly where the choices are apart by more than those tolerances.
"""

import numpy as np

from oracle import bf16

SOFTMAX, SIGMOID, SQRTSOFTPLUS = 0, 1, 2


def logits(x: np.ndarray, kernel: np.ndarray, bias: np.ndarray | None = None,
           scale: float = 1.0) -> np.ndarray:
    """Return the router's float32 logits: bfloat16 bits `x` (t, d) times bfloat16 bits
    `kernel` (d, n), each product exact, summed (here in float64, rounded once), plus
    the float32 `bias`, times `scale` (moe.py:249, 275-284)."""
    y = bf16.to_f32(x).astype(np.float64) @ bf16.to_f32(kernel).astype(np.float64)
    y = y.astype(np.float32)
    if bias is not None:
        y = y + np.asarray(bias, np.float32)
    return (y * np.float32(scale)).astype(np.float32)


def scores_of(logit: np.ndarray, router: int) -> np.ndarray:
    """Return the float32 scores of float32 logits (moe.py:251-257)."""
    z = logit.astype(np.float64)
    if router == SOFTMAX:
        e = np.exp(z - z.max(-1, keepdims=True))
        s = e / e.sum(-1, keepdims=True)
    elif router == SIGMOID:
        s = 1.0 / (1.0 + np.exp(-z))
    elif router == SQRTSOFTPLUS:
        s = np.sqrt(np.logaddexp(z, 0.0))
    else:
        raise ValueError(f"router {router}")
    return s.astype(np.float32)


def top_k(choice: np.ndarray, k: int) -> np.ndarray:
    """Return the indices of each row's k largest, the largest first, equal values in
    index order (``jax.lax.top_k``); -inf sorts last like any smaller value."""
    return np.argsort(-choice.astype(np.float64), axis=-1, kind="stable")[..., :k].astype(np.int32)


def limit_groups(choice: np.ndarray, groups: int, keep: int) -> np.ndarray:
    """Return `choice` (t, n) at -inf outside each row's `keep` best of `groups` groups
    of n / groups experts, a group scored by its best two (moe.py:474-483)."""
    t, n = choice.shape
    grouped = choice.reshape(t, groups, n // groups).astype(np.float32)
    best = -np.sort(-grouped, axis=-1)[..., : min(2, n // groups)]
    score = best[..., 0].copy()
    for j in range(1, best.shape[-1]):
        score = (score + best[..., j]).astype(np.float32)
    kept = np.zeros((t, groups), bool)
    np.put_along_axis(kept, top_k(score, keep), True, axis=-1)
    out = np.where(kept[..., None], grouped, np.float32(-np.inf))
    return out.reshape(t, n).astype(np.float32)


def times_in_bf16(w: np.ndarray, factor: float) -> np.ndarray:
    """Return bfloat16 bits of ``w.astype(bfloat16) * factor`` as jax computes it: the
    python float rounded to bfloat16, the product of the two rounded to bfloat16."""
    wb = bf16.to_bf16(np.asarray(w, np.float32))
    if factor == 1.0:
        return wb
    f = bf16.to_f32(bf16.to_bf16(np.float32(factor)))
    return bf16.to_bf16((bf16.to_f32(wb) * f).astype(np.float32))


def route(logit: np.ndarray, scored: int, k: int, router: int = SOFTMAX,
          choice_bias: np.ndarray | None = None, groups: int = 1, keep: int = 1,
          normalize: bool = True, scaling: float = 1.0):
    """Return (idx int32 (t, k), weights bf16 bits (t, k), sinks bf16 bits (t, s) or
    None, scores float32 (t, scored)) from float32 logits (t, scored + s): moe.py:
    236-273 off training."""
    scores_all = scores_of(logit, router)
    scores, sinks = scores_all[:, :scored], scores_all[:, scored:]
    choice = scores if choice_bias is None else (scores + np.asarray(choice_bias, np.float32))
    choice = choice.astype(np.float32)
    if groups > 1:
        choice = limit_groups(choice, groups, keep)
    idx = top_k(choice, k)
    w = np.take_along_axis(scores, idx, axis=-1).astype(np.float32)
    if normalize:
        total = w[:, 0].copy()
        for j in range(1, k):
            total = (total + w[:, j]).astype(np.float32)
        if sinks.shape[-1]:
            s_sum = sinks[:, 0].copy()
            for j in range(1, sinks.shape[-1]):
                s_sum = (s_sum + sinks[:, j]).astype(np.float32)
            total = (total + s_sum).astype(np.float32)
        w = (w / total[:, None]).astype(np.float32)
        sinks = (sinks / total[:, None]).astype(np.float32)
    weights = times_in_bf16(w, scaling)
    sink_bits = times_in_bf16(sinks, scaling) if sinks.shape[-1] else None
    return idx, weights, sink_bits, scores
