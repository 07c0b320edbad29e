"""The exact restatement of the layer: every GEMM and token sum in float64, rounded once,
the quantization and rounding points unchanged (`oracle.moe` with exact=True). It tells
how far a float32 summation order lands from the exact result, and how far an error of
the block-scaled MFMA's size in each GEMM carries the layer end to end.

Measured here (the CPU, "small": t 1024, k 4, 16 experts, d 256, f 256):
- the oracle's float32 order (numpy's BLAS, as XLA:CPU sums in float32) against the
  exact layer: 3e-6 to 8e-5 for y and every gradient, far below the north star's 1e-3;
- each GEMM's float64 result perturbed by Gaussian noise of relative norm 1.5e-5 (what
  the MI355X's v_mfma_scale_f32_32x32x64_f8f6f4 leaves against the exact sum of the
  same products, inside each instruction: chaining its accumulator or summing each
  instruction's partial in float32 or float64 gives the same error) carries the layer
  1.0e-3 to 2.1e-3 from the exact one, the GPU layer's own drift from the oracle: a
  GEMM output's last bits flip its bfloat16 rounding now and then, that flips an E4M3
  code downstream (a step of 1/16), and so on through the chain.
"""

from fractions import Fraction

import numpy as np
import pytest

from oracle import bf16, moe, mxfp8

SMALL = (1024, 4, 16, 256, 256)


def _exact_bf16(v: float) -> int:
    """The bfloat16 nearest to v (ties to even), by exact rationals."""
    f = Fraction(v)
    c = int(bf16.to_bf16(np.array([v], np.float32))[0])
    cands = [(c + d) & 0xFFFF for d in (-1, 0, 1)]
    vals = [Fraction(float(bf16.to_f32(np.array([q], np.uint16))[0])) for q in cands]
    best = min(range(3), key=lambda i: (abs(vals[i] - f), cands[i] & 1))
    return cands[best]


def test_rounding_from_float64_is_one_rounding():
    """`bf16.from_f64` against exact rational rounding on values just off bfloat16 ties
    (where a rounding through float32 rounds twice and differs), and on plain values."""
    rng = np.random.default_rng(3)
    b = bf16.to_f32(bf16.to_bf16(rng.standard_normal(2000).astype(np.float32))).astype(np.float64)
    half = 2.0 ** (np.floor(np.log2(np.abs(b))) - 8)
    near = b + half * (1 + rng.choice([-1, 1], b.size) * 2.0 ** -30)
    plain = rng.standard_normal(500) * 10.0 ** rng.integers(-5, 5, 500)
    for x in (near, plain):
        want = np.array([_exact_bf16(v) for v in x], np.uint16)
        np.testing.assert_array_equal(bf16.from_f64(x), want)
    assert (bf16.to_bf16(near.astype(np.float32)) != np.array([_exact_bf16(v) for v in near])).any()


def _blocks(rng, shape):
    x = rng.standard_normal(shape).astype(np.float32)
    if len(shape) == 3:
        parts = [mxfp8.mx_quantize(m) for m in x]
        return mxfp8.Blocks(np.stack([p.values for p in parts]), np.stack([p.scales for p in parts]))
    return mxfp8.mx_quantize(x)


def test_the_exact_gemms_are_float64_sums_rounded_once():
    """rows_mx and contract_mx with exact=True: brute-force float64 sums of the
    dequantized products (Python's float adds, term by term), each rounded once."""
    rng = np.random.default_rng(4)
    sizes = np.array([20, 0, 31, 13], np.int32)
    m, k, n = int(sizes.sum()), 64, 16
    a, b = _blocks(rng, (m, k)), _blocks(rng, (len(sizes), n, k))
    x, w = mxfp8.dequantized(a).astype(np.float64), mxfp8.dequantized(b).astype(np.float64)
    want = np.zeros((m, n))
    ends = np.cumsum(sizes)
    for i in range(m):
        g = int(np.searchsorted(ends, i, side="right"))
        for j in range(n):
            want[i, j] = sum(float(x[i, q]) * float(w[g, j, q]) for q in range(k))
    np.testing.assert_array_equal(moe.rows_mx(a, b, sizes, exact=True), bf16.from_f64(want))
    np.testing.assert_allclose(moe.rows_mx(a, b, sizes, out="f64", exact=True), want, rtol=1e-15,
                               atol=1e-300)
    at, bt = _blocks(rng, (k, m)), _blocks(rng, (n, m))
    xa, ya = mxfp8.dequantized(at).astype(np.float64), mxfp8.dequantized(bt).astype(np.float64)
    dw = np.zeros((len(sizes), k, n))
    start = 0
    for g, size in enumerate(sizes):
        for i in range(k):
            for j in range(n):
                dw[g, i, j] = sum(float(xa[i, r]) * float(ya[j, r]) for r in range(start, start + size))
        start += size
    np.testing.assert_array_equal(moe.contract_mx(at, bt, sizes, exact=True), bf16.from_f64(dw))


def layer_inputs(rng, t, k, e, d, f):
    """The GPU layer tests' inputs (tests/test_gpu_layer.py `_inputs`)."""
    def nb(shape, scale=1.0):
        return bf16.to_bf16((rng.standard_normal(shape) * scale).astype(np.float32))
    z = nb((t, d))
    idx = np.stack([rng.choice(e, k, replace=False) for _ in range(t)]).astype(np.int32)
    w = bf16.to_bf16(rng.random((t, k)).astype(np.float32) / k)
    return z, idx, w, nb((e, d, f, 2), 0.02), nb((e, f, d), 0.02), nb((t, d), 1e-2)


def rel(got, want) -> float:
    a = bf16.to_f32(got).astype(np.float64)
    b = bf16.to_f32(want).astype(np.float64)
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


def run_layer(z, idx, w, up, down, dy, exact, ffn=moe.Ffn()):
    """y and the gradients to z, the weights, up and down."""
    k = idx.shape[1]
    y, saved = moe.layer_forward(z, idx, w, up, down, ffn, exact=exact)
    g = moe.layer_backward(saved, dy, z, up, down, k, ffn, exact=exact)
    return {"y": y, **{key: g[key] for key in ("z", "weights", "up", "down")}}


def with_gemm_noise(monkeypatch, sigma: float, seed: int) -> None:
    """Make the oracle's MXFP8 GEMMs exact, then perturb each float64 result by Gaussian
    noise of relative norm `sigma` before its one rounding to bfloat16."""
    rng = np.random.default_rng(seed)
    rows, contract = moe.rows_mx, moe.contract_mx

    def perturbed(fn):
        def call(*a, out="bf16", exact=False, **kw):
            y = fn(*a, out="f64", exact=True, **kw)
            rms = float(np.sqrt(np.mean(y * y))) if y.size else 0.0
            y = y + rng.standard_normal(y.shape) * sigma * rms
            return bf16.from_f64(y) if out == "bf16" else y.astype(np.float32)
        return call

    monkeypatch.setattr(moe, "rows_mx", perturbed(rows))
    monkeypatch.setattr(moe, "contract_mx", perturbed(contract))


def test_a_float32_order_lands_far_inside_the_bar_of_the_exact_layer():
    rng = np.random.default_rng(47)
    args = layer_inputs(rng, *SMALL)
    f32, exact = run_layer(*args, exact=False), run_layer(*args, exact=True)
    errs = {key: rel(f32[key], exact[key]) for key in exact}
    print("[exact] float32 order vs exact", {key: f"{v:.2e}" for key, v in errs.items()})
    assert max(errs.values()) <= 2e-4, errs


def test_an_error_of_the_mfmas_size_in_each_gemm_carries_the_layer_past_1e3(monkeypatch):
    """The GPU's drift reproduced on the CPU: per-GEMM noise of the block-scaled MFMA's
    measured size (1.5e-5 relative) in the exact layer lands 0.5e-3 to 4e-3 from it."""
    rng = np.random.default_rng(47)
    args = layer_inputs(rng, *SMALL)
    exact = run_layer(*args, exact=True)
    with_gemm_noise(monkeypatch, 1.5e-5, seed=5)
    noisy = run_layer(*args, exact=True)
    errs = {key: rel(noisy[key], exact[key]) for key in exact}
    print("[exact] mfma-sized noise vs exact", {key: f"{v:.2e}" for key, v in errs.items()})
    assert all(5e-4 <= v <= 4e-3 for v in errs.values()), errs
