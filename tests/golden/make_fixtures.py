"""Writes the golden fixtures of the MoE expert path: small seeded inputs and the
outputs the CPU oracle (`oracle/`) gives for them, as ``tests/golden/*.npz``.

The reference holds no array fixtures of its own (its tests draw with ``jax.random``
at run time), so these are the repository's: the CPU suite re-derives each from the
oracle (tests/test_golden.py) and the GPU suite runs the HIP kernels on the same
inputs against the stored outputs (tests/test_gpu_golden.py), with no oracle call on
the box. The inputs reach the edge cases the reference's tests name: its group size
patterns (tests/test_grouped.py:24, tests/test_grouped_mxfp8.py:23), empty groups,
out-of-range picks, a block of zeros (tests/test_grouped_mxfp8.py:62-68), rows past
`filled`, K not a whole tile, values at and beyond the clamp of gpt-oss's activation
(tests/test_moe.py:519-528).

    python -m tests.golden.make_fixtures      # rewrites the .npz files
"""

import os

import numpy as np

from oracle import bf16, moe, mxfp8

HERE = os.path.dirname(os.path.abspath(__file__))
SIZES = np.array([70, 0, 100, 3, 77], np.int32)  # tests/test_grouped.py:24


def _bf16(rng, shape, scale=1.0, outliers=0.01):
    v = (rng.standard_normal(shape) * scale).astype(np.float32)
    flat = v.reshape(-1)
    flat[rng.choice(flat.size, max(1, int(flat.size * outliers)), replace=False)] *= 100
    return bf16.to_bf16(v)


def permute() -> dict:
    """sort_by_expert: 125 tokens x 2 picks over 5 experts, expert 1 empty, two picks
    out of range."""
    rng = np.random.default_rng(100)
    idx = rng.choice([0, 2, 3, 4], size=(125, 2)).astype(np.int32)
    idx[7, 1], idx[90, 0] = -1, 7
    s = moe.sort_by_expert(idx, 5)
    return {"idx": idx, "order": s.order, "inverse": s.inverse, "sizes": s.sizes,
            "offsets": s.offsets}


def quantize() -> dict:
    """Both MXFP8 copies of a (96, 160) matrix with a block of zeros, x100 outliers,
    powers of two at 448 * 2^e and tiny negatives; and of 100 rows read by index from
    40 tokens (k = 3), some indices -1, rows from 90 on past `filled`, height 128."""
    rng = np.random.default_rng(101)
    x = _bf16(rng, (96, 160))
    x[:32, :32] = 0
    x[40, 64] = bf16.to_bf16(np.array([448.0 * 2.0 ** -3], np.float32))[0]
    x[41, 96:128] = bf16.to_bf16(np.full(32, -1e-30, np.float32))
    rows, cols = mxfp8.quantized_twice(x, 96, True)
    z = _bf16(rng, (40, 64))
    order = rng.permutation(120)[:100].astype(np.int32)
    order[[3, 50, 97]] = -1
    index = np.where(order >= 0, order // 3, -1)
    g_rows, g_cols = mxfp8.quantized_twice(z, 90, True, index=index, height=128)
    return {"x": x, "rows_values": rows.values, "rows_scales": rows.scales,
            "cols_values": cols.values, "cols_scales": cols.scales,
            "z": z, "order": order, "k": np.int32(3), "filled": np.int32(90), "height": np.int32(128),
            "g_rows_values": g_rows.values, "g_rows_scales": g_rows.scales,
            "g_cols_values": g_cols.values, "g_cols_scales": g_cols.scales}


def _blocks(rng, shape, scale):
    x = bf16.to_f32(_bf16(rng, shape, scale))
    if len(shape) == 3:
        parts = [mxfp8.mx_quantize(a) for a in x]
        return mxfp8.Blocks(np.stack([p.values for p in parts]), np.stack([p.scales for p in parts]))
    return mxfp8.mx_quantize(x)


def _rows64(a, b, sizes, height):
    x, w = mxfp8.dequantized(a).astype(np.float64), mxfp8.dequantized(b).astype(np.float64)
    y = np.zeros((height, w.shape[1]))
    start = 0
    for g, size in enumerate(sizes.tolist()):
        y[start:start + size] = x[start:start + size] @ w[g].T
        start += size
    return y


def _contract64(a, b, sizes):
    x, y = mxfp8.dequantized(a).astype(np.float64), mxfp8.dequantized(b).astype(np.float64)
    dw = np.zeros((len(sizes), x.shape[0], y.shape[0]))
    start = 0
    for g, size in enumerate(sizes.tolist()):
        dw[g] = x[:, start:start + size] @ y[:, start:start + size].T
        start += size
    return dw


def gemm() -> dict:
    """The grouped MXFP8 GEMMs on operands of K = 96 (not a whole 128): rows of a
    (256, 96) by 5 experts' (64, 96), sizes [70, 0, 100, 3, 77]; contract of a
    (48, 256) and b (32, 256) over the same groups. Outputs are the float64 sums of
    the dequantized operands, stored as float32."""
    rng = np.random.default_rng(102)
    a = _blocks(rng, (256, 96), 1.0)
    b = _blocks(rng, (5, 64, 96), 0.02)
    y = _rows64(a, b, SIZES, 256)
    ca = _blocks(rng, (48, 256), 1.0)
    cb = _blocks(rng, (32, 256), 0.01)
    dw = _contract64(ca, cb, SIZES)
    return {"sizes": SIZES, "a_values": a.values, "a_scales": a.scales, "b_values": b.values,
            "b_scales": b.scales, "y": y.astype(np.float32),
            "ca_values": ca.values, "ca_scales": ca.scales, "cb_values": cb.values,
            "cb_scales": cb.scales, "dw": dw.astype(np.float32)}


ACTIVATIONS = {  # name: (activation, limit, up offset)
    "swish": ("swish", None, 0.0),
    "clamped": ("quick_gelu", 7.0, 1.0),  # gpt-oss (tests/test_moe.py:519-528)
}


def activation() -> dict:
    """The experts' activation and its gradient on projected (64, 32, 2) with values at
    and beyond the clamp of 7, row weights and dh; for SwiGLU and gpt-oss's clamped
    quick-GELU."""
    rng = np.random.default_rng(103)
    p = bf16.to_f32(_bf16(rng, (64, 32, 2), 3.0, 0.0))
    p[0, :4, 0] = [7.0, -7.0, 9.0, -8.0]
    p[0, :4, 1] = [7.0, 8.0, -9.0, 6.5]
    projected = bf16.to_bf16(p)
    weights = bf16.to_bf16(rng.random(64).astype(np.float32))
    dh = _bf16(rng, (64, 32), 0.01, 0.0)
    out = {"projected": projected, "weights": weights, "dh": dh}
    for name, (act, limit, offset) in ACTIVATIONS.items():
        ffn = moe.Ffn(act, limit, offset)
        out[f"{name}_h"] = moe.weighted_units(ffn, projected, weights)
        dp, dw = moe.weighted_units_backward(ffn, projected, weights, dh)
        out[f"{name}_dp"], out[f"{name}_dw"] = dp, dw
    return out


def token_sums() -> dict:
    """Each of 16 tokens' sum of its 3 rows of y (40, 24), indices 40..47 outside y
    (they add 0)."""
    rng = np.random.default_rng(104)
    y = _bf16(rng, (40, 24))
    inverse = rng.permutation(48)[:48].reshape(16, 3).astype(np.int32)
    return {"y": y, "inverse": inverse, "out": moe.sum_by_token(y, inverse)}


FIXTURES = {"permute": permute, "quantize": quantize, "gemm": gemm, "activation": activation,
            "token_sums": token_sums}


def path(name: str) -> str:
    return os.path.join(HERE, f"{name}.npz")


def load(name: str) -> dict:
    with np.load(path(name), allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def main() -> None:
    for name, make in FIXTURES.items():
        np.savez_compressed(path(name), **make())
        print("wrote", path(name), os.path.getsize(path(name)), "bytes")


if __name__ == "__main__":
    main()
