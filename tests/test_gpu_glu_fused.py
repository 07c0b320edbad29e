"""The fused up GEMM (`grouped_mxfp8.activated`, the reference's
grouped_cudnn.activated, grouped_cudnn.py:161-205) and the fused down dgrad
(`grouped_mxfp8.activation_grad`, grouped_cudnn.activation_grad, :211-263) against the
unfused kernels they replace: the rows GEMM into the product (into dh), then the
activation's quantizer (its quantizing backward). Both run on
the same GPU operands; the fused kernel must give the same bits in every output (the
product, h along its units, h^T along the rows). The unfused pair is pinned against
the oracle by test_gpu_gemm.py and test_gpu_layer.py.

The cases move the groups' first rows off the 32-row blocks of h^T (whose blocks with a
group's first row inside go through the fix-up kernel), hold empty groups, groups
smaller than a block and several groups' first rows inside one block, rows past the
groups (zeros), a hidden width that is not a whole number of 128s (the row copy's K
padding) and the three gated activations the fused kernel runs."""

import numpy as np
import pytest
import torch

from tests._util import announce

pytestmark = pytest.mark.gpu

# (sizes, rows, d, f, activation)
CASES = [
    ([0, 130, 1, 3, 256, 0, 300, 100, 29], 900, 256, 160, "swiglu"),
    ([33, 31, 64, 0, 0, 517, 2, 2, 2], 700, 128, 32, "clamped"),
    ([5, 3, 10, 7, 0, 1, 1, 1], 64, 128, 96, "swiglu"),
    ([512, 256, 0, 768], 1536, 256, 256, "clamped"),
    ([40, 0, 300, 7, 100], 480, 256, 192, "situglu"),
    ("multinomial", 16 * 1024, 512, 384, "swiglu"),
]

# (activation, limit, up_offset, up_softcap): SwiGLU, gpt-oss's clamped GeGLU form, and
# SiTU-GLU with its soft cap (grouped_glu.epilogue, experts/grouped_glu.py:119-136)
ACTS = {"swiglu": ("swish", None, 0.0, None), "clamped": ("quick_gelu", 7.0, 1.0, None),
        "situglu": ("situ", None, 0.0, 6.0)}


def _sizes(spec, rows, groups_if_random, rng):
    if spec != "multinomial":
        return np.array(spec, np.int32)
    s = rng.multinomial(rows - 37, np.ones(groups_if_random) / groups_if_random)
    return s.astype(np.int32)


def _run(sizes_np, rows, d, f, act, seed):
    from bux_amd import grouped_mxfp8 as gm, moe
    torch.manual_seed(seed)
    dev = torch.device("cuda")
    groups = len(sizes_np)
    height = gm.whole(rows)
    filled = int(sizes_np.sum())
    assert filled <= rows
    x = (torch.randn(rows, d, device=dev) * 2.0).to(torch.bfloat16)
    x.view(-1)[torch.randint(0, x.numel(), (max(1, x.numel() // 500),), device=dev)] *= 100
    w_up = (torch.randn(groups, d, 2 * f, device=dev) * 0.05).to(torch.bfloat16)
    weights = torch.rand(rows, device=dev).to(torch.bfloat16)
    sizes = torch.tensor(sizes_np, dtype=torch.int32, device=dev)
    filled_t = torch.tensor([filled], dtype=torch.int32, device=dev)
    x_k, _ = gm.quantized_twice(x, filled_t, False, height=height)
    _, up_k = gm.quantized_twice(w_up)
    ffn = moe.Ffn(*ACTS[act])
    # unfused: the rows GEMM, then the activation's quantizer
    projected = gm.rows(x_k, up_k, sizes, height=rows)
    h_k, h_m, _ = moe.weighted_units_quantized(ffn, projected.view(rows, f, 2), weights, filled_t,
                                               height)
    # fused
    p2, h_k2, h_m2 = gm.activated(x_k, up_k, sizes, weights, ffn.struct(True), rows)
    torch.cuda.synchronize()
    return (projected, h_k, h_m), (p2, h_k2, h_m2)


def _same(name, a, b):
    assert a.shape == b.shape, (name, a.shape, b.shape)
    diff = (a.view(torch.uint8) != b.view(torch.uint8)) if a.dtype != torch.uint8 else (a != b)
    bad = int(diff.sum())
    if bad:
        where = diff.nonzero()[:5].tolist()
        pytest.fail(f"{name}: {bad} bytes differ, first at {where}")


@pytest.mark.parametrize("case", range(len(CASES)))
def test_fused_up_gemm_is_the_unfused_pair_bit_for_bit(lib, case):
    spec, rows, d, f, act = CASES[case]
    rng = np.random.default_rng(70 + case)
    sizes = _sizes(spec, rows, 64, rng)
    announce("glu fused", case, f"groups={len(sizes)} rows={rows} d={d} f={f} {act}")
    (p, hk, hm), (p2, hk2, hm2) = _run(sizes, rows, d, f, act, 70 + case)
    _same("product", p, p2)
    _same("h values", hk.values, hk2.values)
    _same("h scales", hk.scales, hk2.scales)
    _same("h^T values", hm.values, hm2.values)
    _same("h^T scales", hm.scales, hm2.scales)


def test_fused_up_gemm_at_config_3(lib):
    """Qwen3-30B-A3B's experts: 131072 rows, 128 experts, d 2048, f 768."""
    rng = np.random.default_rng(77)
    rows = 16384 * 8
    sizes = rng.multinomial(rows, np.ones(128) / 128).astype(np.int32)
    announce("glu fused", "config 3")
    (p, hk, hm), (p2, hk2, hm2) = _run(sizes, rows, 2048, 768, "swiglu", 77)
    _same("product", p, p2)
    _same("h values", hk.values, hk2.values)
    _same("h scales", hk.scales, hk2.scales)
    _same("h^T values", hm.values, hm2.values)
    _same("h^T scales", hm.scales, hm2.scales)


@pytest.mark.parametrize("t,k,e,d,f,act", [(300, 4, 8, 256, 160, "clamped"),
                                           (4096, 8, 64, 512, 384, "swiglu"),
                                           (500, 4, 16, 256, 128, "situglu")])
def test_layer_with_the_fused_up_gemm_is_bit_identical(lib, t, k, e, d, f, act):
    """The whole layer, forward and backward, with and without the fused up GEMM and
    the fused down dgrad."""
    from bux_amd import moe
    torch.manual_seed(t)
    dev = torch.device("cuda")
    z = torch.randn(t, d, device=dev).to(torch.bfloat16)
    idx = torch.stack([torch.randperm(e, device=dev)[:k] for _ in range(t)]).to(torch.int32)
    idx[::7, 0] = e  # picks outside the experts: rows past the groups
    w = torch.rand(t, k, device=dev).to(torch.bfloat16)
    up = (torch.randn(e, d, f, 2, device=dev) * 0.05).to(torch.bfloat16)
    down = (torch.randn(e, f, d, device=dev) * 0.05).to(torch.bfloat16)
    dy = (torch.randn(t, d, device=dev) * 0.01).to(torch.bfloat16)
    ffn = moe.Ffn(*ACTS[act])
    announce("layer fused", t, k, e, d, f, act)
    results = []
    for fused in (False, True):
        out, saved = moe.experts_forward(z, idx, w, up, down, ffn, fused=fused)
        grads = moe.experts_backward(saved, dy, up, down, ffn, fused=fused)
        results.append((out, grads))
    torch.cuda.synchronize()
    (o0, g0), (o1, g1) = results
    _same("y", o0, o1)
    for key in g0:
        _same(f"d{key}", g0[key], g1[key])


@pytest.mark.parametrize("case", [0, 1, 5])
def test_fused_up_gemm_against_the_oracle(lib, case):
    """The fused kernel's outputs against the oracle run on its own from the same bits
    (x and the kernels quantized by the oracle's quantizer, which the GPU's matches bit
    for bit): the product within the north star's bar; h's copies E4M3 code for code,
    every code or scale that differs attributed to a bfloat16 step between the GPU's h
    (the unfused kernels', bit for bit the fused kernel's) and the oracle's."""
    from bux_amd import grouped_mxfp8 as gm, moe
    from oracle import bf16, moe as omoe, mxfp8 as omx
    from tests._util import attribute_codes, bf16_bits, rel_err, untiled
    spec, rows, d, f, act = CASES[case]
    rng = np.random.default_rng(80 + case)
    sizes_np = _sizes(spec, rows, 64, rng)
    announce("glu fused vs oracle", case)
    torch.manual_seed(80 + case)
    dev = torch.device("cuda")
    groups, height, filled = len(sizes_np), gm.whole(rows), int(sizes_np.sum())
    x = (torch.randn(rows, d, device=dev) * 2.0).to(torch.bfloat16)
    w_up = (torch.randn(groups, d, 2 * f, device=dev) * 0.05).to(torch.bfloat16)
    weights = torch.rand(rows, device=dev).to(torch.bfloat16)
    sizes = torch.tensor(sizes_np, dtype=torch.int32, device=dev)
    filled_t = torch.tensor([filled], dtype=torch.int32, device=dev)
    x_k, _ = gm.quantized_twice(x, filled_t, False, height=height)
    _, up_k = gm.quantized_twice(w_up)
    ffn = moe.Ffn(*ACTS[act])
    product, h_k, h_m = gm.activated(x_k, up_k, sizes, weights, ffn.struct(True), rows)
    _, _, h = moe.weighted_units_quantized(ffn, product.view(rows, f, 2), weights, filled_t, height,
                                           keep=True)
    torch.cuda.synchronize()
    xb, wb, rw = bf16_bits(x), bf16_bits(w_up), bf16_bits(weights)
    ox_k, _ = omx.quantized_twice(xb, filled, True, height=height)
    _, oup_k = omx.quantized_twice(wb, d)
    want = omoe.rows_mx(ox_k, oup_k, sizes_np, height=rows)
    err = rel_err(bf16.to_f32(bf16_bits(product)), bf16.to_f32(want))
    o = omoe.Ffn(*ACTS[act])
    oh = np.zeros((rows, f), np.uint16)
    oh[:filled] = omoe.weighted_units(o, want[:filled].reshape(filled, f, 2), rw[:filled])
    gh = bf16_bits(h)
    want_k, want_m = omx.quantized_twice(oh, filled, True, height=height)
    gpad, opad = np.zeros((height, f), np.uint16), np.zeros((height, f), np.uint16)
    gpad[:rows], opad[:rows] = gh, oh
    v, sc = untiled(h_k, f)
    along = attribute_codes(v, sc, want_k.values, want_k.scales, gpad, opad)
    v, sc = untiled(h_m, height)
    across = attribute_codes(v, sc, want_m.values, want_m.scales, gpad.T, opad.T)
    print(f"[fused] case {case} product {err:.2e} h codes {along} h^T codes {across}", flush=True)
    assert err <= 1e-3
    for c in (along, across):
        assert c["codes"] <= 0.02 * c["of"], c


# --- the activation's gradient in the down dgrad's epilogue ---------------------------


def _run_dgrad(sizes_np, rows, d, f, act, seed):
    """The down dgrad then the activation's quantizing backward, and the fused kernel
    (`grouped_mxfp8.activation_grad`, the reference's grouped_cudnn.activation_grad,
    grouped_cudnn.py:211-263), on the same GPU operands: dy (rows, d) with outliers and
    rows past the groups holding garbage, W_down (g, f, d), the product (rows, 2f) and
    the rows' weights."""
    from bux_amd import grouped_mxfp8 as gm, moe
    torch.manual_seed(seed)
    dev = torch.device("cuda")
    groups = len(sizes_np)
    height = gm.whole(rows)
    filled = int(sizes_np.sum())
    dy = (torch.randn(rows, d, device=dev) * 0.01).to(torch.bfloat16)
    dy.view(-1)[torch.randint(0, dy.numel(), (max(1, dy.numel() // 500),), device=dev)] *= 100
    dy[filled:] = float("nan")  # rows past the groups: never read as values
    w_down = (torch.randn(groups, f, d, device=dev) * 0.05).to(torch.bfloat16)
    projected = (torch.randn(rows, 2 * f, device=dev) * 2.0).to(torch.bfloat16)
    weights = torch.rand(rows, device=dev).to(torch.bfloat16)
    sizes = torch.tensor(sizes_np, dtype=torch.int32, device=dev)
    filled_t = torch.tensor([filled], dtype=torch.int32, device=dev)
    dy_n, _ = gm.quantized_twice(dy, filled_t, False, height=height)
    down_n, _ = gm.quantized_twice(w_down)
    ffn = moe.Ffn(*ACTS[act])
    dh = gm.rows(dy_n, down_n, sizes, height=rows)
    unfused = moe.weighted_units_backward_quantized(ffn, projected.view(rows, f, 2), weights, dh,
                                                    filled_t, height, keep=True)
    fused = gm.activation_grad(dy_n, down_n, sizes, projected, weights, ffn.struct(True), rows,
                               keep=True)
    torch.cuda.synchronize()
    return unfused, fused, (dy, w_down, projected, weights, dh)


def _same_dgrad(unfused, fused):
    (dk, dm, dw, dp), (dk2, dm2, dw2, dp2) = unfused, fused
    _same("dp values", dk.values, dk2.values)
    _same("dp scales", dk.scales, dk2.scales)
    _same("dp^T values", dm.values, dm2.values)
    _same("dp^T scales", dm.scales, dm2.scales)
    _same("d weights", dw, dw2)
    _same("dp", dp.reshape(dp2.shape), dp2)


@pytest.mark.parametrize("case", range(len(CASES)))
def test_fused_dgrad_is_the_unfused_pair_bit_for_bit(lib, case):
    spec, rows, d, f, act = CASES[case]
    rng = np.random.default_rng(90 + case)
    sizes = _sizes(spec, rows, 64, rng)
    announce("dglu fused", case, f"groups={len(sizes)} rows={rows} d={d} f={f} {act}")
    unfused, fused, _ = _run_dgrad(sizes, rows, d, f, act, 90 + case)
    _same_dgrad(unfused, fused)


def test_fused_dgrad_at_config_3(lib):
    """Qwen3-30B-A3B's experts: 131072 rows, 128 experts, d 2048, f 768."""
    rng = np.random.default_rng(97)
    rows = 16384 * 8
    sizes = rng.multinomial(rows, np.ones(128) / 128).astype(np.int32)
    announce("dglu fused", "config 3")
    unfused, fused, _ = _run_dgrad(sizes, rows, 2048, 768, "swiglu", 97)
    _same_dgrad(unfused, fused)


@pytest.mark.parametrize("case", [0, 1, 4])
def test_fused_dgrad_against_the_oracle(lib, case):
    """The fused kernel's outputs against the oracle run from the same bits (dy and
    W_down quantized by the oracle's quantizer, which the GPU's matches bit for bit):
    dh (not stored by the kernel; the unfused GEMM's, bit for bit the epilogue's) within
    the north star's bar of the oracle's GEMM; from it, d projected within a bfloat16
    rounding of the oracle's float64 gradient (below 2^-20 of the largest magnitude,
    float32 cancellation where a derivative crosses 0) and the weights' gradient within
    1e-3; d projected's two MXFP8 copies the oracle quantizer's of the kernel's d
    projected, code for code."""
    from bux_amd import grouped_mxfp8 as gm
    from oracle import bf16, moe as omoe, mxfp8 as omx
    from tests._util import bf16_bits, rel_err, untiled
    spec, rows, d, f, act = CASES[case]
    rng = np.random.default_rng(100 + case)
    sizes_np = _sizes(spec, rows, 64, rng)
    announce("dglu fused vs oracle", case)
    _, (dk, dm, dw, dp), (dy, w_down, projected, weights, dh) = _run_dgrad(
        sizes_np, rows, d, f, act, 100 + case)
    height, filled = gm.whole(rows), int(sizes_np.sum())
    ody_n, _ = omx.quantized_twice(bf16_bits(dy), filled, False, height=height)
    odown_n, _ = omx.quantized_twice(bf16_bits(w_down), f)
    odh = omoe.rows_mx(ody_n, odown_n, sizes_np, height=rows)
    gdh = bf16_bits(dh)
    dh_err = rel_err(bf16.to_f32(gdh), bf16.to_f32(odh))
    o = omoe.Ffn(*ACTS[act])
    pb, rw = bf16_bits(projected), bf16_bits(weights)
    want_dp, want_dw = omoe.weighted_units_backward(o, pb[:filled].reshape(filled, f, 2),
                                                    rw[:filled], gdh[:filled])
    gdp = bf16_bits(dp)
    got, want = bf16.to_f32(gdp[:filled]), bf16.to_f32(want_dp.reshape(filled, 2 * f))
    floor = 2.0 ** -20 * float(np.abs(want).max())
    bad = np.abs(got - want) > np.abs(want) * 2.0 ** -7 + floor
    dp_err = rel_err(got, want)
    dw_err = rel_err(bf16.to_f32(bf16_bits(dw))[:filled], bf16.to_f32(want_dw))
    print(f"[dglu] case {case} dh {dh_err:.2e} dp {dp_err:.2e} (outside a rounding "
          f"{int(bad.sum())}) d weights {dw_err:.2e}", flush=True)
    assert dh_err <= 1e-3
    assert not bad.any() and dp_err <= 2.0 ** -9
    assert dw_err <= 1e-3
    assert (gdp[filled:] == 0).all() and (bf16_bits(dw)[filled:] == 0).all()
    want_k, want_m = omx.quantized_twice(gdp, filled, True, height=height)
    for tiled, w, cols in ((dk, want_k, 2 * f), (dm, want_m, height)):
        v, sc = untiled(tiled, cols)
        np.testing.assert_array_equal(v, w.values)
        np.testing.assert_array_equal(sc, w.scales)
