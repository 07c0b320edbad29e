"""The experts' activation, and the whole routed-experts layer forward and backward,
on the GPU against the oracle.

The activation computes in float32 and rounds once; the oracle computes in float64
and rounds once: the two agree to a bfloat16 rounding (XLA's own rounding inside the
fused chain is not observable without jax: parity at bit level is unpinned). In the
layer, every GEMM meets the north star's bar, ||y - y_ref|| / ||y_ref|| <= 1e-3, on the
GPU's own inputs to it, and the quantizer is bit-exact on the GPU's own activations;
end to end, see END_TO_END and the attribution test."""

import numpy as np
import pytest
import torch

from oracle import bf16, moe as omoe
from tests._util import (announce, attribute_codes, bf16_bits, normal_bf16, rel_err, to_gpu,
                         to_gpu_bf16, ulps_apart, untiled)

pytestmark = pytest.mark.gpu

FFNS = {"swiglu": (omoe.Ffn(), None), "clamped": (omoe.Ffn("quick_gelu", 7.0, 1.0), None)}


def _ffn(name):
    from bux_amd import moe
    o = FFNS[name][0]
    return o, moe.Ffn(o.activation, o.limit, o.up_offset)


@pytest.mark.parametrize("name", list(FFNS))
def test_weighted_units_and_gradients(lib, name):
    from bux_amd import moe
    o, g = _ffn(name)
    rng = np.random.default_rng(40)
    m, f, filled = 1000, 768, 937
    p = normal_bf16(rng, (m, f, 2), 4.0)
    p.reshape(-1)[:64] = bf16.to_bf16(np.array([7.0, -7.0, 6.99, 7.01] * 16, np.float32))
    w = bf16.to_bf16(rng.random(m).astype(np.float32))
    dh = normal_bf16(rng, (m, f))
    announce("glu", name)
    fg = to_gpu(np.array([filled], np.int32))
    h = moe.weighted_units(g, to_gpu_bf16(p), to_gpu_bf16(w), fg)
    dp, dw = moe.weighted_units_backward(g, to_gpu_bf16(p), to_gpu_bf16(w), to_gpu_bf16(dh), fg)
    torch.cuda.synchronize()
    want_h = bf16.to_f32(omoe.weighted_units(o, p[:filled], w[:filled]))
    want_dp, want_dw = omoe.weighted_units_backward(o, p[:filled], w[:filled], dh[:filled])
    got_h = bf16.to_f32(bf16_bits(h))
    # one bfloat16 rounding apart at most
    ulp = np.abs(want_h) * 2.0 ** -7 + 1e-30
    assert (np.abs(got_h[:filled] - want_h) <= ulp).all()
    assert (got_h[filled:] == 0).all()
    got_dp = bf16.to_f32(bf16_bits(dp))
    wdp = bf16.to_f32(want_dp)
    assert (np.abs(got_dp[:filled] - wdp) <= np.abs(wdp) * 2.0 ** -7 + 1e-30).all()
    assert (got_dp[filled:] == 0).all()
    got_dw = bf16.to_f32(bf16_bits(dw))
    assert rel_err(got_dw[:filled], bf16.to_f32(want_dw)) <= 1e-3
    assert (got_dw[filled:] == 0).all()


@pytest.mark.parametrize("name", list(FFNS))
def test_activation_quantized_in_one_pass(lib, name):
    """The fused kernels (activation, then both MXFP8 copies, no bfloat16 round trip)
    against the separate ones: the same bfloat16 h and d projected bit for bit, their
    copies bit for bit what the oracle's quantizer makes of those values (rows from
    `filled` on as 0, padding to whole tiles), d weights within a bfloat16 step."""
    from bux_amd import moe
    from oracle import mxfp8 as omx
    o, g = _ffn(name)
    rng = np.random.default_rng(42)
    m, f, filled = 1000, 768, 937
    height = 1024
    p = normal_bf16(rng, (m, f, 2), 4.0)
    p.reshape(-1)[:64] = bf16.to_bf16(np.array([7.0, -7.0, 6.99, 7.01] * 16, np.float32))
    w = bf16.to_bf16(rng.random(m).astype(np.float32))
    dh = normal_bf16(rng, (m, f))
    announce("glu quantized", name)
    fg = to_gpu(np.array([filled], np.int32))
    gp, gw, gdh = to_gpu_bf16(p), to_gpu_bf16(w), to_gpu_bf16(dh)
    h_sep = moe.weighted_units(g, gp, gw, fg)
    dp_sep, dw_sep = moe.weighted_units_backward(g, gp, gw, gdh, fg)
    h_k, h_m, h = moe.weighted_units_quantized(g, gp, gw, fg, height, keep=True)
    dp_n, dp_m, dw, dp = moe.weighted_units_backward_quantized(g, gp, gw, gdh, fg, height, keep=True)
    _, _, none = moe.weighted_units_quantized(g, gp, gw, fg, height)
    torch.cuda.synchronize()
    assert none is None
    np.testing.assert_array_equal(bf16_bits(h), bf16_bits(h_sep))
    np.testing.assert_array_equal(bf16_bits(dp), bf16_bits(dp_sep))
    want_k, want_m = omx.quantized_twice(bf16_bits(h), filled, True, height=height)
    for got, want, cols in ((h_k, want_k, f), (h_m, want_m, height)):
        v, sc = untiled(got, cols)
        np.testing.assert_array_equal(v, want.values)
        np.testing.assert_array_equal(sc, want.scales)
    want_n, want_pm = omx.quantized_twice(bf16_bits(dp).reshape(m, 2 * f), filled, True,
                                          height=height)
    for got, want, cols in ((dp_n, want_n, 2 * f), (dp_m, want_pm, height)):
        v, sc = untiled(got, cols)
        np.testing.assert_array_equal(v, want.values)
        np.testing.assert_array_equal(sc, want.scales)
    a, b = bf16.to_f32(bf16_bits(dw)), bf16.to_f32(bf16_bits(dw_sep))
    assert (np.abs(a - b) <= np.abs(b) * 2.0 ** -7 + 1e-30).all()
    assert (a[filled:] == 0).all()


def _inputs(rng, t, k, e, d, f, skew=None):
    z = normal_bf16(rng, (t, d))
    if skew is None:
        idx = np.stack([rng.choice(e, k, replace=False) for _ in range(t)]).astype(np.int32)
    else:
        idx = np.stack([rng.choice(e, k, replace=False, p=skew) for _ in range(t)]).astype(np.int32)
    w = bf16.to_bf16(rng.random((t, k)).astype(np.float32) / k)
    up = normal_bf16(rng, (e, d, f, 2), 0.02)
    down = normal_bf16(rng, (e, f, d), 0.02)
    dy = normal_bf16(rng, (t, d), 1e-2)
    return z, idx, w, up, down, dy


LAYERS = [
    # name, t, k, e, d, f, ffn, fmt
    ("config1_compute", 4096, 2, 8, 256, 512, "swiglu", "compute"),
    ("small_mxfp8", 1024, 4, 16, 256, 256, "swiglu", "mxfp8"),
    ("gptoss_like_mxfp8", 256, 4, 8, 1440, 1440, "clamped", "mxfp8"),
    ("empty_experts_mxfp8", 700, 2, 12, 128, 192, "swiglu", "mxfp8"),
    ("small_mxfp8_2d", 1024, 4, 16, 256, 256, "swiglu", "mxfp8_2d"),
]

# End to end, two float implementations of a quantized pipeline differ by more than
# their GEMMs do: a GEMM's float32 sum that differs in its last bits (the block-scaled
# MFMA does not add in IEEE float32 order) flips, now and then, the bfloat16 rounding of
# an activation, and that flips its E4M3 code downstream, a step of 1/16.
# test_the_layers_drift_from_the_oracle_is_attributed checks that chain link by link
# and measures 1.1e-3 to 2.3e-3 end to end; the stage-wise checks below hold each GEMM
# to the 1e-3 bar on identical inputs.
END_TO_END = 3e-3
STAGE = 1e-3
# The attribution test's bounds, from its measured values with margin: the share of
# elements that differ (measured 1.1-1.2% for the GEMM outputs, 1.2-2.1% for h and dp),
# a GEMM output by at most a bfloat16 step of itself or FLOOR of the array's largest
# magnitude (near 0 a float32 sum's last bits flip signs and bfloat16 steps are tiny);
# the share of E4M3 codes that differ (measured 0.15-0.18%); and the end-to-end error
# those leave (measured 1.1e-3 to 2.3e-3).
SHARE_APART = {"projected": 0.02, "h": 0.03, "dh": 0.02, "dp": 0.03}
FLOOR = 2.0 ** -12
CODE_SHARE = 0.005
END_TO_END_ATTRIBUTED = 3e-3


def _f32(t):
    return bf16.to_f32(bf16_bits(t)).astype(np.float64)


def _stage(name, got, want, bar=STAGE):
    err = rel_err(got, want)
    print(f"[err] {name} {err:.3e}", flush=True)
    assert err <= bar, (name, err)


@pytest.mark.parametrize("name,t,k,e,d,f,act,fmt", LAYERS)
def test_layer_forward_and_backward(lib, name, t, k, e, d, f, act, fmt):
    from bux_amd import moe
    from oracle import mxfp8 as omx
    o, g = _ffn(act)
    rng = np.random.default_rng(41)
    skew = None
    if name.startswith("empty"):
        skew = np.where(np.arange(e) % 3 == 0, 0.0, 1.0)
        skew /= skew.sum()
    z, idx, w, up, down, dy = _inputs(rng, t, k, e, d, f, skew)
    announce("layer", name)
    gz, gidx, gw, gup, gdown, gdy = (to_gpu_bf16(z), to_gpu(idx), to_gpu_bf16(w), to_gpu_bf16(up),
                                      to_gpu_bf16(down), to_gpu_bf16(dy))
    out, saved = moe.experts_forward(gz, gidx, gw, gup, gdown, g, fmt, intermediates=True)
    grads = moe.experts_backward(saved, gdy, gup, gdown, g, fmt, intermediates=True)
    torch.cuda.synchronize()

    # End to end against the oracle run on its own.
    want, osaved = omoe.layer_forward(z, idx, w, up, down, o, fmt)
    wgrads = omoe.layer_backward(osaved, dy, z, up, down, k, o, fmt)
    bar = STAGE if fmt == "compute" else END_TO_END
    _stage(f"{name} end-to-end y", _f32(out), bf16.to_f32(want), bar)
    for key in ("z", "weights", "up", "down"):
        _stage(f"{name} end-to-end d{key}", _f32(grads[key]), bf16.to_f32(wgrads[key]), bar)
    if fmt != "mxfp8":
        return

    # Stage by stage: the oracle takes the GPU's own input to each stage.
    s = osaved.sorted
    m, filled = t * k, int(s.sizes.sum())
    hp = -(-m // 128) * 128  # the copies' rows: whole tiles of 128, as the GPU's
    np.testing.assert_array_equal(saved.sorted.order.cpu().numpy(), s.order)
    tokens = s.order // k
    up2 = up.reshape(e, d, 2 * f)
    x_k, x_m = omx.quantized_twice(z, filled, True, index=tokens, height=hp)
    up_n, up_k = omx.quantized_twice(up2, d)
    _stage(f"{name} up fprop", _f32(saved.projected), bf16.to_f32(omoe.rows_mx(x_k, up_k, s.sizes, height=m)))
    h_want = omoe.weighted_units(o, bf16_bits(saved.projected).reshape(m, f, 2), osaved.row_weights)
    _stage(f"{name} activation", _f32(saved.h), bf16.to_f32(h_want), 2.0 ** -8)
    # the quantizer, bit for bit, on the GPU's own h (the x^T copy the down wgrad takes)
    h_k, h_m = omx.quantized_twice(bf16_bits(saved.h), filled, True, height=hp)
    got_v, got_s = untiled(saved.h_m, hp)
    np.testing.assert_array_equal(got_v, h_m.values)
    np.testing.assert_array_equal(got_s, h_m.scales)
    down_n, down_k = omx.quantized_twice(down, f)
    y_rows = omoe.rows_mx(h_k, down_k, s.sizes, height=m)
    _stage(f"{name} down fprop + combine", _f32(out),
           bf16.to_f32(omoe.sum_by_token(y_rows, s.inverse.reshape(t, k))))
    dy_n, dy_m = omx.quantized_twice(dy, filled, True, index=tokens, height=hp)
    _stage(f"{name} down dgrad", _f32(grads["dh"]), bf16.to_f32(omoe.rows_mx(dy_n, down_n, s.sizes, height=m)))
    _stage(f"{name} down wgrad", _f32(grads["down"]), bf16.to_f32(omoe.contract_mx(h_m, dy_m, s.sizes)))
    dp_want, drw_want = omoe.weighted_units_backward(
        o, bf16_bits(saved.projected).reshape(m, f, 2), osaved.row_weights, bf16_bits(grads["dh"]))
    _stage(f"{name} activation backward", _f32(grads["dp"]), bf16.to_f32(dp_want).reshape(m, 2 * f), 2.0 ** -8)
    _stage(f"{name} d row weights", _f32(grads["d_row_weights"]), bf16.to_f32(drw_want))
    dp_n, dp_m = omx.quantized_twice(bf16_bits(grads["dp"]), filled, True, height=hp)
    dx_rows = omoe.rows_mx(dp_n, up_n, s.sizes, height=m)
    _stage(f"{name} up dgrad", _f32(grads["dx"]), bf16.to_f32(dx_rows))
    _stage(f"{name} up dgrad + combine", _f32(grads["z"]),
           bf16.to_f32(omoe.sum_by_token(bf16_bits(grads["dx"]), s.inverse.reshape(t, k))))
    _stage(f"{name} up wgrad", _f32(grads["up"]).reshape(e, d, 2 * f),
           bf16.to_f32(omoe.contract_mx(x_m, dp_m, s.sizes)))
    d_weights = bf16_bits(grads["d_row_weights"])[s.inverse].reshape(t, k)
    np.testing.assert_array_equal(bf16_bits(grads["weights"]), d_weights)


@pytest.mark.parametrize("fmt", ["mxfp8", "mxfp8_2d"])
def test_the_layer_quantizes_its_weights_by_its_recipe(lib, fmt):
    """The weights' copies the layer keeps for its backward are exactly its recipe's:
    1x32 blocks (mxfp8) or one scale per 32 x 32 tile (mxfp8_2d), bit for bit the
    quantizer's, and the same as `in_mxfp8` gives to callers that quantize once."""
    from bux_amd import grouped_mxfp8, moe
    rng = np.random.default_rng(43)
    z, idx, w, up, down, dy = _inputs(rng, 256, 4, 8, 256, 256, None)
    gz, gidx, gw, gup, gdown = (to_gpu_bf16(z), to_gpu(idx), to_gpu_bf16(w), to_gpu_bf16(up),
                                to_gpu_bf16(down))
    announce("layer weights", fmt)
    _, saved = moe.experts_forward(gz, gidx, gw, gup, gdown, fmt=fmt)
    e, d, f, p = up.shape
    tiles = fmt == "mxfp8_2d"
    want_up, _ = grouped_mxfp8.quantized_twice(gup.reshape(e, d, f * p), tiles=tiles)
    want_down, _ = grouped_mxfp8.quantized_twice(gdown, tiles=tiles)
    given = moe.in_mxfp8(gup, gdown, fmt)
    torch.cuda.synchronize()
    for got, want in ((saved.up_n, want_up), (saved.down_n, want_down),
                      (given.up_n, want_up), (given.down_n, want_down)):
        assert torch.equal(got.values, want.values) and torch.equal(got.scales, want.scales)
    # the two recipes differ: a 1x32 copy is not the tile-scaled one
    other, _ = grouped_mxfp8.quantized_twice(gup.reshape(e, d, f * p), tiles=not tiles)
    assert not torch.equal(saved.up_n.scales, other.scales)


def test_a_layer_given_its_weights_in_mxfp8_is_the_same_layer(lib):
    """experts_forward(quantized=in_mxfp8(up, down)) (the reference's `quantized`,
    moe.py:799) gives the bits of the layer that quantizes them itself."""
    from bux_amd import moe
    rng = np.random.default_rng(44)
    z, idx, w, up, down, dy = _inputs(rng, 300, 4, 8, 256, 192, None)
    args = (to_gpu_bf16(z), to_gpu(idx), to_gpu_bf16(w), to_gpu_bf16(up), to_gpu_bf16(down))
    announce("layer given weights")
    out0, saved0 = moe.experts_forward(*args)
    g0 = moe.experts_backward(saved0, to_gpu_bf16(dy), args[3], args[4])
    out1, saved1 = moe.experts_forward(*args, quantized=moe.in_mxfp8(args[3], args[4]))
    g1 = moe.experts_backward(saved1, to_gpu_bf16(dy), args[3], args[4])
    torch.cuda.synchronize()
    assert torch.equal(out0.view(torch.int16), out1.view(torch.int16))
    for key in g0:
        assert torch.equal(g0[key].view(torch.int16), g1[key].view(torch.int16)), key


@pytest.mark.parametrize("fmt", ["mxfp8", "compute"])
def test_a_layer_with_no_pick_inside_the_experts_is_zero(lib, fmt):
    """Every pick outside [0, E) (the reference sorts those last and counts them for no
    expert, moe.py:776-797): no group holds a row, every GEMM output is 0, and so are y
    and every gradient."""
    from bux_amd import moe
    rng = np.random.default_rng(45)
    t, k, e, d, f = 64, 2, 4, 128, 64
    z, idx, w, up, down, dy = _inputs(rng, t, k, e, d, f, None)
    idx[:] = e + 3
    announce("layer no picks", fmt)
    out, saved = moe.experts_forward(to_gpu_bf16(z), to_gpu(idx), to_gpu_bf16(w), to_gpu_bf16(up),
                                     to_gpu_bf16(down), fmt=fmt)
    grads = moe.experts_backward(saved, to_gpu_bf16(dy), to_gpu_bf16(up), to_gpu_bf16(down),
                                 fmt=fmt)
    torch.cuda.synchronize()
    assert int(saved.sorted.sizes.sum()) == 0
    assert (out.float() == 0).all()
    for key, g in grads.items():
        assert (g.float() == 0).all(), key


def test_a_layer_of_one_token(lib):
    """One token, its k picks in k groups of one row each: against the oracle, end to
    end."""
    from bux_amd import moe
    o, g = _ffn("swiglu")
    rng = np.random.default_rng(46)
    t, k, e, d, f = 1, 4, 8, 128, 64
    z, idx, w, up, down, dy = _inputs(rng, t, k, e, d, f, None)
    announce("layer one token")
    out, saved = moe.experts_forward(to_gpu_bf16(z), to_gpu(idx), to_gpu_bf16(w), to_gpu_bf16(up),
                                     to_gpu_bf16(down), g)
    grads = moe.experts_backward(saved, to_gpu_bf16(dy), to_gpu_bf16(up), to_gpu_bf16(down), g)
    torch.cuda.synchronize()
    want, osaved = omoe.layer_forward(z, idx, w, up, down, o, "mxfp8")
    wgrads = omoe.layer_backward(osaved, dy, z, up, down, k, o, "mxfp8")
    _stage("one token y", _f32(out), bf16.to_f32(want), END_TO_END)
    for key in ("z", "weights", "up", "down"):
        _stage(f"one token d{key}", _f32(grads[key]), bf16.to_f32(wgrads[key]), END_TO_END)


@pytest.mark.parametrize("name,t,k,e,d,f,act", [
    ("small", 1024, 4, 16, 256, 256, "swiglu"), ("gptoss_like", 256, 4, 8, 1440, 1440, "clamped"),
    ("config3_slice", 2048, 8, 16, 2048, 768, "swiglu")])
def test_the_layers_drift_from_the_oracle_is_attributed(lib, name, t, k, e, d, f, act):
    """The GPU layer and the oracle's, each run on its own, drift apart end to end by
    more than one GEMM does: a float32 sum that differs in its last bits flips the
    bfloat16 rounding of a product, that moves an activation by a bfloat16 step, that
    moves its E4M3 code by one, a step of 1/16 downstream. Here each link is checked: the
    GEMM outputs (projected, dh) differ at a bounded share of elements, each by a
    rounding; the activation and its gradient (h, dp) by more than a rounding only where
    their unit's inputs differ; every E4M3 code or scale that differs (h^T's as the GPU
    wrote it, h's and dp's as the quantizer, bit-exact to the GPU's, makes them) sits at
    a value that differs, by no more codes than steps; and with those shares, y and every
    gradient
    stay within END_TO_END_ATTRIBUTED (3e-3, where a flat bar would need 1e-2 to hold
without this account of its cause)."""
    from bux_amd import moe
    from oracle import mxfp8 as omx
    o, g = _ffn(act)
    rng = np.random.default_rng(47)
    z, idx, w, up, down, dy = _inputs(rng, t, k, e, d, f, None)
    announce("layer attribution", name)
    gz, gidx, gw, gup, gdown, gdy = (to_gpu_bf16(z), to_gpu(idx), to_gpu_bf16(w), to_gpu_bf16(up),
                                      to_gpu_bf16(down), to_gpu_bf16(dy))
    out, saved = moe.experts_forward(gz, gidx, gw, gup, gdown, g, intermediates=True)
    grads = moe.experts_backward(saved, gdy, gup, gdown, g, intermediates=True)
    torch.cuda.synchronize()
    want, osaved = omoe.layer_forward(z, idx, w, up, down, o)
    wgrads = omoe.layer_backward(osaved, dy, z, up, down, k, o)
    m, filled = t * k, int(osaved.sorted.sizes.sum())
    hp = -(-m // 128) * 128
    p = up.shape[-1]

    def apart(got, ref, shape):
        return ulps_apart(got.reshape(shape)[:filled], ref.reshape(shape)[:filled])

    report = {}
    # the GEMM outputs: float32 sums in another order, rounded: a bfloat16 step apart
    # or, near 0 (signs flip, steps are tiny), FLOOR of the largest magnitude
    steps = {}
    for what, got, ref, shape in (("projected", bf16_bits(saved.projected), osaved.projected, (m, f, p)),
                                  ("dh", bf16_bits(grads["dh"]), wgrads["dh"], (m, f))):
        steps[what] = apart(got, ref, shape)
        a = bf16.to_f32(got.reshape(shape)[:filled]).astype(np.float64)
        b = bf16.to_f32(ref.reshape(shape)[:filled]).astype(np.float64)
        beyond = np.abs(a - b) > np.maximum(np.abs(b) * 2.0 ** -7, FLOOR * np.abs(b).max())
        report[what] = (float((steps[what] > 0).mean()), int(beyond.sum()))
    # the activation and its gradient, elementwise from their unit's inputs: more than a
    # rounding apart only where an input of the unit is apart (up or gate; for dp dh
    # too), with float32 cancellation allowed below 2^-20 of the largest |dp|
    unit = (steps["projected"] > 0).any(-1)
    for what, got, ref, shape, cause in (
            ("h", bf16_bits(saved.h), osaved.h, (m, f), unit),
            ("dp", bf16_bits(grads["dp"]), wgrads["dp"], (m, f, p),
             (unit | (steps["dh"] > 0))[..., None])):
        st = apart(got, ref, shape)
        a = bf16.to_f32(got.reshape(shape)[:filled]).astype(np.float64)
        b = bf16.to_f32(ref.reshape(shape)[:filled]).astype(np.float64)
        rounding = (st <= 1) | (np.abs(a - b) <= 2.0 ** -20 * np.abs(b).max())
        report[what] = (float((st > 0).mean()), int((~rounding & ~cause).sum()))
    # h^T's column copy as the GPU wrote it, against the oracle's
    hm_v, hm_s = untiled(saved.h_m, hp)
    _, want_hm = omx.quantized_twice(osaved.h, filled, True, height=hp)
    h_t = np.zeros((hp, f), np.uint16)
    h_t[:filled] = bf16_bits(saved.h)[:filled]
    oh_t = np.zeros((hp, f), np.uint16)
    oh_t[:filled] = osaved.h[:filled]
    codes = {"h^T": attribute_codes(hm_v, hm_s, want_hm.values, want_hm.scales, h_t.T, oh_t.T)}
    for what, got, ref in (("h", bf16_bits(saved.h), osaved.h),
                           ("dp", bf16_bits(grads["dp"]), wgrads["dp"].reshape(m, -1))):
        a, _ = omx.quantized_twice(got, filled, True, height=hp)
        b, _ = omx.quantized_twice(ref, filled, True, height=hp)
        gb = np.zeros((hp, got.shape[1]), np.uint16)
        gb[:filled] = got[:filled]
        rb = np.zeros((hp, got.shape[1]), np.uint16)
        rb[:filled] = ref[:filled]
        codes[what] = attribute_codes(a.values, a.scales, b.values, b.scales, gb, rb)
    errs = {"y": rel_err(_f32(out), bf16.to_f32(want))}
    for key in ("z", "weights", "up", "down"):
        errs[key] = rel_err(_f32(grads[key]), bf16.to_f32(wgrads[key]))
    print(f"[attribution] {name} steps {report} codes {codes} "
          + " ".join(f"{k_}={v:.2e}" for k_, v in errs.items()), flush=True)
    for what, (share, beyond) in report.items():
        assert share <= SHARE_APART[what] and beyond == 0, (what, share, beyond)
    for what, c in codes.items():
        assert c["codes"] <= CODE_SHARE * c["of"], (what, c)
    for key, err in errs.items():
        assert err <= END_TO_END_ATTRIBUTED, (key, err)


# The GPU layer's distance from the exact layer (oracle.moe with exact sums: float64,
# rounded once), against the two float implementations it is measured beside: the
# oracle's float32 order lands far inside 1e-3 of the exact layer, and the exact layer
# with each GEMM perturbed by noise of the size of the GPU GEMM's own error (measured
# here, float32 out on the same operands, against float64 sums: ~1.5e-5 relative, left
# inside each block-scaled MFMA instruction) lands where the GPU does. The 1e-3 bar of
# the north star holds for a GEMM on identical inputs and for an IEEE float32 order end
# to end; no layer built on this instruction can hold it end to end (tests/test_exact.py
# shows the same on the CPU).
@pytest.mark.parametrize("name,t,k,e,d,f,act", [
    ("small", 1024, 4, 16, 256, 256, "swiglu"), ("gptoss_like", 256, 4, 8, 1440, 1440, "clamped")])
def test_the_gpu_layers_drift_from_the_exact_layer_is_the_mfmas(lib, monkeypatch, name, t, k, e, d,
                                                               f, act):
    from bux_amd import grouped_mxfp8 as gm
    from bux_amd import moe
    from oracle import mxfp8 as omx
    from tests.test_exact import rel as rel_bits, run_layer, with_gemm_noise
    o, g = _ffn(act)
    rng = np.random.default_rng(47)
    z, idx, w, up, down, dy = _inputs(rng, t, k, e, d, f, None)
    announce("layer vs exact", name)
    gz, gidx, gw, gup, gdown, gdy = (to_gpu_bf16(z), to_gpu(idx), to_gpu_bf16(w), to_gpu_bf16(up),
                                      to_gpu_bf16(down), to_gpu_bf16(dy))
    out, saved = moe.experts_forward(gz, gidx, gw, gup, gdown, g)
    grads = moe.experts_backward(saved, gdy, gup, gdown, g)
    # the up GEMM's own error: float32 out on the layer's operands, against float64 sums
    m, hp = t * k, -(-(t * k) // 128) * 128
    x_k, _ = gm.quantized_twice(gz, saved.sorted.filled, False, saved.sorted.order, k, hp)
    _, up_k = gm.quantized_twice(gup.reshape(e, d, 2 * f))
    y32 = gm.rows(x_k, up_k, saved.sorted.sizes, torch.float32, height=m)
    torch.cuda.synchronize()
    gpu = {"y": bf16_bits(out), **{key: bf16_bits(grads[key]) for key in ("z", "weights", "up", "down")}}
    args = (z, idx, w, up, down, dy)
    exact = run_layer(*args, exact=True, ffn=o)
    f32 = run_layer(*args, exact=False, ffn=o)
    s = omoe.sort_by_expert(idx, e)
    filled = int(s.sizes.sum())
    ox_k, _ = omx.quantized_twice(z, filled, True, index=s.order // k, height=hp)
    _, oup_k = omx.quantized_twice(up.reshape(e, d, 2 * f), d)
    y64 = omoe.rows_mx(ox_k, oup_k, s.sizes, out="f64", height=m, exact=True)
    sigma = float(np.linalg.norm(y32.cpu().numpy().astype(np.float64) - y64) / np.linalg.norm(y64))
    with_gemm_noise(monkeypatch, sigma, seed=7)
    model = run_layer(*args, exact=True, ffn=o)
    monkeypatch.undo()
    errs = {key: (rel_bits(gpu[key], exact[key]), rel_bits(f32[key], exact[key]),
                  rel_bits(model[key], exact[key])) for key in exact}
    print(f"[exact] {name} gemm error {sigma:.2e}; vs exact (gpu, float32 order, exact + gemm-sized "
          "noise): " + " ".join(f"{key}=({a:.2e}, {b:.2e}, {c:.2e})" for key, (a, b, c) in errs.items()),
          flush=True)
    # measured on the MI355X: the GEMM's error 1.45e-5 at both shapes; the GPU layer
    # 1.1e-3 to 2.2e-3 from the exact one, the noise model 1.0e-3 to 2.2e-3 (the GPU at
    # most 1.14x the model), the float32 order at most 3.8e-4 (y at gptoss_like)
    assert sigma <= 5e-5
    for key, (a, b, c) in errs.items():
        assert b <= 5e-4, (key, b)
        assert a <= 1.5 * c, (key, a, c)
