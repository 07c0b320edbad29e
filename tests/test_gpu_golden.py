"""The HIP kernels on the golden fixtures' inputs (tests/golden/*.npz, written by the
CPU oracle) against the stored outputs, with no oracle call: sort by expert, both
MXFP8 copies (direct and by index), token sums bit for bit; the grouped GEMMs within
the block-scaled MFMA's measured bars (tests/test_gpu_gemm.py); the activation and
its gradient within one bfloat16 ulp of the oracle's once-rounded float64 value."""

import numpy as np
import pytest
import torch

from oracle import bf16
from tests._util import announce, bf16_bits, rel_err, to_gpu, to_gpu_bf16, to_gpu_tiled, untiled
from tests.golden import make_fixtures as fx
from tests.test_gpu_gemm import _close_f32

pytestmark = pytest.mark.gpu


def test_permute_fixture(lib):
    from bux_amd import moe
    f = fx.load("permute")
    announce("golden permute")
    s = moe.sort_by_expert(to_gpu(f["idx"]), 5)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(s.order.cpu().numpy(), f["order"])
    np.testing.assert_array_equal(s.inverse.cpu().numpy(), f["inverse"])
    np.testing.assert_array_equal(s.sizes.cpu().numpy(), f["sizes"])
    offsets = s.offsets.cpu().numpy()
    np.testing.assert_array_equal(offsets[:5], f["offsets"])
    assert offsets[5] == f["sizes"].sum()


def test_quantize_fixture(lib):
    from bux_amd import grouped_mxfp8
    f = fx.load("quantize")
    announce("golden quantize")
    rows, cols = grouped_mxfp8.quantized_twice(to_gpu_bf16(f["x"]))
    k = int(f["k"])
    g_rows, g_cols = grouped_mxfp8.quantized_twice(
        to_gpu_bf16(f["z"]), to_gpu(np.array([f["filled"]], np.int32)), True, to_gpu(f["order"]),
        k, int(f["height"]))
    torch.cuda.synchronize()
    for got, name, cols_n in ((rows, "rows", 160), (cols, "cols", 96), (g_rows, "g_rows", 64),
                              (g_cols, "g_cols", int(f["height"]))):
        v, s = untiled(got, cols_n)
        np.testing.assert_array_equal(v, f[f"{name}_values"], err_msg=name)
        np.testing.assert_array_equal(s, f[f"{name}_scales"], err_msg=name)


def test_gemm_fixture(lib):
    from bux_amd import grouped_mxfp8
    from oracle.mxfp8 import Blocks
    f = fx.load("gemm")
    announce("golden gemm")
    sizes = to_gpu(f["sizes"])
    a = to_gpu_tiled(Blocks(f["a_values"], f["a_scales"]))
    b = to_gpu_tiled(Blocks(f["b_values"], f["b_scales"]))
    y32 = grouped_mxfp8.rows(a, b, sizes, torch.float32, height=256)
    y16 = grouped_mxfp8.rows(a, b, sizes, torch.bfloat16, height=256)
    ca = to_gpu_tiled(Blocks(f["ca_values"], f["ca_scales"]))
    cb = to_gpu_tiled(Blocks(f["cb_values"], f["cb_scales"]))
    dw32 = grouped_mxfp8.contract(ca, cb, sizes, torch.float32)
    torch.cuda.synchronize()
    filled = int(f["sizes"].sum())
    got = y32.cpu().numpy()
    _close_f32(got[:filled], f["y"][:filled], "golden rows")
    assert (got[filled:] == 0).all()
    got16 = bf16.to_f32(bf16_bits(y16))
    assert rel_err(got16, bf16.round_f32(f["y"])) <= 1e-3
    dw = dw32.cpu().numpy()
    for g in range(len(f["sizes"])):
        if f["sizes"][g] == 0:
            assert (dw[g] == 0).all()
        else:
            _close_f32(dw[g], f["dw"][g], f"golden contract group {g}")


def _ulps(got_bits: np.ndarray, want_bits: np.ndarray) -> int:
    """The largest distance in bfloat16 steps (ordered bit patterns) between two arrays."""
    def ordered(b):
        b = b.astype(np.int32)
        return np.where(b & 0x8000, 0x8000 - (b & 0x7FFF), 0x8000 + b)
    return int(np.abs(ordered(got_bits) - ordered(want_bits)).max())


@pytest.mark.parametrize("name", sorted(fx.ACTIVATIONS))
def test_activation_fixture(lib, name):
    from bux_amd import moe
    f = fx.load("activation")
    act, limit, offset = fx.ACTIVATIONS[name]
    ffn = moe.Ffn(act, limit, offset)
    announce("golden activation", name)
    p, w, dh = to_gpu_bf16(f["projected"]), to_gpu_bf16(f["weights"]), to_gpu_bf16(f["dh"])
    h = moe.weighted_units(ffn, p, w)
    dp, dw = moe.weighted_units_backward(ffn, p, w, dh)
    torch.cuda.synchronize()
    assert _ulps(bf16_bits(h), f[f"{name}_h"]) <= 1
    assert _ulps(bf16_bits(dp), f[f"{name}_dp"]) <= 1
    assert _ulps(bf16_bits(dw), f[f"{name}_dw"]) <= 1


def test_token_sums_fixture(lib):
    from bux_amd import moe
    f = fx.load("token_sums")
    announce("golden token sums")
    out = moe.sum_by_token(to_gpu_bf16(f["y"]), to_gpu(f["inverse"]))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bf16_bits(out), f["out"])
