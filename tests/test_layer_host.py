"""The layer's host-side argument checks, without a GPU: the passes it takes, and
kernels given already in MXFP8 only for the recipe and shapes they were made for."""

import pytest
import torch

from bux_amd import moe


def test_passes_are_a_subset_of_fprop_dgrad_wgrad():
    assert moe.passes_of("mxfp8") == (True, True, True)
    assert moe.passes_of("mxfp8_2d", ("wgrad",)) == (False, False, True)
    assert moe.passes_of("mxfp8", ()) == (False, False, False)
    assert moe.passes_of("compute", ("fprop",)) == (False, False, False)
    with pytest.raises(ValueError, match="bprop"):
        moe.passes_of("mxfp8", ("fprop", "bprop"))
    with pytest.raises(ValueError, match="fp4"):
        moe.passes_of("fp4")


def test_kernels_in_mxfp8_are_checked_against_the_recipe_and_the_kernels():
    up = torch.empty(4, 64, 32, 2, dtype=torch.bfloat16)
    down = torch.empty(4, 32, 64, dtype=torch.bfloat16)
    given = moe.MxWeights(None, None, None, None, "mxfp8", tuple(up.shape), tuple(down.shape))
    given.check("mxfp8", up, down)
    with pytest.raises(ValueError, match="'mxfp8' recipe, not 'mxfp8_2d'"):
        given.check("mxfp8_2d", up, down)
    with pytest.raises(ValueError, match="multiply in 'compute'"):
        given.check("compute", up, down)
    with pytest.raises(ValueError, match="quantized from"):
        given.check("mxfp8", torch.empty(4, 64, 48, 2), down)
    # the layer checks before it runs anything
    with pytest.raises(ValueError, match="recipe"):
        moe.experts_forward(torch.empty(8, 64, dtype=torch.bfloat16),
                            torch.zeros(8, 2, dtype=torch.int32),
                            torch.empty(8, 2, dtype=torch.bfloat16), up, down, fmt="mxfp8_2d",
                            quantized=given)


def test_the_layer_takes_bfloat16_or_float32_tokens():
    """y, dx and dW take x's dtype, the kernels cast to it (moe.py:846,
    grouped_blockscaled.py:129): bfloat16 or float32 tokens, others refused before any
    launch."""
    idx = torch.zeros(8, 2, dtype=torch.int32)
    up, down = torch.empty(4, 64, 32, 2), torch.empty(4, 32, 64)
    w = torch.empty(8, 2)
    with pytest.raises(TypeError, match="bfloat16 or float32, not torch.float16"):
        moe.experts_forward(torch.empty(8, 64, dtype=torch.float16), idx, w, up, down)


def test_the_bias_and_norm_ops_take_one_dtype():
    """Each bias and norm op runs in its rows' dtype, bfloat16 or float32, and refuses a
    tensor of another dtype beside them before any launch."""
    x = torch.empty(8, 16)
    assert moe._runs_f32("add_expert_bias", x, torch.empty(2, 16))
    assert not moe._runs_f32("add_expert_bias", x.bfloat16(), torch.empty(2, 16).bfloat16(), None)
    with pytest.raises(TypeError, match="torch.bfloat16 tensor beside torch.float32 rows"):
        moe._runs_f32("expert_norm_forward", x, torch.empty(16).bfloat16())
    with pytest.raises(TypeError, match="bfloat16 or float32 rows, not torch.float16"):
        moe._runs_f32("expert_sums", x.half())


def test_an_ffn_names_one_of_the_ten_activations():
    assert moe.Ffn("situ", None, 0.0, 4.0).struct(True).capped == 1
    st = moe.Ffn("relu2", 0.0).struct(False)
    assert (st.activation, st.gated, st.clamped, st.limit) == (3, 0, 1, 0.0)
    assert moe.Ffn().fusable(True) and not moe.Ffn().fusable(False)
    assert not moe.Ffn("gelu").fusable(True)
    with pytest.raises(ValueError, match="no activation 'silu'"):
        moe.Ffn("silu").struct()
