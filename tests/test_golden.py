"""The golden fixtures (tests/golden/*.npz) against the oracle that wrote them, on the
CPU: every stored output is what the oracle gives for the stored input today (bit for
bit for integers, codes, scale bytes and bfloat16; float32 GEMM sums to float32's
rounding of a float64 sum), plus the invariants each fixture is meant to carry."""

import numpy as np
import pytest

from tests.golden import make_fixtures as fx


@pytest.mark.parametrize("name", sorted(fx.FIXTURES))
def test_the_oracle_reproduces_the_fixture(name):
    stored = fx.load(name)
    fresh = fx.FIXTURES[name]()
    assert set(stored) == set(fresh)
    for key in stored:
        want, got = stored[key], np.asarray(fresh[key])
        assert want.dtype == got.dtype and want.shape == got.shape, key
        if want.dtype.kind == "f":
            np.testing.assert_allclose(got, want, rtol=1e-6, atol=1e-30, err_msg=key)
        else:
            np.testing.assert_array_equal(got, want, err_msg=key)


def test_the_fixtures_reach_the_edge_cases():
    p = fx.load("permute")
    assert (p["sizes"] == 0).any() and ((p["idx"] < 0) | (p["idx"] >= 5)).sum() == 2
    assert p["sizes"].sum() == p["idx"].size - 2
    q = fx.load("quantize")
    assert (q["rows_scales"][:32, 0] == 1).all()  # the block of zeros
    assert (q["g_rows_values"][90:] == 0).all() and (q["g_rows_scales"][90:] == 1).all()
    assert (q["order"] < 0).sum() == 3
    g = fx.load("gemm")
    assert g["a_values"].shape[1] % 128 != 0  # K not a whole tile
    assert (g["y"][g["sizes"].sum():] == 0).all() and (g["dw"][1] == 0).all()
    t = fx.load("token_sums")
    assert (t["inverse"] >= t["y"].shape[0]).any()
