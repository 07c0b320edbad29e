"""MXFP8 rows of bytes (an expert-parallel dispatch's payload) against the oracle, bit
for bit: packing (with and without the picks' index, widths whose packed rows are 16-,
4- and 1-byte aligned) and unpacking (every scale byte, every code)."""

import numpy as np
import pytest
import torch

from oracle import bf16, moe as omoe, mxfp8
from tests._util import announce, bf16_bits, normal_bf16, to_gpu, to_gpu_bf16, with_outliers

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n,d", [(300, 2048), (77, 2880), (64, 96), (5, 128), (1, 32)])
def test_tokens_pack_as_the_oracle_packs_them(lib, n, d):
    """d=2048 rows are 2112 bytes (16-aligned), 2880 gpt-oss's width (2970: 2-aligned,
    byte stores), 96 (99 bytes), 128 (132: 4-aligned)."""
    from bux_amd import dispatch
    rng = np.random.default_rng(50 + d)
    z = with_outliers(rng, normal_bf16(rng, (n, d)), 1e-2, 1e3)
    z[0, :32] = 0  # a block of zeros: byte 1
    announce("pack", n, d)
    got = dispatch.in_mxfp8(to_gpu_bf16(z)).cpu().numpy()
    np.testing.assert_array_equal(got, mxfp8.in_mxfp8(z))


def test_picks_pack_their_tokens_rows(lib):
    """in_mxfp8(z)[order // k] at config 3's shape: every pick's row, by index."""
    from bux_amd import dispatch
    rng = np.random.default_rng(51)
    t, k, e, d = 16384, 8, 128, 2048
    z = with_outliers(rng, normal_bf16(rng, (t, d)))
    idx = np.stack([rng.choice(e, k, replace=False) for _ in range(t)]).astype(np.int32)
    order = omoe.sort_by_expert(idx, e).order
    announce("pack picks c3")
    got = dispatch.picked_in_mxfp8(to_gpu_bf16(z), to_gpu(order), k)
    torch.cuda.synchronize()
    want = mxfp8.in_mxfp8(z)
    # compare through the token each pick packs (the oracle's gather), in chunks
    for lo in range(0, len(order), 16384):
        part = got[lo:lo + 16384].cpu().numpy()
        np.testing.assert_array_equal(part, want[order[lo:lo + 16384] // k])


def test_a_pick_outside_the_tokens_packs_zeros(lib):
    from bux_amd import dispatch
    rng = np.random.default_rng(52)
    z = normal_bf16(rng, (4, 64))
    # // 2: 0, 3, then 20 (past), -2 and -1 (before; C's division would take -1 to 0)
    order = np.array([0, 7, 40, -3, -1, 2**31 - 1], np.int32)
    announce("pack out of range")
    got = dispatch.picked_in_mxfp8(to_gpu_bf16(z), to_gpu(order), 2).cpu().numpy()
    want = mxfp8.in_mxfp8(z)
    np.testing.assert_array_equal(got[:2], want[[0, 3]])
    zeros = mxfp8.in_mxfp8(np.zeros((1, 64), np.uint16))[0]
    for row in got[2:]:
        np.testing.assert_array_equal(row, zeros)


@pytest.mark.parametrize("d", [2048, 2880, 96, 128])
def test_rows_unpack_as_the_oracle_unpacks_them(lib, d):
    """Random bytes: every code (NaN codes and subnormals too) and every scale byte
    0..255, against the oracle's float32 product rounded to bfloat16."""
    from bux_amd import dispatch
    rng = np.random.default_rng(53 + d)
    m = 512
    packed = rng.integers(0, 256, (m, d + d // 32), dtype=np.uint8)
    packed[:256, d] = np.arange(256, dtype=np.uint8)
    announce("unpack", d)
    got = bf16_bits(dispatch.from_mxfp8(to_gpu(packed), d))
    want = mxfp8.from_mxfp8(packed, d)
    nan = np.isnan(bf16.to_f32(want))
    np.testing.assert_array_equal(np.isnan(bf16.to_f32(got)), nan)
    np.testing.assert_array_equal(got[~nan], want[~nan])


def test_a_token_survives_the_round_trip_as_its_quantized_values(lib):
    """from_mxfp8(in_mxfp8(z)) = z's MXFP8 values in bfloat16 (the reference's round
    trip, tests/test_precision.py:344-352, at c3's width)."""
    from bux_amd import dispatch
    rng = np.random.default_rng(54)
    z = with_outliers(rng, normal_bf16(rng, (1000, 2048)))
    announce("pack round trip")
    back = bf16_bits(dispatch.from_mxfp8(dispatch.in_mxfp8(to_gpu_bf16(z)), 2048))
    np.testing.assert_array_equal(back, bf16.to_bf16(mxfp8.dequantized(mxfp8.mx_quantize(z))))
