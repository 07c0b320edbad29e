"""bux_mx_grouped_rows_noalloc, the rows GEMM whose workspace lives in a static device
array, called through the C ABI: bit for bit bux_mx_grouped_rows (with a workspace the
caller allocates) on the same operands, on two calls in a row, the second smaller (the
array keeps the first call's tile list, which the second's prologue overwrites), in
bfloat16 and float32 out; and a call too large for the array fails before any launch."""

import ctypes

import numpy as np
import pytest
import torch

from tests._util import announce

pytestmark = pytest.mark.gpu


def _operands(rng, sizes, m, k, n):
    from bux_amd import grouped_mxfp8

    g = torch.Generator(device="cuda").manual_seed(int(rng.integers(1 << 30)))
    x = torch.randn(m, k, generator=g, device="cuda").to(torch.bfloat16)
    w = (torch.randn(len(sizes), n, k, generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    a, _ = grouped_mxfp8.quantized_twice(x, columns=False)
    b, _ = grouped_mxfp8.quantized_twice(w, columns=False)
    return a, b, torch.from_numpy(np.asarray(sizes, np.int32)).cuda()


def _both(lib, a, b, sizes, height, dtype):
    from bux_amd import _lib
    from bux_amd.kernels import stream

    groups, n = b.values.shape[0], b.height
    m, k = a.height, a.k
    out = {torch.bfloat16: _lib.BF16, torch.float32: _lib.F32}[dtype]
    want = torch.full((height, n), float("nan"), dtype=dtype, device="cuda")
    got = torch.full((height, n), float("nan"), dtype=dtype, device="cuda")
    ws = torch.empty(lib.bux_mx_grouped_rows_workspace_size(groups, m, height), dtype=torch.uint8,
                     device="cuda")
    _lib.check(lib.bux_mx_grouped_rows(
        a.values.data_ptr(), a.scales.data_ptr(), b.values.data_ptr(), b.scales.data_ptr(),
        sizes.data_ptr(), groups, m, n, k, height, out, want.data_ptr(), ws.data_ptr(), ws.numel(),
        stream()))
    _lib.check(lib.bux_mx_grouped_rows_noalloc(
        a.values.data_ptr(), a.scales.data_ptr(), b.values.data_ptr(), b.scales.data_ptr(),
        sizes.data_ptr(), groups, m, n, k, height, out, got.data_ptr(), stream()))
    torch.cuda.synchronize()
    return got, want


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_noalloc_rows_equal_the_workspace_rows_twice(lib, dtype):
    rng = np.random.default_rng(50)
    # first: config 3's expert count and widths, ragged groups, rows past the groups
    sizes = np.bincount(rng.integers(0, 128, 30000), minlength=128).astype(np.int32)
    sizes[[3, 77]] = 0
    m = -(-int(sizes.sum()) // 128) * 128 + 128
    announce("noalloc rows, first", dtype, m)
    a, b, gs = _operands(rng, sizes, m, 2048, 1536)
    got, want = _both(lib, a, b, gs, m, dtype)
    assert torch.equal(got.view(torch.int16 if dtype == torch.bfloat16 else torch.int32),
                       want.view(torch.int16 if dtype == torch.bfloat16 else torch.int32))
    assert not torch.isnan(got).any()
    # second, smaller: fewer groups and rows, another width
    sizes = np.array([0, 130, 1, 3, 256, 0, 300, 100], np.int32)
    m = 896
    announce("noalloc rows, second", dtype, m)
    a, b, gs = _operands(rng, sizes, m, 256, 384)
    got, want = _both(lib, a, b, gs, 800, dtype)
    assert torch.equal(got.view(torch.int16 if dtype == torch.bfloat16 else torch.int32),
                       want.view(torch.int16 if dtype == torch.bfloat16 else torch.int32))
    assert not torch.isnan(got).any()


def test_noalloc_rejects_a_list_past_its_array(lib):
    from bux_amd import _lib

    p = ctypes.c_void_p(16)  # never dereferenced: the size check fails first
    groups, m = 4096, 1 << 22
    assert lib.bux_mx_grouped_rows_workspace_size(groups, m, m) > _lib.NOALLOC_SCRATCH_BYTES
    rc = lib.bux_mx_grouped_rows_noalloc(p, p, p, p, p, groups, m, 256, 128, m, 0, p, None)
    assert rc == 2 and "bux_mx_grouped_rows_noalloc" in lib.bux_last_error().decode()
