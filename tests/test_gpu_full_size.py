"""The whole MXFP8 layer, forward and backward, at BASELINE.json's full shapes (configs
3, 4 and 5), where the oracle cannot follow: checked by properties that hold bit for bit
whatever the size.

- Scaling dy by 2 doubles every gradient exactly and leaves the forward as it was.
  MXFP8 takes a power of two exactly: the codes stay, each scale byte goes up by one.
  Every product the GEMMs sum then doubles, and so does every bfloat16 rounding and
  float32 sum after them. A second run of the forward also gives the same bits
  (determinism).
- Permuting the tokens permutes y, dz and the weights' gradient exactly. Every row's
  path is a function of that row alone: its quantization along its own width, its GEMM
  row, its activation, and its token's sum over the k picks in pick order. The column
  copies and the weight gradients take blocks of 32 sorted rows, which a permutation
  regroups, so they are not compared.

Inputs follow the configs: config 4's router logits carry a per-expert bias of
N(0, 0.5) and its activation is the clamped SwiGLU (limit 7, up offset 1); config 5's
picks are built from Zipf(1.2) loads over a permutation of the experts, a fifth of them
(51) receiving none and none more than 1/k of the picks (bench.zipf_picks)."""

import pytest
import torch

from bench import zipf_picks
from tests._util import announce

pytestmark = pytest.mark.gpu

CONFIGS = {
    "config3": dict(t=16384, d=2048, e=128, k=8, f=768, act=("swish", None, 0.0), skew=None),
    "config4": dict(t=8192, d=2880, e=128, k=4, f=2880, act=("quick_gelu", 7.0, 1.0),
                    skew="bias"),
    "config5": dict(t=8192, d=7168, e=256, k=8, f=2048, act=("swish", None, 0.0), skew="zipf"),
}


def _inputs(cfg, seed):
    dev = torch.device("cuda")
    g = torch.Generator(device=dev).manual_seed(seed)
    t, d, e, k, f = cfg["t"], cfg["d"], cfg["e"], cfg["k"], cfg["f"]
    z = torch.randn(t, d, generator=g, device=dev)
    hot = torch.randint(0, z.numel(), (z.numel() // 1000,), generator=g, device=dev)
    z.view(-1)[hot] *= 100
    if cfg["skew"] == "zipf":  # the loads built directly, as bench.py builds them
        picks, loads = zipf_picks(t, e, k, seed)
        assert (loads == 0).sum() == e // 5 and loads.max() <= t
        idx = torch.from_numpy(picks).to(dev)
        w = torch.softmax(torch.randn(t, k, generator=g, device=dev), -1).to(torch.bfloat16)
    else:
        logits = torch.randn(t, e, generator=g, device=dev)
        if cfg["skew"] == "bias":
            logits += torch.randn(e, generator=g, device=dev) * 0.5
        top = torch.topk(torch.softmax(logits, -1), k, -1)
        idx = top.indices.to(torch.int32)
        w = (top.values / top.values.sum(-1, keepdim=True)).to(torch.bfloat16)
    up = (torch.randn(e, d, f, 2, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    down = (torch.randn(e, f, d, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    dy = (torch.randn(t, d, generator=g, device=dev) * 0.01).to(torch.bfloat16)
    return z.to(torch.bfloat16), idx, w, up, down, dy


def _layer(z, idx, w, up, down, dy, ffn, **kw):
    from bux_amd import moe
    out, saved = moe.experts_forward(z, idx, w, up, down, ffn, **kw)
    grads = moe.experts_backward(saved, dy, up, down, ffn, **kw)
    del saved
    return out, {key: g for key, g in grads.items() if g is not None}


def _bits(x):
    return x.contiguous().view(torch.int16)


@pytest.mark.parametrize("name", list(CONFIGS))
def test_gradients_double_with_dy_and_the_forward_repeats(lib, name):
    from bux_amd import moe
    cfg = CONFIGS[name]
    z, idx, w, up, down, dy = _inputs(cfg, 1)
    ffn = moe.Ffn(*cfg["act"])
    announce("full size", name, "dy and 2 dy")
    out1, g1 = _layer(z, idx, w, up, down, dy, ffn)
    out2, g2 = _layer(z, idx, w, up, down, dy * 2, ffn)
    torch.cuda.synchronize()
    assert torch.equal(_bits(out1), _bits(out2)), "the forward differs between two runs"
    assert torch.isfinite(out1.float()).all()
    for key in g1:
        assert torch.isfinite(g1[key].float()).all(), key
        assert g1[key].abs().max() > 0, key
        assert torch.equal(_bits(g1[key] * 2), _bits(g2[key])), f"d{key} is not doubled exactly"


@pytest.mark.parametrize("name", ["config3", "config4"])
def test_a_float32_layers_gradients_double_with_dy_and_its_forward_repeats(lib, name):
    """The same properties for tokens and kernels in float32 (the kernels cast to the
    tokens' dtype, y and every gradient float32): doubling dy doubles each float32
    product and sum exactly, and the activation's gradient is linear in dh."""
    from bux_amd import moe
    cfg = CONFIGS[name]
    z, idx, w, up, down, dy = (x.float() if x.dtype == torch.bfloat16 else x
                               for x in _inputs(cfg, 4))
    ffn = moe.Ffn(*cfg["act"])
    announce("full size float32", name, "dy and 2 dy")
    out1, g1 = _layer(z, idx, w, up, down, dy, ffn)
    out2, g2 = _layer(z, idx, w, up, down, dy * 2, ffn)
    torch.cuda.synchronize()
    assert out1.dtype == torch.float32
    assert torch.equal(out1.view(torch.int32), out2.view(torch.int32)), "the forward differs"
    assert torch.isfinite(out1).all()
    for key in g1:
        assert g1[key].dtype == torch.float32, key
        assert torch.isfinite(g1[key]).all(), key
        assert g1[key].abs().max() > 0, key
        assert torch.equal((g1[key] * 2).view(torch.int32), g2[key].view(torch.int32)), \
            f"d{key} is not doubled exactly"


def test_a_float32_layer_with_biases_and_a_norm_at_full_size(lib):
    """Config 3 in float32 with the experts' up and down biases and a layernorm of their
    outputs (gain and bias, moe.py:857-872): the forward repeats bit for bit and doubling
    dy doubles every gradient exactly, the biases' and the norm's included (each is
    linear in dy, and doubling is exact in float32)."""
    from bux_amd import moe
    cfg = CONFIGS["config3"]
    z, idx, w, up, down, dy = (x.float() if x.dtype == torch.bfloat16 else x
                               for x in _inputs(cfg, 5))
    e, d, f = cfg["e"], cfg["d"], cfg["f"]
    g = torch.Generator(device="cuda").manual_seed(6)
    kw = dict(up_bias=torch.randn(e, f, 2, generator=g, device="cuda") * 0.5,
              down_bias=torch.randn(e, d, generator=g, device="cuda") * 0.5,
              norm=moe.ExpertNorm("layernorm", 1e-5, True, True),
              norm_scale=1 + 0.3 * torch.randn(d, generator=g, device="cuda"),
              norm_bias=0.2 * torch.randn(d, generator=g, device="cuda"))
    ffn = moe.Ffn(*cfg["act"])
    announce("full size float32, biases and a norm", "dy and 2 dy")
    out1, g1 = _layer(z, idx, w, up, down, dy, ffn, **kw)
    out2, g2 = _layer(z, idx, w, up, down, dy * 2, ffn, **kw)
    torch.cuda.synchronize()
    assert out1.dtype == torch.float32 and torch.isfinite(out1).all()
    assert torch.equal(out1.view(torch.int32), out2.view(torch.int32)), "the forward differs"
    assert {"up_bias", "down_bias", "norm_scale", "norm_bias"} <= set(g1)
    for key in g1:
        assert g1[key].dtype == torch.float32, key
        assert torch.isfinite(g1[key]).all(), key
        assert g1[key].abs().max() > 0, key
        assert torch.equal((g1[key] * 2).view(torch.int32), g2[key].view(torch.int32)), \
            f"d{key} is not doubled exactly"


@pytest.mark.parametrize("name", list(CONFIGS))
def test_a_permutation_of_the_tokens_permutes_y_and_dz(lib, name):
    from bux_amd import moe
    cfg = CONFIGS[name]
    z, idx, w, up, down, dy = _inputs(cfg, 2)
    ffn = moe.Ffn(*cfg["act"])
    perm = torch.randperm(cfg["t"], generator=torch.Generator(device="cuda").manual_seed(3),
                          device="cuda")
    announce("full size", name, "tokens permuted")
    out1, g1 = _layer(z, idx, w, up, down, dy, ffn)
    dz1, dw1 = g1["z"], g1["weights"]
    del g1
    out2, g2 = _layer(z[perm], idx[perm], w[perm], up, down, dy[perm], ffn)
    torch.cuda.synchronize()
    assert torch.equal(_bits(out1[perm]), _bits(out2))
    assert torch.equal(_bits(dz1[perm]), _bits(g2["z"]))
    assert torch.equal(_bits(dw1[perm]), _bits(g2["weights"]))


# Operands past 4 GiB: the GEMMs load one K chunk at a time from a 64-bit base, so an
# operand's size is bounded by its rows alone (bux_amd.h). Each group's outputs depend on
# its own rows and matrix only, so the GEMM over all groups equals, bit for bit, the
# GEMMs over two runs of whole groups taken apart (each of them under 4 GiB); a sample
# of rows from the operand's last K chunks is checked against float64 sums.
def _tiled_codes(lead, chunks, rows, gen):
    from bux_amd.grouped_mxfp8 import Tiled
    v = torch.randint(0, 0x70, (*lead, chunks, rows, 64), dtype=torch.uint8, device="cuda",
                      generator=gen)
    v |= torch.randint(0, 2, v.shape, dtype=torch.uint8, device="cuda", generator=gen) << 7
    s = torch.randint(118, 124, (*lead, chunks // 2, rows, 4), dtype=torch.uint8, device="cuda",
                      generator=gen)
    return Tiled(v, s)


def _rows_of(t, lo, hi):
    from bux_amd.grouped_mxfp8 import Tiled
    return Tiled(t.values[..., lo:hi, :].contiguous(), t.scales[..., lo:hi, :].contiguous())


def _f64(t):
    """A Tiled operand's values as float64 (rows, K), on the CPU."""
    from oracle import mxfp8
    v = t.values.cpu().numpy()
    s = t.scales.cpu().numpy()
    codes = v.transpose(1, 0, 2).reshape(v.shape[1], -1)
    scales = s.transpose(1, 0, 2).reshape(s.shape[1], -1)
    return mxfp8.dequantized(mxfp8.Blocks(codes, scales)).astype("float64")


def test_a_rows_gemm_over_an_operand_past_4_gib(lib):
    import numpy as np
    from bux_amd import grouped_mxfp8 as gm
    gen = torch.Generator(device="cuda").manual_seed(11)
    k, n, m = 7168, 256, 1_000_064  # a: 7.2 GB of codes, K chunks 64 MB apart
    sizes = torch.tensor([200_000, 0, 300_064, 123_456, 376_544], dtype=torch.int32, device="cuda")
    announce("rows gemm past 4 GiB", m, k)
    a = _tiled_codes((), k // 64, m, gen)
    b = _tiled_codes((5,), k // 64, n, gen)
    y = gm.rows(a, b, sizes, height=m)
    first = 500_064  # groups 0-2 | 3-4
    lo = gm.rows(_rows_of(a, 0, first), gm.Tiled(b.values[:3], b.scales[:3]), sizes[:3])
    hi = gm.rows(_rows_of(a, first, m), gm.Tiled(b.values[3:], b.scales[3:]), sizes[3:])
    torch.cuda.synchronize()
    assert torch.equal(y[:first].view(torch.int16), lo.view(torch.int16))
    assert torch.equal(y[first:].view(torch.int16), hi.view(torch.int16))
    # the last group's last rows against float64 sums (the bars of the GEMM tests)
    sample = _rows_of(a, m - 64, m)
    x = _f64(sample)
    w = _f64(gm.Tiled(b.values[4].contiguous(), b.scales[4].contiguous()))
    y32 = gm.rows(a, b, sizes, torch.float32, height=m)[m - 64:].cpu().numpy().astype(np.float64)
    want = x @ w.T
    assert np.abs(y32 - want).max() <= 5e-4 * np.abs(want).max()


def test_a_contract_gemm_over_an_operand_past_4_gib(lib):
    import numpy as np
    from bux_amd import grouped_mxfp8 as gm
    gen = torch.Generator(device="cuda").manual_seed(12)
    d, f, m = 256, 256, 20_000_000  # a: x^T, 5.1 GB of codes
    sizes = torch.tensor([5_000_000, 0, 7_000_000, 7_999_936], dtype=torch.int32, device="cuda")
    announce("contract gemm past 4 GiB", m)
    a = _tiled_codes((), m // 64, d, gen)
    b = _tiled_codes((), m // 64, f, gen)
    dw = gm.contract(a, b, sizes)
    first = 12_000_000  # groups 0-2 | 3, a multiple of 128 rows (the K chunks align)

    def part(t, lo, hi):
        return gm.Tiled(t.values[lo // 64:hi // 64].contiguous(), t.scales[lo // 128:hi // 128].contiguous())
    lo = gm.contract(part(a, 0, first), part(b, 0, first), sizes[:3])
    hi = gm.contract(part(a, first, m), part(b, first, m), sizes[3:])
    torch.cuda.synchronize()
    assert torch.equal(dw[:3].view(torch.int16), lo.view(torch.int16))
    assert torch.equal(dw[3:].view(torch.int16), hi.view(torch.int16))
    # the last group's sum over its last 1024 rows alone, against float64 sums
    tail = torch.tensor([0, 0, 0, 1024], dtype=torch.int32, device="cuda")
    start = m - 128 - 1024  # a whole 128 rows (the scale chunks align); past the groups none
    sub = gm.contract(part(a, start, m), part(b, start, m), tail, torch.float32)[3].cpu().numpy()
    xa, ya = _f64(part(a, start, start + 1024)), _f64(part(b, start, start + 1024))
    want = xa @ ya.T
    assert np.abs(sub.astype(np.float64) - want).max() <= 5e-4 * np.abs(want).max()
