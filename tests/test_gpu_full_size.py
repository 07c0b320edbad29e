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


def _layer(z, idx, w, up, down, dy, ffn):
    from bux_amd import moe
    out, saved = moe.experts_forward(z, idx, w, up, down, ffn)
    grads = moe.experts_backward(saved, dy, up, down, ffn)
    del saved
    return out, grads


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
