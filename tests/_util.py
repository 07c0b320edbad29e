"""Helpers the tests share: moving bfloat16 bits between numpy and torch, seeded
inputs, and printing which case a GPU step runs (so a failing run names it)."""

import sys

import numpy as np
import torch

from oracle import bf16


def announce(*what) -> None:
    """Print (and flush) the case a GPU step is about to run."""
    print("[case]", *what, file=sys.stderr, flush=True)


def to_gpu_bf16(bits: np.ndarray) -> torch.Tensor:
    """Return bfloat16 bits (uint16) as a bfloat16 tensor on cuda:0."""
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).cuda()


def bf16_bits(t: torch.Tensor) -> np.ndarray:
    """Return a bfloat16 tensor's bits as uint16 numpy."""
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def to_gpu(a: np.ndarray, dtype=None) -> torch.Tensor:
    t = torch.from_numpy(np.ascontiguousarray(a))
    return (t if dtype is None else t.to(dtype)).cuda()


def normal_bf16(rng: np.random.Generator, shape, scale: float = 1.0) -> np.ndarray:
    """Return bfloat16 bits of N(0, scale^2) draws."""
    return bf16.to_bf16((rng.standard_normal(shape) * scale).astype(np.float32))


def with_outliers(rng: np.random.Generator, bits: np.ndarray, fraction: float = 1e-3,
                  factor: float = 100.0) -> np.ndarray:
    """Return bfloat16 bits with a seeded `fraction` of entries scaled by `factor`
    (the benchmark configs' outliers, which exercise the scales)."""
    v = bf16.to_f32(bits).copy()
    flat = v.reshape(-1)
    at = rng.choice(flat.size, max(1, int(flat.size * fraction)), replace=False)
    flat[at] *= factor
    return bf16.to_bf16(v)


def rel_err(got: np.ndarray, want: np.ndarray) -> float:
    """Return ||got - want|| / ||want|| in float64 (0 when both are 0)."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    den = np.linalg.norm(want)
    num = np.linalg.norm(got - want)
    return float(num / den) if den > 0 else float(num)


def untiled(t, cols: int) -> tuple[np.ndarray, np.ndarray]:
    """Return a device `Tiled` (codes (..., K/64, r, 64), scale bytes (..., K/128, r, 4))
    row-major on the host, codes (..., r, cols) and scale bytes (..., r, cols/32), after
    checking that its K padding holds codes 0 and scale bytes 1."""
    v = t.values.cpu().numpy()
    s = t.scales.cpu().numpy()
    n = v.ndim - 3
    v = np.swapaxes(v, n, n + 1).reshape(*v.shape[:n], v.shape[-2], -1)
    s = np.swapaxes(s, n, n + 1).reshape(*s.shape[:n], s.shape[-2], -1)
    assert (v[..., cols:] == 0).all(), "codes past the columns are not 0"
    assert (s[..., cols // 32:] == 1).all(), "scale bytes past the columns are not 1"
    return v[..., :cols], s[..., :cols // 32]


def to_gpu_tiled(blocks):
    """Return row-major MXFP8 blocks (the oracle's) on cuda:0, tiled for the GEMMs."""
    from bux_amd import grouped_mxfp8
    return grouped_mxfp8.tiled(to_gpu(blocks.values), to_gpu(blocks.scales))


def ulps_apart(got_bits: np.ndarray, want_bits: np.ndarray) -> np.ndarray:
    """How many bfloat16 steps apart two arrays of bfloat16 bits are, elementwise (±0
    one value; steps counted through 0 across a sign change)."""
    def rank(bits):
        b = bits.astype(np.int64)
        mag = b & 0x7FFF
        return np.where(b & 0x8000, -mag, mag)
    return np.abs(rank(np.asarray(got_bits)) - rank(np.asarray(want_bits)))


def e4m3_steps_apart(got: np.ndarray, want: np.ndarray) -> np.ndarray:
    """How many E4M3 codes apart two arrays of codes are in value order, elementwise."""
    def rank(codes):
        c = codes.astype(np.int64)
        mag = c & 0x7F
        return np.where(c & 0x80, -mag, mag)
    return np.abs(rank(got) - rank(want))


def attribute_codes(got_codes, got_scales, want_codes, want_scales, got_bits, want_bits):
    """Attribute the differences between two MXFP8 copies (row-major codes (r, c) and
    scale bytes (r, c/32)) of two bfloat16 arrays (r, c) to the differences between those
    arrays. Returns counts; raises AssertionError on a difference with no cause:
    - a block's scale byte differs only if one of its 32 values differs;
    - where the scale agrees, a code differs only where its value differs, and then by
      at most as many codes as its value by bfloat16 steps (E4M3 keeps fewer mantissa
      bits than bfloat16, so neighbouring values round to the same or neighbouring
      codes)."""
    r, c = got_codes.shape
    val_diff = ulps_apart(got_bits, want_bits)
    block_diff = (val_diff.reshape(r, c // 32, 32) > 0).any(-1)
    scale_diff = got_scales != want_scales
    assert not (scale_diff & ~block_diff).any(), "a scale differs in a block of equal values"
    same_scale = np.repeat(~scale_diff, 32, axis=1)
    steps = e4m3_steps_apart(got_codes, want_codes)
    code_diff = (steps > 0) & same_scale
    assert not (code_diff & (val_diff == 0)).any(), "a code differs where its value does not"
    assert (steps[code_diff] <= np.maximum(val_diff[code_diff], 1)).all(), \
        "a code differs by more steps than its value"
    return {"values": int((val_diff > 0).sum()), "codes": int(code_diff.sum()),
            "scales": int(scale_diff.sum()), "max_value_steps": int(val_diff.max(initial=0)),
            "max_code_steps": int(steps[same_scale].max(initial=0)), "of": int(r * c)}
