"""bfloat16 as numpy uint16 bit patterns. TEST INFRASTRUCTURE ONLY (see `oracle`).

numpy has no bfloat16; bux's arrays on this path are bfloat16, so the oracle keeps
their bits in uint16 and widens to float32 exactly.

Pins (``tests/test_oracle.py``): `to_bf16` against torch's float32 -> bfloat16 cast on
random and edge values (ties, subnormals, overflow to inf); `to_f32` is exact by
construction (a shift), checked on all 65536 patterns against torch; `from_f64` (one
rounding from float64) against exact rational rounding (``fractions.Fraction``) on
values just off bfloat16 ties, where rounding through float32 would round twice.
"""

import numpy as np


def to_f32(bits: np.ndarray) -> np.ndarray:
    """Return bfloat16 bits (uint16) as float32, exactly."""
    return (np.asarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32)


def to_bf16(x: np.ndarray) -> np.ndarray:
    """Return float32 values rounded to nearest even bfloat16, as uint16 bits. NaN
    stays NaN (quiet)."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32)
    rounded = (u + np.uint32(0x7FFF) + ((u >> 16) & np.uint32(1))) >> 16
    nan = (u & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
    out = rounded.astype(np.uint16)
    out[nan] = ((u[nan] >> 16) | np.uint32(0x40)).astype(np.uint16)
    return out


def round_f32(x: np.ndarray) -> np.ndarray:
    """Return float32 values rounded to bfloat16 and widened back: x.astype(bf16)."""
    return to_f32(to_bf16(x))


def from_f64(x: np.ndarray) -> np.ndarray:
    """Return float64 values rounded once to nearest even bfloat16, as uint16 bits
    (finite, normal-range values): float64 -> float32 rounded to odd (truncated, its
    last bit set when inexact), then float32 -> bfloat16 to nearest even. Rounding to
    odd keeps the information a second rounding needs, since float32 carries 16 more
    bits than bfloat16."""
    x = np.asarray(x, np.float64)
    r = x.astype(np.float32)
    # truncate toward zero: step back where rounding went away from 0
    away = np.abs(r.astype(np.float64)) > np.abs(x)
    r = np.where(away, np.nextafter(r, np.float32(0)), r)
    u = r.view(np.uint32).copy()
    inexact = r.astype(np.float64) != x
    u[inexact] |= np.uint32(1)
    return to_bf16(u.view(np.float32))
