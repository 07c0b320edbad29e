"""bfloat16 as numpy uint16 bit patterns. TEST INFRASTRUCTURE ONLY (see `oracle`).

numpy has no bfloat16; bux's arrays on this path are bfloat16, so the oracle keeps
their bits in uint16 and widens to float32 exactly.

Pins (``tests/test_oracle.py``): `to_bf16` against torch's float32 -> bfloat16 cast on
random and edge values (ties, subnormals, overflow to inf); `to_f32` is exact by
construction (a shift), checked on all 65536 patterns against torch.
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
