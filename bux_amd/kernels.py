"""Where the kernels run, and the plumbing every op shares: device checks, the current
stream, raw pointers.

Replaces ``bux.kernels`` (src/bux/kernels.py:25-72) and the CUDA-capability gates
``grouped_mxfp8.runs`` (src/bux/architecture/experts/grouped_mxfp8.py:84-87) and
``grouped_blockscaled._triton`` (grouped_blockscaled.py:320-323): the HIP kernels run
on a gfx950 GPU (MI355X), unless ``BUX_KERNELS=off``. There is no other
implementation to fall back to: an op called where they do not run raises.
"""

import functools
import os

import torch

from bux_amd import _lib


def off() -> bool:
    """Return whether ``BUX_KERNELS=off`` turns the kernels off (src/bux/kernels.py:25-30)."""
    return os.environ.get("BUX_KERNELS", "").lower() == "off"


@functools.lru_cache(maxsize=None)
def _arch(index: int) -> str:
    return torch.cuda.get_device_properties(index).gcnArchName.split(":")[0]


def runs(device: torch.device | None = None) -> bool:
    """Return whether the HIP kernels run on `device` (the current GPU if None): a
    gfx950 GPU, the library built, and the kernels not turned off."""
    if off() or not torch.cuda.is_available():
        return False
    index = torch.cuda.current_device() if device is None or device.index is None else device.index
    return _arch(index) == "gfx950" and os.path.exists(_lib.PATH)


def lib():
    """Return the library; raises if it is not built."""
    return _lib.load()


def require(*tensors: torch.Tensor) -> None:
    """Raise unless every tensor lies on a gfx950 GPU where the kernels run, and is
    contiguous."""
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise ValueError(f"bux_amd kernels take GPU tensors, got one on {t.device}")
        if not t.is_contiguous():
            raise ValueError("bux_amd kernels take contiguous tensors")
    device = next((t.device for t in tensors if t is not None), None)
    if not runs(device):
        raise RuntimeError("bux_amd kernels do not run here: they need a gfx950 GPU and the "
                           "built library (python -m bux_amd.build), with BUX_KERNELS unset")


def ptr(t: torch.Tensor | None) -> int | None:
    """Return a tensor's device address (None for None)."""
    return None if t is None else t.data_ptr()


def stream() -> int:
    """Return the current HIP stream's handle, on which every op enqueues its kernels."""
    return torch.cuda.current_stream().cuda_stream


def workspace(nbytes: int, device: torch.device) -> torch.Tensor:
    """Return a scratch buffer of at least `nbytes` bytes (at least 1) on `device`."""
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)
