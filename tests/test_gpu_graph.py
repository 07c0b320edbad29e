"""The layer's forward and backward captured in one HIP graph (torch.cuda.CUDAGraph on
ROCm) and replayed: every replay, on new inputs copied into the captured ones and with
eager work and synchronisations between replays, bit for bit what the eager ops give
(the kernels are deterministic: fixed summation orders, no atomics). Nothing on the
path records a memset or synchronises with the host, so the capture holds."""

import numpy as np
import pytest
import torch

from tests._util import announce, normal_bf16, to_gpu, to_gpu_bf16

pytestmark = pytest.mark.gpu


def _inputs(rng, t, k, e, d, f):
    z = normal_bf16(rng, (t, d))
    idx = np.stack([rng.choice(e, k, replace=False) for _ in range(t)]).astype(np.int32)
    from oracle import bf16
    w = bf16.to_bf16(rng.random((t, k)).astype(np.float32) / k)
    up = normal_bf16(rng, (e, d, f, 2), 0.02)
    down = normal_bf16(rng, (e, f, d), 0.02)
    dy = normal_bf16(rng, (t, d), 1e-2)
    return (to_gpu_bf16(z), to_gpu(idx), to_gpu_bf16(w), to_gpu_bf16(up), to_gpu_bf16(down),
            to_gpu_bf16(dy))


def _step(z, idx, w, up, down, dy, fmt):
    from bux_amd import moe
    out, saved = moe.experts_forward(z, idx, w, up, down, fmt=fmt)
    grads = moe.experts_backward(saved, dy, up, down, fmt=fmt)
    return [out, grads["z"], grads["weights"], grads["up"], grads["down"]]


@pytest.mark.parametrize("fmt", ["mxfp8", "compute"])
def test_a_captured_step_replays_as_the_eager_one(lib, fmt):
    rng = np.random.default_rng(60)
    t, k, e, d, f = 512, 4, 16, 256, 256
    static = _inputs(rng, t, k, e, d, f)
    announce("graph capture", fmt)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            _step(*static, fmt)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = _step(*static, fmt)
    torch.cuda.synchronize()
    for replay in range(3):
        fresh = _inputs(rng, t, k, e, d, f)
        for dst, src in zip(static, fresh):
            dst.copy_(src)
        torch.cuda.synchronize()
        announce("graph replay", fmt, replay)
        graph.replay()
        torch.cuda.synchronize()
        want = _step(*fresh, fmt)  # eager, on the same values
        torch.cuda.synchronize()
        for name, got, ref in zip(("y", "dz", "dweights", "dup", "ddown"), captured, want):
            assert torch.equal(got, ref), (fmt, replay, name)
