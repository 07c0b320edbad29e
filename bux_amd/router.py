"""The MoE router on MI355X: each token's top-k experts and their weights, from its
logits, in one HIP kernel (``bux_route``).

Mirrors ``MoE._route`` (src/bux/architecture/experts/moe.py:236-273) off training —
no random logits (moe.py:250), no balance or observation taps (moe.py:263-265) — with
``MoE._logits`` (moe.py:275-284) and ``_limit_groups`` (moe.py:474-483). The router's
fields are ``MoEConfig``'s (src/bux/config.py:236-275): ``router``,
``router_logit_scale``, ``normalize_top_k``, ``routed_scaling_factor``,
``num_groups``, ``top_k_groups``; the kernel's columns past the scored experts are the
shared experts' sinks (``shared_expert_sink``, moe.py:143-153).
"""

from typing import NamedTuple

import torch

from bux_amd import _lib
from bux_amd.kernels import lib, ptr, require, stream, workspace

ROUTERS = {"softmax": _lib.ROUTER_SOFTMAX, "sigmoid": _lib.ROUTER_SIGMOID,
           "sqrtsoftplus": _lib.ROUTER_SQRTSOFTPLUS}


class Routed(NamedTuple):
    """What ``MoE._route`` returns (idx, weights, sinks), and the scores and logits."""

    idx: torch.Tensor  # int32 (t, k): the picks, the largest choice first
    weights: torch.Tensor  # bfloat16 (t, k): their weights
    sinks: torch.Tensor | None  # bfloat16 (t, s): the sinks' weights, None without sinks
    scores: torch.Tensor | None  # float32 (t, scored), if asked for
    logits: torch.Tensor | None  # float32 (t, scored + s), if asked for


def route(x: torch.Tensor, kernel: torch.Tensor, *, top_k: int, scored: int | None = None,
          router: str = "softmax", bias: torch.Tensor | None = None,
          router_logit_scale: float = 1.0, router_bias: torch.Tensor | None = None,
          num_groups: int = 1, top_k_groups: int = 1, normalize_top_k: bool = True,
          routed_scaling_factor: float = 1.0, with_scores: bool = False,
          with_logits: bool = False) -> Routed:
    """Route the bfloat16 tokens `x` (..., d) by the router's bfloat16 `kernel` (d, n):
    the first `scored` (default n) columns score the experts (routed, then zero
    experts), the rest are sinks. `bias` is the router's own float32 bias on the
    logits; `router_bias` the aux-free float32 bias on the choice (the reference's
    ``MoE.router_bias``). Raises ValueError for what the kernel does not take (more
    than 1024 logits, k or top_k_groups over 16, d not a multiple of 16)."""
    require(x, kernel)
    if x.dtype != torch.bfloat16 or kernel.dtype != torch.bfloat16:
        raise TypeError("x and kernel are bfloat16")
    if router not in ROUTERS:
        raise ValueError(f"router {router!r}: one of {sorted(ROUTERS)}")
    lead, d = x.shape[:-1], x.shape[-1]
    if kernel.dim() != 2 or kernel.shape[0] != d:
        raise ValueError(f"kernel {tuple(kernel.shape)} for width {d}")
    n = kernel.shape[1]
    scored = n if scored is None else scored
    xs = x.reshape(-1, d).contiguous()
    t = xs.shape[0]
    dev = x.device
    for name, v, size in (("bias", bias, n), ("router_bias", router_bias, scored)):
        if v is not None and (v.dtype != torch.float32 or v.numel() != size):
            raise ValueError(f"{name}: float32 of {size} elements")
    idx = torch.empty(t, top_k, dtype=torch.int32, device=dev)
    weights = torch.empty(t, top_k, dtype=torch.bfloat16, device=dev)
    sinks = torch.empty(t, n - scored, dtype=torch.bfloat16, device=dev) if n > scored else None
    scores = torch.empty(t, scored, dtype=torch.float32, device=dev) if with_scores else None
    logits = torch.empty(t, n, dtype=torch.float32, device=dev) if with_logits else None
    ws = workspace(lib().bux_route_workspace_size(d, n), dev)
    rc = lib().bux_route(
        ptr(xs), ptr(kernel.contiguous()), ptr(bias), t, d, n, router_logit_scale,
        ROUTERS[router], scored, ptr(router_bias), num_groups, top_k_groups, top_k,
        int(normalize_top_k), routed_scaling_factor, ptr(idx), ptr(weights), ptr(sinks),
        ptr(scores), ptr(logits), ptr(ws), ws.numel(), stream())
    if rc == 1:  # BUX_E_ARGUMENT
        raise ValueError(lib().bux_last_error().decode())
    _lib.check(rc)

    def shaped(v, width):
        return None if v is None else v.reshape(*lead, width)

    return Routed(shaped(idx, top_k), shaped(weights, top_k), shaped(sinks, n - scored),
                  shaped(scores, scored), shaped(logits, n))
