"""Optional timing of the ops the layer enqueues: HIP events recorded on the current
stream (the one every op launches on) before and after each op, named. Off unless a
`Spans` is active, when `span` is a no-op context.

    with Spans() as spans:
        moe.experts_forward(...)
    spans.milliseconds()  # {"x quantize": [..], "up fprop": [..], ...}
"""

import contextlib
from collections import defaultdict

import torch

_ACTIVE: "Spans | None" = None


class Spans:
    """Collects event pairs by name while active."""

    def __init__(self) -> None:
        self.events: dict[str, list[tuple[torch.cuda.Event, torch.cuda.Event]]] = defaultdict(list)

    def __enter__(self) -> "Spans":
        global _ACTIVE
        self._outer = _ACTIVE
        _ACTIVE = self
        return self

    def __exit__(self, *exc) -> None:
        global _ACTIVE
        _ACTIVE = self._outer

    def milliseconds(self) -> dict[str, list[float]]:
        """Return each name's durations in ms (synchronises on the last events)."""
        out = {}
        for name, pairs in self.events.items():
            if pairs:
                pairs[-1][1].synchronize()
            out[name] = [a.elapsed_time(b) for a, b in pairs]
        return out


@contextlib.contextmanager
def span(name: str):
    """Time what the block enqueues on the current stream under `name`, if a `Spans` is
    active."""
    spans = _ACTIVE
    if spans is None:
        yield
        return
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    yield
    end.record()
    spans.events[name].append((start, end))
