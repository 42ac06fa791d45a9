"""HIP-event phase timer for the wave loop.

``mark(phase)`` records an event on torch's current stream (the stream the library's kernels
are launched on) and attributes the interval up to the next mark to ``phase``.
"""
from __future__ import annotations

from collections import defaultdict

import torch


class PhaseTimer:
    def __init__(self, device=None):
        self.device = device
        self.events: list[tuple[str | None, torch.cuda.Event]] = []
        self.counts: dict[str, int] = defaultdict(int)

    def mark(self, phase: str | None) -> None:
        ev = torch.cuda.Event(enable_timing=True)
        ev.record(torch.cuda.current_stream(self.device))
        self.events.append((phase, ev))
        if phase is not None:
            self.counts[phase] += 1

    def totals_ms(self) -> dict[str, float]:
        torch.cuda.synchronize(self.device)
        out: dict[str, float] = defaultdict(float)
        for (p0, e0), (_, e1) in zip(self.events, self.events[1:]):
            if p0 is not None:
                out[p0] += e0.elapsed_time(e1)
        return dict(out)

    def reset(self) -> None:
        self.events.clear()
        self.counts.clear()
