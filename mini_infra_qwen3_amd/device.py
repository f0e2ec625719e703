"""Device synchronisation and step timing. Reference src/mini_infra/device.py:20-62."""

from __future__ import annotations

import time
from types import TracebackType

import torch


def synchronize(device: torch.device) -> None:
    if device.type == "cuda":
        torch.cuda.synchronize(device)


class StepTimer:
    """Times one step: on the GPU a sync, an event pair around the body, a sync; else wall clock."""

    def __init__(self, device: torch.device):
        self.device = device
        self.elapsed_ms = 0.0
        self._events: tuple[torch.cuda.Event, torch.cuda.Event] | None = None
        self._t0 = 0.0

    def __enter__(self) -> "StepTimer":
        if self.device.type == "cuda":
            synchronize(self.device)
            self._events = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
            self._events[0].record()
        else:
            self._t0 = time.perf_counter()
        return self

    def __exit__(self, exc_type: type[BaseException] | None, exc: BaseException | None,
                 tb: TracebackType | None) -> None:
        if self._events is not None:
            start, end = self._events
            end.record()
            synchronize(self.device)
            self.elapsed_ms = start.elapsed_time(end)
        else:
            self.elapsed_ms = (time.perf_counter() - self._t0) * 1000.0


__all__ = ["StepTimer", "synchronize"]
