"""Per-boundary GPU timing for executor launches.

Counterpart of the reference's ``BoundaryProfiler``
(``models/flashnext/boundary_profiler.py:1-30``): opt-in through
``FLASHNEXT_PROFILE_BOUNDARIES=1`` (or the constructor), optionally restricted
to one label, and timed with GPU events on the current stream instead of a
host round trip.
"""
from __future__ import annotations

import os
from typing import Any, Callable

LABELS = ("gate_qmv", "up_qmv", "swiglu", "down_qmv", "fused_down", "router")


class BoundaryProfiler:
    def __init__(self, enabled: bool | None = None, boundary: str | None = None):
        if enabled is None:
            enabled = os.environ.get("FLASHNEXT_PROFILE_BOUNDARIES") == "1"
        if boundary is None:
            boundary = os.environ.get("FLASHNEXT_PROFILE_BOUNDARY") or None
        if boundary is not None and boundary not in LABELS:
            raise ValueError(f"unknown boundary {boundary!r}; expected one of {LABELS}")
        self.enabled = bool(enabled)
        self.boundary = boundary
        self.reset()

    def selected_for(self, label: str) -> bool:
        return self.enabled and (self.boundary is None or self.boundary == label)

    def reset(self) -> None:
        self._events: list[tuple[str, Any, Any]] = []

    def measure(self, label: str, issue: Callable[[], Any]) -> Any:
        import torch

        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()
        result = issue()
        end.record()
        self._events.append((label, start, end))
        return result

    def snapshot(self) -> dict[str, Any]:
        import torch

        if self._events:
            torch.cuda.synchronize()
        events = [{"label": label, "ms": start.elapsed_time(end)} for label, start, end in self._events]
        totals: dict[str, float] = {}
        for item in events:
            totals[item["label"]] = totals.get(item["label"], 0.0) + item["ms"]
        return {"enabled": self.enabled, "boundary": self.boundary, "events": events, "totals_ms": totals}
