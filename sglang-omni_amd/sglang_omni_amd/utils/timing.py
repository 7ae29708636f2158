"""Per-launch timing of the decode kernels with HIP events on the launch stream.

A ``LaunchTimer`` installed on a decoder records an event pair around every kernel launch of a
given kind, together with that launch's algorithmic work (FLOPs or bytes). ``summary()`` (after a
synchronize) gives, per kind, the launch count, total kernel time and total work, from which the
roofline fractions follow. Without a timer the decoders record nothing.
"""

from __future__ import annotations

from contextlib import contextmanager
from dataclasses import dataclass, field

import torch


@dataclass
class _Kind:
    events: list[tuple[torch.cuda.Event, torch.cuda.Event]] = field(default_factory=list)
    work: float = 0.0


class LaunchTimer:
    """``per_layer`` also keys every launch by ``kind:detail`` (the layer name)."""

    def __init__(self, per_layer: bool = False) -> None:
        self.kinds: dict[str, _Kind] = {}
        self.per_layer = per_layer

    @contextmanager
    def launch(self, kind: str, work: float, detail: str | None = None):
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()
        yield  # a launch that raises (nothing enqueued) is not recorded
        end.record()
        keys = [kind]
        if self.per_layer and detail is not None:
            keys.append(f"{kind}:{detail}")
        for key in keys:
            entry = self.kinds.setdefault(key, _Kind())
            entry.events.append((start, end))
            entry.work += work

    def reset(self) -> None:
        self.kinds.clear()

    def summary(self) -> dict[str, dict[str, float]]:
        """{kind: {"launches", "ms", "work"}}; call after torch.cuda.synchronize()."""
        out = {}
        for kind, entry in self.kinds.items():
            ms = sum(s.elapsed_time(e) for s, e in entry.events)
            out[kind] = {"launches": len(entry.events), "ms": ms, "work": entry.work}
        return out


class _NoTimer:
    @contextmanager
    def launch(self, kind: str, work: float, detail: str | None = None):
        yield


NO_TIMER = _NoTimer()
