"""Pinned host staging buffers and device completion events for waveform egress.

Keeps the API of the reference's ``sglang_omni/utils/cuda_staging.py:20-204``
(``allocate_pinned``, ``new_device_event``, ``normalize_device``, ``GrowablePinnedBuffer``,
``PinnedTransferSlot``) with the same contract: the owner serializes access, grows a buffer only
while no asynchronous copy can still be using it, and leaves a slot alone between ``record()``
and observed completion (``synchronize()`` returned, or ``query()`` reported True).

Pinned memory is allocated (torch's ``pin_memory=True``, hipHostMalloc underneath); existing
host memory is never registered.
"""

from __future__ import annotations

import torch


def allocate_pinned(numel: int, dtype: torch.dtype) -> torch.Tensor:
    """A fresh pinned host tensor, created outside inference mode so it can be filled under
    inference mode and reused or cloned outside it."""
    with torch.inference_mode(False):
        return torch.empty(numel, dtype=dtype, pin_memory=True)


def new_device_event(device: torch.device, *, blocking: bool = False) -> torch.cuda.Event:
    """A completion event; a blocking one makes synchronize() sleep instead of spinning."""
    del device  # HIP events are not bound to a device until recorded
    return torch.cuda.Event(blocking=blocking)


def normalize_device(device: torch.device | str | int) -> torch.device:
    """The device with its index filled in (the current device for a bare "cuda")."""
    resolved = torch.device("cuda", device) if isinstance(device, int) else torch.device(device)
    if resolved.type == "cuda" and resolved.index is None:
        return torch.device("cuda", torch.cuda.current_device())
    return resolved


class GrowablePinnedBuffer:
    """A pinned host buffer that only grows, to exactly the size asked for. ``view()`` never
    allocates; ``ensure_capacity()`` keeps the old storage if the new allocation fails."""

    def __init__(self, dtype: torch.dtype, *, initial_capacity: int = 0) -> None:
        if initial_capacity < 0:
            raise ValueError("initial_capacity must be >= 0")
        self.dtype = dtype
        self.storage: torch.Tensor | None = None
        if initial_capacity:
            self.ensure_capacity(initial_capacity)

    @property
    def capacity(self) -> int:
        return 0 if self.storage is None else int(self.storage.numel())

    def ensure_capacity(self, required: int) -> None:
        if required < 0:
            raise ValueError("required capacity must be >= 0")
        if required > self.capacity:
            self.storage = allocate_pinned(required, self.dtype)

    def view(self, numel: int) -> torch.Tensor:
        if numel < 0 or numel > self.capacity:
            raise ValueError(f"requested {numel} elements from a pinned buffer with capacity "
                             f"{self.capacity}")
        if self.storage is None:
            with torch.inference_mode(False):
                return torch.empty(0, dtype=self.dtype)
        return self.storage[:numel]


class PinnedTransferSlot:
    """One growable pinned buffer plus one reusable completion event. ``recorded`` is True only
    while the latest ``record()`` succeeded, so a failed record never leaves an earlier
    transfer's event readable as this one's."""

    def __init__(self, device: torch.device | str, dtype: torch.dtype, *,
                 initial_capacity: int = 0, blocking: bool = False) -> None:
        self.device = normalize_device(device)
        self.buffer = GrowablePinnedBuffer(dtype, initial_capacity=initial_capacity)
        self.blocking = blocking
        self.event: torch.cuda.Event | None = None
        self.recorded = False

    @property
    def capacity(self) -> int:
        return self.buffer.capacity

    def ensure_capacity(self, required: int) -> None:
        self.buffer.ensure_capacity(required)

    def view(self, numel: int) -> torch.Tensor:
        return self.buffer.view(numel)

    def device_guard(self) -> torch.cuda.device:
        return torch.cuda.device(self.device)

    def record(self, stream: torch.cuda.Stream | None) -> None:
        """Record the completion event on ``stream`` (a stream of this slot's device)."""
        self.recorded = False
        stream_device = getattr(stream, "device", None)
        if stream_device is not None and normalize_device(stream_device) != self.device:
            raise ValueError(f"cannot record a transfer slot on {self.device} from a stream on "
                             f"{stream_device}")
        with self.device_guard():
            if self.event is None:
                self.event = new_device_event(self.device, blocking=self.blocking)
            self.event.record(stream)
        self.recorded = True

    def recorded_event(self) -> torch.cuda.Event:
        if not self.recorded:
            raise RuntimeError("transfer event was not recorded: no record() has succeeded on "
                               "this slot since it was created or since its last record() raised")
        return self.event

    def query(self) -> bool:
        """Whether the recorded transfer has completed, without blocking."""
        event = self.recorded_event()
        with self.device_guard():
            return bool(event.query())

    def synchronize(self) -> None:
        """Block until the recorded transfer has completed."""
        event = self.recorded_event()
        with self.device_guard():
            event.synchronize()


__all__ = ["GrowablePinnedBuffer", "PinnedTransferSlot", "allocate_pinned", "new_device_event",
           "normalize_device"]
