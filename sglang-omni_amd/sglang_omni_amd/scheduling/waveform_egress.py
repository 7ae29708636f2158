"""Device-to-host egress of decoded waveforms through a bounded pool of pinned slots.

The slot policy is the reference scheduler's (``Code2WavScheduler.stage_window`` /
``flush_pending`` / ``acquire_slot`` / ``release_slot`` / ``retire_slot`` / ``quarantine_slot`` /
``reap_retired``, sglang_omni/models/qwen3_omni/components/code2wav_scheduler.py:756-928):

* a window's samples go into a free pinned slot by an asynchronous copy on the decode stream,
  fenced by the slot's event, and are read only after the event completed;
* at most ``max_pinned_slots`` slots exist; with none free the oldest pending window is flushed
  first, and if that frees none the window is copied synchronously;
* a copy that fails before its event was recorded quarantines the slot (never reused, and the
  pipeline stops overlapping); one that fails after retires it until its event completes.

Where the reference stages each request's window with its own copy, a decode step here leaves
the device as one transfer: all of the step's rows in one slot, by one copy. The samples travel
as float32 or, with ``format="pcm16"``, as signed 16-bit PCM encoded on the device by
``omni_waveform_egress`` (half the bytes over PCIe).
"""

from __future__ import annotations

import time
from collections import deque
from collections.abc import Hashable, Sequence
from dataclasses import dataclass

import numpy as np
import torch

from ..kernels.egress import FORMATS, waveform_egress
from ..utils.cuda_staging import PinnedTransferSlot, normalize_device


@dataclass
class PendingStep:
    """A decode step's rows on their way to the host."""

    slot: PinnedTransferSlot
    request_ids: list[Hashable]
    row_stride: int  # slot elements per row
    samples: list[int]  # each row's sample count
    launch_index: int


class WaveformEgress:
    """Stages decode steps' waveforms (B, 1, samples) toward the host; returns each row's audio
    as an owned numpy array (float32, or int16 for ``format="pcm16"``) once its copy is done."""

    def __init__(self, device: torch.device | str, *, format: str = "f32",
                 max_pinned_slots: int = 4, default_slot_samples: int = 0) -> None:
        if format not in FORMATS:
            raise ValueError(f"format must be one of {sorted(FORMATS)}; got {format!r}")
        if max_pinned_slots < 0:
            raise ValueError("max_pinned_slots must be >= 0")
        self.device = normalize_device(device)
        self.format = format
        self.dtype = FORMATS[format][1]
        self.max_pinned_slots = max_pinned_slots
        self.default_slot_samples = default_slot_samples
        self.pinned_free: list[PinnedTransferSlot] = []
        self.pinned_retired: list[PinnedTransferSlot] = []
        self.pinned_quarantined: list[PinnedTransferSlot] = []
        self.pinned_created = 0
        self.pending: deque[PendingStep] = deque()
        self.pipeline_active = True
        self.step_launch_count = 0
        self.wait_ns = 0  # host time spent waiting for copies

    # ------------------------------------------------------------------ staging

    def stage_step(self, request_ids: Sequence[Hashable], waveform: torch.Tensor,
                   row_samples: Sequence[int] | None = None) -> list[tuple[Hashable, np.ndarray]]:
        """Start the copy of one decode step's waveform (B, 1, samples) or (B, samples), row r
        belonging to request_ids[r] and keeping its first row_samples[r] samples (all by
        default). Returns the audio that had to be completed now: earlier steps flushed to free
        a slot, and this step itself when it was copied synchronously."""
        rows = waveform[:, 0] if waveform.dim() == 3 else waveform
        if rows.dim() != 2 or rows.shape[0] != len(request_ids):
            raise ValueError("one request id per waveform row")
        batch, width = rows.shape
        counts = [width] * batch if row_samples is None else [int(n) for n in row_samples]
        if len(counts) != batch or any(n < 0 or n > width for n in counts):
            raise ValueError(f"row_samples must give 0..{width} samples for each of {batch} rows")
        packed = self._packed(rows)
        total = batch * width
        ready: list[tuple[Hashable, np.ndarray]] = []
        slot = self.acquire_slot(total)
        if slot is None and self.pending:
            ready += self._flush_one()
            slot = self.acquire_slot(total)
        if slot is None:
            host = packed.cpu()
            ready += self._rows_of(host.view(batch, width), list(request_ids), counts)
            return ready
        recorded = False
        try:
            slot.view(total).view(batch, width).copy_(packed, non_blocking=True)
            slot.record(torch.cuda.current_stream(self.device))
            recorded = True
        except Exception:
            if recorded:
                self.retire_slot(slot)
            else:
                self.quarantine_slot(slot)
            raise
        self.step_launch_count += 1
        self.pending.append(PendingStep(slot, list(request_ids), width, counts,
                                        self.step_launch_count))
        return ready

    def _packed(self, rows: torch.Tensor) -> torch.Tensor:
        """The step's samples in this egress's format as one contiguous (B, samples) device
        tensor: the waveform itself when it already is one, else the egress kernel's output."""
        if self.format == "f32" and rows.dtype == torch.float32 and rows.is_contiguous():
            return rows
        return waveform_egress(rows, format=self.format)

    # ------------------------------------------------------------------ completion

    def poll(self) -> list[tuple[Hashable, np.ndarray]]:
        """The audio of every pending step whose copy has finished, in launch order, without
        blocking."""
        ready: list[tuple[Hashable, np.ndarray]] = []
        while self.pending and self.pending[0].slot.query():
            ready += self._flush_one()
        return ready

    def flush(self) -> list[tuple[Hashable, np.ndarray]]:
        """The audio of every pending step, waiting for their copies."""
        ready: list[tuple[Hashable, np.ndarray]] = []
        while self.pending:
            ready += self._flush_one()
        return ready

    def _flush_one(self) -> list[tuple[Hashable, np.ndarray]]:
        step = self.pending.popleft()
        start = time.monotonic_ns()
        if not step.slot.query():
            step.slot.synchronize()
        self.wait_ns += time.monotonic_ns() - start
        host = step.slot.view(len(step.request_ids) * step.row_stride)
        audio = self._rows_of(host.view(-1, step.row_stride), step.request_ids, step.samples)
        self.release_slot(step.slot)
        return audio

    @staticmethod
    def _rows_of(host: torch.Tensor, request_ids: list[Hashable],
                 counts: list[int]) -> list[tuple[Hashable, np.ndarray]]:
        array = host.numpy()
        return [(rid, array[r, :n].copy()) for r, (rid, n) in enumerate(zip(request_ids, counts))]

    # ------------------------------------------------------------------ slot pool

    def acquire_slot(self, elements: int) -> PinnedTransferSlot | None:
        self.reap_retired()
        if self.pinned_free:
            slot = self.pinned_free.pop()
            try:
                slot.ensure_capacity(elements)
            except Exception:
                self.release_slot(slot)
                raise
            return slot
        if self.pinned_created < self.max_pinned_slots:
            slot = PinnedTransferSlot(self.device, self.dtype,
                                      initial_capacity=max(elements, self.default_slot_samples),
                                      blocking=True)
            self.pinned_created += 1
            return slot
        return None

    def release_slot(self, slot: PinnedTransferSlot) -> None:
        self.pinned_free.append(slot)

    def retire_slot(self, slot: PinnedTransferSlot) -> None:
        self.pinned_retired.append(slot)

    def quarantine_slot(self, slot: PinnedTransferSlot) -> None:
        self.pinned_quarantined.append(slot)
        self.pipeline_active = False

    def reap_retired(self) -> None:
        """Return retired slots whose copies finished to the free list, without blocking; a slot
        whose event cannot be queried is quarantined."""
        still: list[PinnedTransferSlot] = []
        for slot in self.pinned_retired:
            try:
                complete = slot.query()
            except Exception:
                self.quarantine_slot(slot)
                continue
            if complete:
                self.release_slot(slot)
            else:
                still.append(slot)
        self.pinned_retired = still


__all__ = ["PendingStep", "WaveformEgress"]
