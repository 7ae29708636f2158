"""Device-to-host egress of decoded waveforms through a ring of pinned step buffers.

A decode step's waveform (B rows of samples) leaves the GPU as one transfer: the rows are packed
on the device (float32, or signed 16-bit PCM encoded by ``omni_waveform_egress``, half the bytes
over PCIe), copied asynchronously on the decode stream into a pinned host buffer, and handed to
the caller as owned numpy rows once that copy has completed. It replaces the per-request pinned
staging of the reference scheduler (sglang_omni/models/qwen3_omni/components/
code2wav_scheduler.py:756-928), which copies each request's window on its own.

The host side is a ring of ``depth`` entries, each a pinned buffer and one HIP event. Step n
(counted from 0) travels through entry n % depth, so at most ``depth`` steps are in flight and
they complete in step order: before step n reuses its entry, step n - depth, the oldest one still
pending, is delivered (its event waited for), and every step older than that was delivered
before it. An entry's buffer grows only while the entry holds no transfer.

A transfer that fails part-way leaves its buffer possibly still targeted by a copy that no event
fences: that buffer is set aside for the life of the egress (never reused, never freed early) and
every later step is copied synchronously. Audio of older steps delivered while staging the failed
step is kept and returned by the next ``poll`` or ``flush``. ``depth = 0`` copies every step
synchronously.
"""

from __future__ import annotations

import time
from collections.abc import Hashable, Sequence
from dataclasses import dataclass, field

import numpy as np
import torch

from ..kernels.egress import FORMATS, waveform_egress


@dataclass
class _Entry:
    """One ring entry: its pinned buffer, its event, and the step it carries (None when free)."""

    host: torch.Tensor | None = None
    event: torch.cuda.Event | None = None
    step: int | None = None
    request_ids: list[Hashable] = field(default_factory=list)
    width: int = 0  # elements per row in `host`
    counts: list[int] = field(default_factory=list)  # samples kept per row


class WaveformEgress:
    """Stages decode steps' waveforms (B, 1, samples) or (B, samples) toward the host and returns
    each row's audio as an owned numpy array (float32, or int16 for ``format="pcm16"``), in step
    order, once its copy has completed."""

    def __init__(self, device: torch.device | str, *, format: str = "f32", depth: int = 4,
                 min_samples: int = 0) -> None:
        if format not in FORMATS:
            raise ValueError(f"format must be one of {sorted(FORMATS)}; got {format!r}")
        if depth < 0:
            raise ValueError(f"depth is a count of ring entries, not {depth}")
        device = torch.device(device)
        if device.type != "cuda":
            raise ValueError(f"waveform egress copies from a GPU, not {device}")
        self.device = torch.device("cuda", device.index if device.index is not None
                                   else torch.cuda.current_device())
        self.format = format
        self.dtype = FORMATS[format][1]
        self.min_samples = min_samples
        self.ring = [_Entry() for _ in range(depth)]
        self.steps = 0  # steps staged so far; the next one is number `steps`
        self.delivered = 0  # steps delivered so far (they leave in step order)
        self.overlapped = depth > 0  # False once a transfer failed: synchronous from then on
        self.set_aside: list[torch.Tensor] = []  # buffers a failed transfer may still target
        # audio delivered while staging a step whose transfer then failed: returned first by the
        # next poll / flush
        self.carried: list[tuple[Hashable, np.ndarray]] = []
        self.wait_ns = 0  # host time spent waiting for copies

    @property
    def in_flight(self) -> int:
        return self.steps - self.delivered

    # ------------------------------------------------------------------ staging

    def stage_step(self, request_ids: Sequence[Hashable], waveform: torch.Tensor,
                   row_samples: Sequence[int] | None = None) -> list[tuple[Hashable, np.ndarray]]:
        """Start the transfer of one decode step, row r belonging to request_ids[r] and keeping
        its first row_samples[r] samples (all by default). Returns the audio delivered now: the
        step that had to leave to free this step's ring entry, and this step itself when it was
        copied synchronously."""
        rows = waveform[:, 0] if waveform.dim() == 3 else waveform
        if rows.dim() != 2 or rows.shape[0] != len(request_ids):
            raise ValueError(f"{len(request_ids)} request ids for a waveform of shape "
                             f"{tuple(waveform.shape)}")
        batch, width = rows.shape
        counts = [width] * batch if row_samples is None else [int(n) for n in row_samples]
        if len(counts) != batch or min(counts, default=0) < 0 or max(counts, default=0) > width:
            raise ValueError(f"row_samples must keep between 0 and {width} samples of each of "
                             f"the {batch} rows")
        packed = self._packed(rows)
        ids = list(request_ids)
        step = self.steps
        if not self.overlapped:
            delivered = self.flush()  # carried audio and the steps still in flight leave first
            host = packed.cpu()
            self.steps += 1
            self.delivered += 1
            return delivered + self._rows(host, ids, width, counts)
        delivered: list[tuple[Hashable, np.ndarray]] = []
        entry = self.ring[step % len(self.ring)]
        if entry.step is not None:  # the oldest pending step still holds this entry
            delivered += self._deliver_through(entry.step)
        total = batch * width
        if entry.host is None or entry.host.numel() < total:
            entry.host = torch.empty(max(total, self.min_samples), dtype=self.dtype,
                                     pin_memory=True)
        try:
            entry.host[:total].view(batch, width).copy_(packed, non_blocking=True)
            if entry.event is None:
                entry.event = torch.cuda.Event(blocking=True)
            entry.event.record(torch.cuda.current_stream(self.device))
        except Exception:
            # no event fences whatever part of the copy was enqueued: keep the buffer alive and
            # out of the ring, and copy synchronously from now on; the older steps' audio
            # delivered above waits for the next poll / flush
            self.set_aside.append(entry.host)
            entry.host = None
            entry.event = None
            self.overlapped = False
            self.carried += delivered
            raise
        entry.step, entry.request_ids, entry.width, entry.counts = step, ids, width, counts
        self.steps += 1
        return delivered

    def _packed(self, rows: torch.Tensor) -> torch.Tensor:
        """The step in this egress's format as one contiguous (B, samples) device tensor: the
        waveform itself when it already is one, else the egress kernel's output."""
        if self.format == "f32" and rows.dtype == torch.float32 and rows.is_contiguous():
            return rows
        return waveform_egress(rows, format=self.format)

    # ------------------------------------------------------------------ delivery

    def poll(self) -> list[tuple[Hashable, np.ndarray]]:
        """The audio of the pending steps whose copies have completed, oldest first, without
        blocking (delivery stops at the first step still in flight)."""
        out, self.carried = self.carried, []
        while self.in_flight:
            entry = self._entry_of(self.delivered)
            if not entry.event.query():
                break
            out += self._deliver(entry)
        return out

    def flush(self) -> list[tuple[Hashable, np.ndarray]]:
        """The audio of every pending step, waiting for their copies."""
        out, self.carried = self.carried, []
        return out + (self._deliver_through(self.steps - 1) if self.in_flight else [])

    def _entry_of(self, step: int) -> _Entry:
        entry = self.ring[step % len(self.ring)]
        assert entry.step == step, "ring entries are delivered in step order"
        return entry

    def _deliver_through(self, step: int) -> list[tuple[Hashable, np.ndarray]]:
        out: list[tuple[Hashable, np.ndarray]] = []
        while self.delivered <= step:
            out += self._deliver(self._entry_of(self.delivered))
        return out

    def _deliver(self, entry: _Entry) -> list[tuple[Hashable, np.ndarray]]:
        start = time.monotonic_ns()
        entry.event.synchronize()
        self.wait_ns += time.monotonic_ns() - start
        audio = self._rows(entry.host, entry.request_ids, entry.width, entry.counts)
        entry.step = None
        entry.request_ids, entry.counts = [], []
        self.delivered += 1
        return audio

    @staticmethod
    def _rows(host: torch.Tensor, request_ids: list[Hashable], width: int,
              counts: list[int]) -> list[tuple[Hashable, np.ndarray]]:
        flat = host.reshape(-1).numpy()
        return [(rid, flat[r * width: r * width + n].copy())
                for r, (rid, n) in enumerate(zip(request_ids, counts))]


__all__ = ["WaveformEgress"]
