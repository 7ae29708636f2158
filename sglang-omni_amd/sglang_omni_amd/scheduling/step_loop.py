"""The serving loop around the codec decoder: streams of code frames in, waveform windows out,
one batched decode step at a time. It restates the window / step policy of the reference's
Code2Wav scheduler (sglang_omni/models/qwen3_omni/components/code2wav_scheduler.py:654-694,
1032-1100) for the slot decoders here:

* a stream takes a state slot with its first codes and gives it back (zeroed) when it ends or is
  aborted; when no slot is free it decodes each window from its codes with a left context of
  ``context_frames`` (a whole decode whose leading samples are dropped); a stream that ends
  before its first full window still holds its slot and decodes its remainder as that slot's
  first decode;
* a window is ``window_frames`` new frames, or a finished stream's remainder;
* a step decodes the windows of one group: first windows go before later ones (they carry their
  requests' time to first audio), then the longest-waiting window; the group is the ready windows
  of the same length, the same first|next state and the same slot mode as that one, oldest first,
  capped at the largest published graph batch that fits (or at ``max_rows`` without a runner);
* slot windows run through the graph runner (a graph of the group's key if published, else
  eagerly), their waveform staged toward the host in the same stream order, so a later replay
  cannot overwrite it first;
* a failing step fails its participants only: each gets the error, its slot is released, and the
  other streams continue (the runner disables its graphs itself when a replay raises);
* a step never waits for the GPU on the host: codes and slot ids go up from pinned memory
  without blocking, the slot ids are checked distinct on the host, and the waveform leaves
  through the egress ring (the host waits only for the step ``egress_depth`` steps older).
"""

from __future__ import annotations

import logging
import time
from collections.abc import Hashable
from dataclasses import dataclass, field
from typing import Any

import numpy as np
import torch

from .waveform_egress import WaveformEgress

logger = logging.getLogger(__name__)


@dataclass
class _Stream:
    request_id: Hashable
    slot: int | None
    frames: list[torch.Tensor] = field(default_factory=list)  # pending [Q, n] chunks
    pending: int = 0
    emitted: int = 0  # frames decoded so far
    history: torch.Tensor | None = None  # context frames for a stream without a slot
    finished: bool = False
    ready_since: float | None = None
    windowed: bool = False  # decodes with left context (no slot)


class CodecStepLoop:
    """Streams -> batched decode steps -> per-request waveform windows (numpy, float32)."""

    def __init__(self, decoder, pool, *, window_frames: int, context_frames: int = 0,
                 max_rows: int = 64, runner=None, egress_depth: int = 4,
                 clock=time.monotonic) -> None:
        if window_frames < 1 or max_rows < 1 or context_frames < 0:
            raise ValueError("window_frames and max_rows must be positive, context_frames >= 0")
        self.decoder = decoder
        self.pool = pool
        self.window_frames = window_frames
        self.context_frames = context_frames
        self.max_rows = max_rows
        self.runner = runner
        self.clock = clock
        self.hop = decoder.frame_length
        self.streams: dict[Hashable, _Stream] = {}
        self.egress = WaveformEgress(decoder.device, depth=egress_depth) \
            if decoder.device.type == "cuda" else None

    # ------------------------------------------------------------------ stream lifecycle

    def push(self, request_id: Hashable, codes: torch.Tensor) -> None:
        """Append code frames [Q, n] to a stream (opening it, and taking a slot, on its first
        codes)."""
        if codes.dim() != 2 or codes.shape[1] == 0:
            raise ValueError("codes are [Q, frames] with at least one frame")
        s = self.streams.get(request_id)
        if s is None:
            slot = self.pool.acquire()
            if slot is None:
                logger.warning("%s decodes with left context: the state pool is full", request_id)
            s = _Stream(request_id, slot, windowed=slot is None)
            self.streams[request_id] = s
        if s.finished:
            raise ValueError(f"{request_id} has finished")
        s.frames.append(codes)
        s.pending += int(codes.shape[1])
        self._mark_ready(s)

    def finish(self, request_id: Hashable) -> None:
        """No more codes will come: the stream's remainder becomes its last window."""
        s = self.streams[request_id]
        s.finished = True
        self._mark_ready(s)
        if s.pending == 0:
            self._close(s)

    def abort(self, request_id: Hashable) -> None:
        s = self.streams.pop(request_id, None)
        if s is not None and s.slot is not None:
            self._release(s.slot)

    def _close(self, s: _Stream) -> None:
        self.streams.pop(s.request_id, None)
        if s.slot is not None:
            self._release(s.slot)

    def _release(self, slot: int) -> None:
        self.pool.zero_slots(self.pool.stage_index([slot]))
        self.pool.release(slot)

    def _window(self, s: _Stream) -> int:
        """Frames of the stream's next window, 0 when none is ready."""
        if s.pending >= self.window_frames:
            return self.window_frames
        return s.pending if s.finished else 0

    def _context(self, s: _Stream) -> int:
        """Left-context frames a stream without a slot decodes its next window behind."""
        return min(self.context_frames, s.emitted) if s.windowed else 0

    def _mark_ready(self, s: _Stream) -> None:
        if self._window(s) and s.ready_since is None:
            s.ready_since = self.clock()

    # ------------------------------------------------------------------ grouping

    def ready_group(self) -> list[_Stream]:
        """The ready windows the next step decodes (see the module docstring)."""
        ready = [s for s in self.streams.values() if self._window(s)]
        if not ready:
            return []
        anchor = min(ready, key=lambda s: (s.emitted > 0, s.ready_since))
        frames = self._window(anchor)
        follows = anchor.emitted > 0
        group = sorted((s for s in ready if self._window(s) == frames
                        and (s.emitted > 0) == follows and s.windowed == anchor.windowed
                        and self._context(s) == self._context(anchor)),
                       key=lambda s: s.ready_since)
        if anchor.windowed or self.runner is None:
            rows = min(len(group), self.max_rows)
        else:
            sizes = self.runner.available_batch_sizes(frames, "next" if follows else "first")
            rows = next((n for n in sizes if n <= len(group)), min(len(group), self.max_rows))
        return group[:rows]

    # ------------------------------------------------------------------ stepping

    def _take(self, s: _Stream, n: int) -> torch.Tensor:
        codes = torch.cat(s.frames, dim=1) if len(s.frames) > 1 else s.frames[0]
        window, rest = codes[:, :n], codes[:, n:]
        s.frames = [rest] if rest.shape[1] else []
        s.pending -= n
        return window

    def run_ready_step(self) -> tuple[list[tuple[Hashable, np.ndarray]],
                                      list[tuple[Hashable, BaseException]]]:
        """Decode one group's windows. Returns the audio delivered (request id, samples) and
        the streams that failed in this step (request id, error)."""
        group = self.ready_group()
        if not group:
            return self._poll(), []
        frames = self._window(group[0])
        windows = [self._take(s, frames) for s in group]
        ids = [s.request_id for s in group]
        try:
            if group[0].windowed:
                wave = self._decode_windowed(group, windows)
            else:
                codes = self._to_device(torch.stack(windows))
                index = self.pool.stage_index([s.slot for s in group])
                first = group[0].emitted == 0
                if self.runner is not None:
                    wave = self.runner.run(codes, index, first_decode=first).output
                else:
                    wave = self.decoder.decode_slots(codes, self.pool, index, first_decode=first)
            delivered = self._stage(ids, wave)
        except Exception as exc:
            failures: list[tuple[Hashable, BaseException]] = []
            for s in group:
                self.abort(s.request_id)
                failures.append((s.request_id, exc))
            logger.warning("decode step failed for %s: %s", ids, exc)
            return self._poll(), failures
        for s in group:
            s.emitted += frames
            s.ready_since = None
            self._mark_ready(s)
            if s.finished and s.pending == 0:
                self._close(s)
        return delivered, []

    def _decode_windowed(self, group: list[_Stream], windows: list[torch.Tensor]) -> torch.Tensor:
        """Whole decodes of each window behind up to context_frames of its stream's earlier
        codes, keeping the window's samples (a group shares one context length)."""
        ctx = self._context(group[0])
        rows = []
        for s, w in zip(group, windows):
            past = s.history[:, s.history.shape[1] - ctx:] if ctx else w[:, :0]
            rows.append(torch.cat([past, w], dim=1))
            keep = torch.cat([s.history, w], dim=1) if s.history is not None else w
            s.history = keep[:, max(0, keep.shape[1] - self.context_frames):]
        codes = self._to_device(torch.stack(rows))
        wave = self.decoder.from_indices(codes)
        return wave[..., ctx * self.hop:]

    def _to_device(self, codes: torch.Tensor) -> torch.Tensor:
        """The step's codes on the decoder's device; host codes go up through pinned memory
        without blocking the host (the caching host allocator keeps the pinned block until the
        copy has completed)."""
        device = self.decoder.device
        if codes.device == device or device.type != "cuda":
            return codes.to(device)
        if codes.device.type == "cpu":
            codes = codes.pin_memory()
        return codes.to(device, non_blocking=True)

    def _stage(self, ids: list[Hashable], wave: torch.Tensor) -> list[tuple[Hashable, np.ndarray]]:
        if self.egress is None:
            rows = wave.reshape(len(ids), -1).float().cpu().numpy()
            return [(rid, rows[r].copy()) for r, rid in enumerate(ids)]
        return self.egress.stage_step(ids, wave) + self.egress.poll()

    def _poll(self) -> list[tuple[Hashable, np.ndarray]]:
        return [] if self.egress is None else self.egress.poll()

    def flush(self) -> list[tuple[Hashable, np.ndarray]]:
        """Every staged window still on its way to the host."""
        return [] if self.egress is None else self.egress.flush()

    def stats(self) -> dict[str, Any]:
        out: dict[str, Any] = {"streams": len(self.streams),
                               "free_slots": self.pool.available_size()}
        if self.runner is not None:
            out["runner"] = self.runner.stats()
        return out


__all__ = ["CodecStepLoop"]
