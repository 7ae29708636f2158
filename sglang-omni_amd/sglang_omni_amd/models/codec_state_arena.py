"""Slot-indexed, reusable storage of Qwen3-TTS incremental decoder state.

Mirrors the reference's ``Qwen3TTSCodecStateArena`` (sglang_omni/models/qwen3_tts/
codec_state_arena.py:50-333), the storage its streaming vocoder decodes cohorts from
(``arena.gather(slots)`` -> ``decoder.decode(codes, state)`` -> ``arena.scatter(slots, state)``,
qwen3_tts/streaming_vocoder.py:2084-2086), over the HIP decoder's slot pool:

* the arena is one ``Code2WavStatePool`` of ``num_slots`` slots plus a scratch slot: per slot the
  conv stack's histories (two parity copies), the transposed convs' contexts, the ConvNeXt
  depthwise histories, each layer's K / V ring and the slot's absolute frame position;
* ``gather`` hands back a state bound to the cohort's slots (a device index), not a copy: the
  decode reads and advances the arena in place, so ``scatter`` of that state has nothing to move
  (it still copies a state that lives elsewhere, e.g. one from ``init_state``, into the slots);
* ``acquire`` zeroes a slot before handing it out, so a reused slot is a cold start and cold and
  warm rows decode in one launch (a zero slot reads as a stream's start); ``release`` returns a
  slot without clearing it, after the work queued on the current stream, and ``retire`` withdraws
  a slot whose last decode could not be shown complete;
* ``stage_index`` copies a cohort's slot ids from pinned memory without a host sync.

The lock guards the free list, as the reference's does; decodes of one arena run on one stream.
"""

from __future__ import annotations

import threading
from collections.abc import Sequence
from typing import Any

import torch

from .qwen3_code2wav import Code2WavStatePool, Qwen3TTSCodecDecoder, Qwen3TTSCodecState


class Qwen3TTSCodecStateArena:
    """Bounded, reusable per-stream state of a ``Qwen3TTSCodecDecoder``. ``dtype`` is taken for
    the reference's signature; the HIP state keeps its own layout (bf16 histories, contexts and
    K / V, float32 depthwise histories). ``max_fresh_frames`` bounds the frames one decode of a
    row may take (its K / V ring holds the window and them)."""

    def __init__(self, decoder: Qwen3TTSCodecDecoder, *, num_slots: int,
                 device: torch.device | str | None = None, dtype: torch.dtype | None = None,
                 max_fresh_frames: int | None = None):
        if num_slots <= 0:
            raise ValueError("Qwen3-TTS codec state arena needs at least one slot")
        device = torch.device(device) if device is not None else decoder.device
        if device.type != decoder.device.type or device.index not in (None, decoder.device.index):
            raise ValueError(f"the arena's device {device} is not the decoder's {decoder.device}")
        device = decoder.device
        self.decoder = decoder
        self.device = device
        self.dtype = dtype
        self._num_slots = int(num_slots)
        self.scratch_slot = self._num_slots
        retained = decoder.config.sliding_window - 1
        extra = decoder.DEFAULT_RING_EXTRA if max_fresh_frames is None else int(max_fresh_frames)
        self.pool: Code2WavStatePool = decoder.new_state_pool(
            num_slots=self._num_slots, capture_slots=1, ring_frames=retained + extra)
        self.lock = threading.Lock()
        self.release_events: dict[int, Any] = {}
        self.free: list[int] = list(reversed(range(self._num_slots)))
        self.retired: set[int] = set()
        self._exhausted = 0

    # ------------------------------------------------------------------ sizes

    @property
    def num_slots(self) -> int:
        return self._num_slots

    @property
    def bytes_per_slot(self) -> int:
        return self.pool.bytes_per_slot

    @property
    def total_bytes(self) -> int:
        return self.bytes_per_slot * self._num_slots

    @property
    def exhausted_count(self) -> int:
        return self._exhausted

    def active_slots(self) -> int:
        with self.lock:
            return self._num_slots - len(self.free) - len(self.retired)

    def describe(self) -> dict[str, int]:
        return {"slots": self._num_slots, "active_slots": self.active_slots(),
                "bytes_per_slot": self.bytes_per_slot, "total_bytes": self.total_bytes,
                "exhausted": self._exhausted}

    # ------------------------------------------------------------------ slot lifecycle

    def acquire(self) -> int | None:
        """A zeroed slot, or None when every slot is taken."""
        with self.lock:
            if not self.free:
                self._exhausted += 1
                return None
            slot = self.free.pop()
            released = self.release_events.pop(slot, None)
        if released is not None:
            torch.cuda.current_stream(self.device).wait_event(released)
        self.zero_slot(slot)
        return slot

    def release(self, slot: int) -> None:
        """Give a slot back (not cleared: ``acquire`` clears it), after the work queued on the
        current stream. Releasing a free slot twice raises; a retired slot stays retired."""
        released = None
        if self.device.type == "cuda":
            released = torch.cuda.Event()
            released.record(torch.cuda.current_stream(self.device))
        with self.lock:
            if slot in self.retired:
                return
            if slot in self.free:
                raise RuntimeError(f"Qwen3-TTS codec state slot {slot} was released twice")
            if not 0 <= slot < self._num_slots:
                raise ValueError(f"slot {slot} is not one of the arena's {self._num_slots}")
            if released is not None:
                self.release_events[slot] = released
            self.free.append(slot)

    def retire(self, slot: int) -> None:
        """Withdraw a slot for the life of the arena (a decode that touched it could not be
        shown complete, so its memory is never handed to later work)."""
        with self.lock:
            self.retired.add(slot)
            self.release_events.pop(slot, None)
            if slot in self.free:
                self.free.remove(slot)

    def zero_slot(self, slot: int) -> None:
        """Clear the slot's state: histories, contexts, K / V, parity and frame position."""
        self.pool.zero_slots(self.stage_index([slot]))

    # ------------------------------------------------------------------ cohorts

    def stage_index(self, slots: Sequence[int]) -> torch.Tensor:
        """A cohort's slot ids on the device, copied from pinned memory without a host sync."""
        slots = [int(s) for s in slots]
        if not slots:
            raise ValueError("Qwen3-TTS codec state arena needs at least one slot")
        return self.pool.stage_index(slots)

    def gather(self, slots: Sequence[int]) -> Qwen3TTSCodecState:
        """The cohort's state: its rows bound to these slots of the arena (no copy)."""
        state = self.gather_by_index(self.stage_index(slots))
        state.slots = [int(s) for s in slots]
        return state

    def gather_by_index(self, index: torch.Tensor) -> Qwen3TTSCodecState:
        """The state of the slots a device index names (capturable with a static index)."""
        if index.dim() != 1 or index.dtype != torch.int64 or index.device != self.device:
            raise ValueError("the index must be int64 [B] on the arena's device")
        return Qwen3TTSCodecState(self.pool, int(index.shape[0]), self.device,
                                  slot_index=index, per_row_positions=True)

    def scatter(self, slots: Sequence[int], state: Qwen3TTSCodecState) -> None:
        """Write an advanced cohort state back into its slots: nothing to move for a state
        gathered from these slots (it advanced in place); another state's rows are copied."""
        slots = [int(s) for s in slots]
        if state.pool is self.pool and getattr(state, "slots", None) == slots:
            return
        self.scatter_by_index(self.stage_index(slots), state)

    def scatter_by_index(self, index: torch.Tensor, state: Qwen3TTSCodecState) -> None:
        """Write a cohort state into the slots a device index names."""
        if int(index.shape[0]) != state.batch_size:
            raise RuntimeError(f"Qwen3-TTS codec state arena expected {state.batch_size} slots, "
                               f"got {int(index.shape[0])}")
        if state.pool is self.pool and index is state.slot_index:
            return
        src, dst = state.pool, self.pool
        if src.ring_frames != dst.ring_frames:
            raise RuntimeError(f"the state's K / V rings hold {src.ring_frames} frames, the "
                               f"arena's {dst.ring_frames}")
        rows = state.slot_index
        for name, buf in dst.histories.items():
            buf.index_copy_(0, index, src.histories[name].index_select(0, rows))
        dst.parity.index_copy_(0, index, src.parity.index_select(0, rows))
        for name, buf in dst.dw_histories.items():
            buf.index_copy_(0, index, src.dw_histories[name].index_select(0, rows))
        width = dst.ring_frames
        for a, b in zip((*dst.keys, *dst.values), (*src.keys, *src.values)):
            ra, rb = a.view(-1, width, a.shape[1]), b.view(-1, width, b.shape[1])
            ra.index_copy_(0, index, rb.index_select(0, rows))
        dst.frame_positions.index_copy_(0, index, src.frame_positions.index_select(0, rows))


__all__ = ["Qwen3TTSCodecStateArena"]
