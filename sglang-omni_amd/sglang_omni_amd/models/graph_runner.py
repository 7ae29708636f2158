"""HIP-graph replay of streaming decode steps.

A decode step of ``DacCodecDecoder.decode_slots`` is ~26 kernel launches whose shapes depend only
on (rows, frames) and whose history mode depends on whether the rows start their streams. The
runner captures one HIP graph per ``GraphKey(batch_size, frames, decode)`` with ``decode`` in
{"first", "next"}, over a static codes buffer and a static slot-index buffer, and replays it with
the caller's codes and slots copied in; keys without a graph run eagerly. It mirrors the slot
decode half of ``Code2WavDeviceGraphRunner``
(sglang_omni/models/qwen3_omni/components/code2wav_cuda_graph.py:673-763,812-830):

* capture on a side stream after warm-up decodes, into one shared graph memory pool;
* the capture-time decodes read and write the pool's scratch slots (``capture_slots`` of
  ``CodecStatePool``), never a stream's slots, and both the eager reference decode and the
  verifying replay start from zeroed scratch slots;
* a graph is published only if its replay equals the eager decode bit for bit (and is finite);
* the runner belongs to the process that built it (a forked child must build its own).

Replays launch on the caller's current stream; the returned waveform is the graph's static
output, valid until the next replay of the same key.
"""

from __future__ import annotations

import os
from dataclasses import dataclass

import torch

from .dac_codec import CodecStatePool, DacCodecDecoder


@dataclass(frozen=True)
class GraphKey:
    batch_size: int
    frames: int
    decode: str  # "first": the rows start their streams (cold history); "next": they continue


class GraphBuildError(RuntimeError):
    """A captured graph's replay differed from the eager decode, or capture failed."""


@dataclass
class _Captured:
    graph: torch.cuda.CUDAGraph
    codes: torch.Tensor  # static input [B, Q, T]
    index: torch.Tensor  # static slot index [B]
    out: torch.Tensor  # static output [B, 1, T * hop]


class CodecGraphRunner:
    WARMUP_ITERATIONS = 2

    def __init__(self, decoder: DacCodecDecoder, pool: CodecStatePool, keys: list[GraphKey]):
        if decoder.device.type != "cuda":
            raise ValueError("graph capture needs the decoder on a GPU")
        for key in keys:
            if key.decode not in ("first", "next"):
                raise ValueError(f"decode must be 'first' or 'next', got {key.decode!r}")
            if key.batch_size < 1 or key.frames < 1:
                raise ValueError(f"empty graph key {key}")
            if key.batch_size > len(pool.scratch_slots):
                raise ValueError(f"{key} needs {key.batch_size} scratch slots; the pool has "
                                 f"{len(pool.scratch_slots)} (CodecStatePool capture_slots)")
        self.decoder = decoder
        self.pool = pool
        self.keys = list(dict.fromkeys(keys))
        self.graphs: dict[GraphKey, _Captured] = {}
        self.owner_pid = os.getpid()
        self.mempool = None
        self.stream: torch.cuda.Stream | None = None

    # ------------------------------------------------------------------ capture

    def capture_all(self) -> None:
        """Capture every key, largest first (they share one memory pool)."""
        order = sorted(self.keys, key=lambda k: (k.batch_size, k.frames), reverse=True)
        for key in order:
            self.graphs[key] = self._capture(key)

    def _scratch_index(self, batch: int) -> torch.Tensor:
        return torch.tensor(self.pool.scratch_slots[:batch], dtype=torch.long,
                            device=self.decoder.device)

    def _capture(self, key: GraphKey) -> _Captured:
        dec = self.decoder
        dev = dec.device
        first = key.decode == "first"
        n_books = dec.num_codebooks
        codes = torch.zeros(key.batch_size, n_books, key.frames, dtype=torch.long, device=dev)
        index = self._scratch_index(key.batch_size)

        def step() -> torch.Tensor:
            return dec.decode_slots(codes, self.pool, index, first_decode=first)

        if self.stream is None:
            self.stream = torch.cuda.Stream(device=dev)
        if self.mempool is None:
            self.mempool = torch.cuda.graph_pool_handle()
        self.stream.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(self.stream):
            for _ in range(self.WARMUP_ITERATIONS):
                step()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, pool=self.mempool, stream=self.stream):
                out = step()
        torch.cuda.current_stream(dev).wait_stream(self.stream)
        # eager reference and verifying replay, both from zeroed scratch slots
        self.pool.zero_slots(index)
        eager = step().clone()
        self.pool.zero_slots(index)
        graph.replay()
        if not (out.shape == eager.shape and bool(torch.isfinite(out).all().item())
                and torch.equal(out, eager)):
            raise GraphBuildError(f"{key}: the graph's replay differs from the eager decode")
        self.pool.zero_slots(index)
        return _Captured(graph, codes, index, out)

    # ------------------------------------------------------------------ replay

    def run(self, codes: torch.Tensor, slot_index: torch.Tensor, *,
            first_decode: bool) -> tuple[torch.Tensor, bool]:
        """Decode one step: the graph of (rows, frames, first|next) if one was captured, else
        eagerly. Returns (waveform [B, 1, T * hop], whether a graph ran)."""
        if os.getpid() != self.owner_pid:
            raise RuntimeError(f"this graph runner belongs to PID {self.owner_pid}; rebuild it "
                               f"in PID {os.getpid()}")
        if codes.dim() != 3 or slot_index.dim() != 1 or slot_index.shape[0] != codes.shape[0]:
            raise ValueError("codes must be [B, Q, T] and slot_index [B]")
        key = GraphKey(int(codes.shape[0]), int(codes.shape[2]),
                       "first" if first_decode else "next")
        cap = self.graphs.get(key)
        if cap is None or codes.shape[1] != cap.codes.shape[1]:
            return self.decoder.decode_slots(codes, self.pool, slot_index,
                                             first_decode=first_decode), False
        cap.codes.copy_(codes, non_blocking=True)
        cap.index.copy_(slot_index, non_blocking=True)
        cap.graph.replay()
        return cap.out, True
