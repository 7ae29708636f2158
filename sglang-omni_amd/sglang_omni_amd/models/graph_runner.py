"""HIP-graph replay of streaming decode steps, with the build and runtime failure policy of the
reference's graph runner (sglang_omni/models/qwen3_omni/components/code2wav_cuda_graph.py:
673-763 capture and verification, 765-803 build rollback, 806-962 replay and runtime disable).

A decode step of ``DacCodecDecoder.decode_slots`` is ~26 kernel launches whose shapes depend only
on (rows, frames) and whose history mode depends on whether the rows start their streams. The
runner captures one graph per ``GraphKey(batch_size, frames, decode)`` with ``decode`` in
{"first", "next"} over a static codes buffer and a static slot-index buffer, and replays it with
the caller's codes and slots copied in:

* capture on a side stream after warm-up decodes, into one shared graph memory pool, largest keys
  first; the capture-time decodes use the pool's scratch slots (``capture_slots``), never a
  stream's, and the eager reference decode and the verifying replay both start from zeroed
  scratch slots;
* a key is published only if its replay equals the eager decode bit for bit and is finite. A key
  whose capture raises or whose replay differs is rolled back (its graph dropped, its scratch
  slots zeroed, the reason kept in ``failed_keys``) and the build goes on with the other keys;
* a replay that raises disables the runner: every graph is dropped, ``disable_reason`` records
  why, the error is re-raised to the caller (no eager retry of the failed step), and every later
  step runs eagerly with fallback reason "disabled";
* the runner belongs to the process that built it (a forked child must build its own).

Replays launch on the caller's current stream; the returned waveform is the graph's static
output, valid until the next replay of the same key (callers consume it first, e.g. by staging it
to the host on the same stream).

The graph operations go through a small backend (capture a function into a graph, replay it), so
the failure paths can be exercised on the host with a backend that raises on demand.
"""

from __future__ import annotations

import collections
import gc
import logging
import os
from dataclasses import dataclass, field
from typing import Any, Callable, Protocol

import torch

logger = logging.getLogger(__name__)


@dataclass(frozen=True)
class GraphKey:
    batch_size: int
    frames: int
    decode: str  # "first": the rows start their streams (cold history); "next": they continue


class GraphBuildError(RuntimeError):
    """A captured graph's replay differed from the eager decode."""


class GraphBackend(Protocol):
    def capture(self, fn: Callable[[], torch.Tensor], warmup: int) -> tuple[Any, torch.Tensor]:
        """Run fn `warmup` times, then capture one call of it: (graph, its static output)."""

    def replay(self, graph: Any) -> None: ...

    def release(self) -> None:
        """Drop the backend's shared graph resources (memory pool, capture stream)."""


class HipGraphBackend:
    """torch's HIP graphs: capture on a side stream into one shared memory pool."""

    def __init__(self, device: torch.device):
        self.device = device
        self.stream: torch.cuda.Stream | None = None
        self.mempool = None

    def capture(self, fn: Callable[[], torch.Tensor], warmup: int) -> tuple[Any, torch.Tensor]:
        if self.stream is None:
            self.stream = torch.cuda.Stream(device=self.device)
        if self.mempool is None:
            self.mempool = torch.cuda.graph_pool_handle()
        current = torch.cuda.current_stream(self.device)
        self.stream.wait_stream(current)
        try:
            with torch.cuda.stream(self.stream):
                for _ in range(warmup):
                    fn()
                graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(graph, pool=self.mempool, stream=self.stream):
                    out = fn()
        finally:
            current.wait_stream(self.stream)
        return graph, out

    def replay(self, graph: Any) -> None:
        graph.replay()

    def release(self) -> None:
        self.stream = None
        self.mempool = None


@dataclass
class _Captured:
    graph: Any
    codes: torch.Tensor  # static input [B, Q, T]
    index: torch.Tensor  # static slot index [B]
    out: torch.Tensor  # static output [B, 1, T * hop]


@dataclass
class RunResult:
    """A step's waveform, whether a graph produced it, its key and, for an eager step, why."""

    output: torch.Tensor
    graph: bool
    key: GraphKey | None
    fallback_reason: str | None


@dataclass
class _Stats:
    graph_replays: int = 0
    replay_failures: int = 0
    fallback_counts: collections.Counter = field(default_factory=collections.Counter)


class CodecGraphRunner:
    WARMUP_ITERATIONS = 2

    def __init__(self, decoder, pool, keys: list[GraphKey], *,
                 backend: GraphBackend | None = None):
        for key in keys:
            if key.decode not in ("first", "next"):
                raise ValueError(f"decode must be 'first' or 'next', got {key.decode!r}")
            if key.batch_size < 1 or key.frames < 1:
                raise ValueError(f"empty graph key {key}")
            if key.batch_size > len(pool.scratch_slots):
                raise ValueError(f"{key} needs {key.batch_size} scratch slots; the pool has "
                                 f"{len(pool.scratch_slots)} (CodecStatePool capture_slots)")
        if backend is None:
            if decoder.device.type != "cuda":
                raise ValueError("graph capture needs the decoder on a GPU")
            backend = HipGraphBackend(decoder.device)
        self.decoder = decoder
        self.pool = pool
        self.keys = list(dict.fromkeys(keys))
        self.backend = backend
        self.graphs: dict[GraphKey, _Captured] = {}
        self.failed_keys: dict[GraphKey, str] = {}
        self.enabled = True
        self.disable_reason: str | None = None
        self.owner_pid = os.getpid()
        self.runtime = _Stats()

    # ------------------------------------------------------------------ build

    def capture_all(self) -> dict[GraphKey, str]:
        """Capture every key, largest first (they share one memory pool); returns the keys that
        failed and why (those run eagerly; the others are published)."""
        order = sorted(self.keys, key=lambda k: (k.batch_size, k.frames), reverse=True)
        for key in order:
            if key in self.graphs:
                continue
            try:
                self.graphs[key] = self._capture(key)
            except Exception as exc:  # a key's failure rolls back that key only
                reason = str(exc) if isinstance(exc, GraphBuildError) else \
                    f"capture_failed: {type(exc).__name__}: {exc}"
                self.failed_keys[key] = reason
                self._zero_scratch(key.batch_size)
                logger.warning("graph for %s not published: %s", key, reason)
        return dict(self.failed_keys)

    build = capture_all

    def _scratch_index(self, batch: int) -> torch.Tensor:
        return torch.tensor(self.pool.scratch_slots[:batch], dtype=torch.long,
                            device=self.decoder.device)

    def _zero_scratch(self, batch: int) -> None:
        self.pool.zero_slots(self._scratch_index(batch))

    def _capture(self, key: GraphKey) -> _Captured:
        dec = self.decoder
        first = key.decode == "first"
        codes = torch.zeros(key.batch_size, dec.num_codebooks, key.frames, dtype=torch.long,
                            device=dec.device)
        index = self._scratch_index(key.batch_size)

        def step() -> torch.Tensor:
            return dec.decode_slots(codes, self.pool, index, first_decode=first)

        graph, out = self.backend.capture(step, self.WARMUP_ITERATIONS)
        # the eager reference and the verifying replay, both from zeroed scratch slots
        self.pool.zero_slots(index)
        eager = step().clone()
        self.pool.zero_slots(index)
        self.backend.replay(graph)
        ok = out.shape == eager.shape and bool(torch.isfinite(out).all()) and torch.equal(out, eager)
        self.pool.zero_slots(index)
        if not ok:
            raise GraphBuildError(f"equivalence_failed: {key}: the graph's replay differs from "
                                  "the eager decode")
        return _Captured(graph, codes, index, out)

    # ------------------------------------------------------------------ runtime

    def available_batch_sizes(self, frames: int, decode: str) -> tuple[int, ...]:
        """Rows of the published graphs for (frames, decode), largest first."""
        return tuple(sorted((k.batch_size for k in self.graphs
                             if k.frames == frames and k.decode == decode), reverse=True))

    def run(self, codes: torch.Tensor, slot_index: torch.Tensor, *,
            first_decode: bool) -> RunResult:
        """Decode one step: the graph of (rows, frames, first|next) when one is published,
        else eagerly (fallback reason "disabled" or "key_miss"). A replay that raises disables
        every graph and re-raises."""
        if os.getpid() != self.owner_pid:
            raise RuntimeError(f"this graph runner belongs to PID {self.owner_pid}; rebuild it "
                               f"in PID {os.getpid()}")
        if codes.dim() != 3 or slot_index.dim() != 1 or slot_index.shape[0] != codes.shape[0]:
            raise ValueError("codes must be [B, Q, T] and slot_index [B]")
        key = GraphKey(int(codes.shape[0]), int(codes.shape[2]),
                       "first" if first_decode else "next")
        if not self.enabled:
            return self._eager(codes, slot_index, first_decode, None, "disabled")
        cap = self.graphs.get(key)
        if cap is None or codes.shape[1] != cap.codes.shape[1]:
            return self._eager(codes, slot_index, first_decode, key, "key_miss")
        try:
            cap.codes.copy_(codes, non_blocking=True)
            cap.index.copy_(slot_index, non_blocking=True)
            self.backend.replay(cap.graph)
        except Exception as exc:
            self.runtime.replay_failures += 1
            self.disable(f"runtime_replay_failed: {type(exc).__name__}: {exc}")
            raise
        self.runtime.graph_replays += 1
        return RunResult(cap.out, True, key, None)

    def _eager(self, codes, slot_index, first_decode, key, reason) -> RunResult:
        self.runtime.fallback_counts[reason] += 1
        out = self.decoder.decode_slots(codes, self.pool, slot_index, first_decode=first_decode)
        return RunResult(out, False, key, reason)

    def disable(self, reason: str) -> None:
        """Drop every graph and run eagerly from now on."""
        self.graphs.clear()
        self.enabled = False
        self.disable_reason = reason
        self.backend.release()
        gc.collect()
        logger.warning("codec graph runner disabled: %s", reason)

    def stats(self) -> dict[str, Any]:
        return {
            "enabled": self.enabled,
            "disable_reason": self.disable_reason,
            "published": sorted((k.batch_size, k.frames, k.decode) for k in self.graphs),
            "failed": {f"b{k.batch_size}t{k.frames}{k.decode}": r
                       for k, r in self.failed_keys.items()},
            "runtime": {"graph_replays": self.runtime.graph_replays,
                        "replay_failures": self.runtime.replay_failures,
                        "fallback_counts": dict(self.runtime.fallback_counts)},
        }
