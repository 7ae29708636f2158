"""The serving step loop and the graph runner's failure policy on the host, with a causal fake
decoder and a fake graph backend whose capture and replay fail on demand (the reference's
FakeCudaGraphRunner approach, tests/unit_test/qwen3_omni/test_code2wav.py:83-106):

* a key whose capture raises, or whose replay differs from the eager decode, is rolled back and
  the other keys stay published (code2wav_cuda_graph.py:765-803);
* a replay that raises re-raises to the caller, drops every graph and leaves the runner eager
  with reason "disabled" (code2wav_cuda_graph.py:861-888,947-962);
* the step loop groups ready windows (first windows first, one length, capped at the largest
  published batch), keeps each stream's slot across replays, fails only a failing step's
  participants, decodes streams without a free slot from left context, and returns slots."""

from __future__ import annotations

import pytest
import torch

from sglang_omni_amd.models.dac_codec import CodecStatePool
from sglang_omni_amd.models.graph_runner import CodecGraphRunner, GraphKey
from sglang_omni_amd.scheduling.step_loop import CodecStepLoop

HOP = 3


class CausalFakeDecoder:
    """y[t, h] = 10 * code[t] + code[t - 1] + h: one frame of receptive field, its state (the
    last code) in the slot pool, zero before a stream starts."""

    device = torch.device("cpu")
    num_codebooks = 2
    frame_length = HOP

    def __init__(self):
        self.calls: list[tuple[int, int, bool]] = []

    def new_state_pool(self, num_slots, capture_slots=0):
        return CodecStatePool([("last", 1, 1)], num_slots=num_slots, capture_slots=capture_slots,
                              device=self.device)

    def _decode(self, codes, prev):
        c = codes[:, 0].float()  # [B, T]
        shifted = torch.cat([prev[:, None], c[:, :-1]], dim=1)
        y = 10 * c + shifted
        return (y[..., None] + torch.arange(HOP)).reshape(codes.shape[0], 1, -1)

    def decode_slots(self, codes, pool, slot_index, *, first_decode):
        self.calls.append((codes.shape[0], codes.shape[2], first_decode))
        hist = pool.histories["last"]
        prev = torch.zeros(codes.shape[0]) if first_decode else hist[slot_index, 0, 0, 0].float()
        out = self._decode(codes, prev)
        hist[slot_index, 0, 0, 0] = codes[:, 0, -1].to(hist.dtype)
        return out

    def from_indices(self, codes):
        return self._decode(codes, torch.zeros(codes.shape[0]))


class FakeGraph:
    def __init__(self, fn, out):
        self.fn, self.out = fn, out


class FakeBackend:
    def __init__(self, *, capture_error_for=None, mismatch_for=None):
        self.capture_error_for = capture_error_for or set()
        self.mismatch_for = mismatch_for or set()
        self.replay_error: Exception | None = None
        self.released = False

    def capture(self, fn, warmup):
        for _ in range(warmup):
            fn()
        out = fn()
        shape = tuple(out.shape)
        if shape in self.capture_error_for:
            raise RuntimeError("capture refused")
        return FakeGraph(fn, out), out

    def replay(self, graph):
        if self.replay_error is not None:
            raise self.replay_error
        graph.out.copy_(graph.fn() + (1 if tuple(graph.out.shape) in self.mismatch_for else 0))

    def release(self):
        self.released = True


def make(keys, backend, slots=4, capture_slots=2):
    dec = CausalFakeDecoder()
    pool = dec.new_state_pool(slots, capture_slots)
    return dec, pool, CodecGraphRunner(dec, pool, keys, backend=backend)


def test_a_failed_capture_rolls_back_its_key_and_keeps_the_others():
    keys = [GraphKey(2, 4, "first"), GraphKey(2, 4, "next"), GraphKey(1, 4, "next")]
    backend = FakeBackend(capture_error_for={(1, 1, 4 * HOP)})
    dec, pool, runner = make(keys, backend)
    failed = runner.capture_all()
    assert set(failed) == {GraphKey(1, 4, "next")} and "capture_failed" in failed[GraphKey(1, 4, "next")]
    assert set(runner.graphs) == {GraphKey(2, 4, "first"), GraphKey(2, 4, "next")}
    assert runner.enabled and runner.available_batch_sizes(4, "next") == (2,)
    assert torch.equal(pool.histories["last"][4:], torch.zeros(2, 2, 1, 1, dtype=torch.bfloat16))
    codes = torch.randint(0, 9, (1, 2, 4))
    res = runner.run(codes, torch.tensor([1]), first_decode=False)
    assert not res.graph and res.fallback_reason == "key_miss"


def test_a_replay_that_differs_is_not_published():
    backend = FakeBackend(mismatch_for={(2, 1, 4 * HOP)})
    _, _, runner = make([GraphKey(2, 4, "first")], backend)
    failed = runner.capture_all()
    assert "equivalence_failed" in failed[GraphKey(2, 4, "first")] and not runner.graphs


def test_a_replay_failure_disables_every_graph_and_reraises():
    keys = [GraphKey(2, 4, "first"), GraphKey(2, 4, "next")]
    backend = FakeBackend()
    dec, pool, runner = make(keys, backend)
    runner.capture_all()
    codes = torch.randint(0, 9, (2, 2, 4))
    idx = torch.tensor([0, 1])
    assert runner.run(codes, idx, first_decode=True).graph
    backend.replay_error = RuntimeError("replay failed")
    with pytest.raises(RuntimeError, match="replay failed"):
        runner.run(codes, idx, first_decode=False)
    assert not runner.enabled and not runner.graphs and backend.released
    assert runner.disable_reason.startswith("runtime_replay_failed")
    res = runner.run(codes, idx, first_decode=False)
    assert not res.graph and res.fallback_reason == "disabled"
    stats = runner.stats()
    assert stats["runtime"]["replay_failures"] == 1 and stats["runtime"]["graph_replays"] == 1
    assert stats["runtime"]["fallback_counts"] == {"disabled": 1}


def codes_for(n, seed):
    return torch.randint(1, 9, (2, n), generator=torch.Generator().manual_seed(seed))


def drain(loop, limit=50):
    audio, failures = {}, []
    for _ in range(limit):
        got, failed = loop.run_ready_step()
        failures += failed
        for rid, a in got:
            audio.setdefault(rid, []).append(a)
        if not loop.ready_group():
            break
    for rid, a in loop.flush():
        audio.setdefault(rid, []).append(a)
    return {rid: torch.cat([torch.as_tensor(x) for x in parts]) for rid, parts in audio.items()}, failures


def whole(dec, codes):
    return dec.from_indices(codes[None]).reshape(-1)


def test_streams_keep_their_slots_across_replays_and_equal_their_whole_decode():
    keys = [GraphKey(2, 3, "first"), GraphKey(2, 3, "next")]
    dec, pool, runner = make(keys, FakeBackend(), slots=3)
    runner.capture_all()
    loop = CodecStepLoop(dec, pool, window_frames=3, runner=runner)
    a, b = codes_for(8, 1), codes_for(8, 2)
    for start in (0, 3, 6):
        loop.push("a", a[:, start:start + 3])
        loop.push("b", b[:, start:start + 3])
        if start == 6:
            loop.finish("a")
            loop.finish("b")
    audio, failures = drain(loop)
    assert not failures
    assert torch.equal(audio["a"], whole(dec, a)) and torch.equal(audio["b"], whole(dec, b))
    assert runner.stats()["runtime"]["graph_replays"] == 2  # two full windows; the tail is eager
    assert pool.available_size() == 3 and not loop.streams


def test_first_windows_go_first_and_groups_cap_at_the_published_batch():
    keys = [GraphKey(2, 3, "first"), GraphKey(2, 3, "next")]
    dec, pool, runner = make(keys, FakeBackend(), slots=5, capture_slots=2)
    runner.capture_all()
    dec.calls.clear()
    t = iter(range(100))
    loop = CodecStepLoop(dec, pool, window_frames=3, runner=runner, clock=lambda: next(t))
    for rid in ("old0", "old1", "old2"):
        loop.push(rid, codes_for(3, 3))
    loop.run_ready_step()  # two first windows (the published batch), oldest first
    assert [c[:2] for c in dec.calls] == [(2, 3)]
    for rid in ("old0", "old1"):
        loop.push(rid, codes_for(3, 4))
    loop.push("new", codes_for(3, 5))
    group = loop.ready_group()
    assert [s.request_id for s in group] == ["old2", "new"]  # first windows before later ones
    assert all(s.emitted == 0 for s in group)


def test_a_failing_step_fails_its_participants_only():
    keys = [GraphKey(1, 3, "first"), GraphKey(1, 3, "next")]
    backend = FakeBackend()
    dec, pool, runner = make(keys, backend, slots=3, capture_slots=1)
    runner.capture_all()
    t = iter(range(100))
    loop = CodecStepLoop(dec, pool, window_frames=3, runner=runner, clock=lambda: next(t))
    loop.push("x", codes_for(3, 6))
    loop.push("y", codes_for(3, 7))
    backend.replay_error = RuntimeError("replay failed")
    _, failures = loop.run_ready_step()
    assert [rid for rid, _ in failures] == ["x"] and isinstance(failures[0][1], RuntimeError)
    assert "x" not in loop.streams and not runner.enabled
    assert pool.available_size() == 2  # x's slot is back
    audio, failures = drain(loop)  # y continues, eagerly
    assert not failures and set(audio) == {"y"}


def test_a_stream_without_a_free_slot_decodes_from_left_context():
    dec = CausalFakeDecoder()
    pool = dec.new_state_pool(1)
    loop = CodecStepLoop(dec, pool, window_frames=3, context_frames=2)
    a, b = codes_for(7, 8), codes_for(7, 9)
    loop.push("a", a)
    loop.push("b", b)  # the pool's only slot went to "a"
    assert loop.streams["b"].windowed
    loop.finish("a")
    loop.finish("b")
    audio, failures = drain(loop)
    assert not failures
    assert torch.equal(audio["a"], whole(dec, a)) and torch.equal(audio["b"], whole(dec, b))
    assert pool.available_size() == 1


def test_abort_returns_the_slot_zeroed():
    dec = CausalFakeDecoder()
    pool = dec.new_state_pool(1)
    loop = CodecStepLoop(dec, pool, window_frames=2)
    loop.push("r", codes_for(2, 10))
    loop.run_ready_step()
    assert pool.available_size() == 0 and pool.histories["last"].abs().sum() > 0
    loop.abort("r")
    assert pool.available_size() == 1 and pool.histories["last"].abs().sum() == 0
