"""GPU parity of the waveform egress: the packing / PCM16 kernel against the oracle's encoding
bit for bit (aligned and unaligned rows, per-row sample counts, special values), and the pinned
staging of decode steps (WaveformEgress) against the waveform copied to the host, through slot
reuse, a full pool and the synchronous fallback."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import codec_oracle as O
from sglang_omni_amd import _native as N
from sglang_omni_amd.kernels.egress import waveform_egress
from sglang_omni_amd.scheduling import WaveformEgress

pytestmark = pytest.mark.gpu


def _wave(rows: int, samples: int, seed: int) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(rows, 1, samples, generator=g) * 0.6
    flat = w.view(-1)
    specials = torch.tensor([float("nan"), float("inf"), float("-inf"), 1.0, -1.0, 0.5, -0.5,
                             2.5, -3.0, 1e-6, -1e-6, 0.99999])
    flat[: min(flat.numel(), specials.numel())] = specials[: flat.numel()]
    return w


@pytest.mark.parametrize("fmt", ["f32", "pcm16"])
@pytest.mark.parametrize("rows,samples", [(64, 23040), (3, 1001), (1, 7), (5, 8)])
def test_egress_matches_the_oracle(gpu, fmt, rows, samples):
    w = _wave(rows, samples, rows * 31 + samples)
    out = waveform_egress(w.to(gpu), format=fmt).cpu()
    ref = O.waveform_egress_reference(w, format=fmt)
    for r in range(rows):
        if fmt == "f32":
            assert torch.equal(out[r].view(torch.int32), ref[r].view(torch.int32))  # NaN too
        else:
            assert torch.equal(out[r], ref[r])


@pytest.mark.parametrize("fmt", ["f32", "pcm16"])
def test_egress_unaligned_strided_rows_and_counts(gpu, fmt):
    """Rows inside a longer buffer at an odd offset (the element path) and a packed output with
    padding, rows cut short by row_samples; samples past a row's count stay untouched."""
    w = _wave(6, 1003, 5)
    big = torch.zeros(6, 1, 1010)
    big[:, :, 3:1006] = w
    dev = big.to(gpu)[:, 0, 3:1006]  # stride 1010, offset 3 floats
    counts = [1003, 0, 17, 1000, 8, 999]
    fill = -123 if fmt == "pcm16" else -123.0
    dtype = torch.int16 if fmt == "pcm16" else torch.float32
    out = torch.full((6, 1040), fill, dtype=dtype, device=gpu)
    waveform_egress(dev, format=fmt, out=out,
                    row_samples=torch.tensor(counts, dtype=torch.int64, device=gpu))
    out = out.cpu()
    ref = O.waveform_egress_reference(w, counts, format=fmt)
    for r, n in enumerate(counts):
        if fmt == "f32":
            assert torch.equal(out[r, :n].view(torch.int32), ref[r].view(torch.int32))
        else:
            assert torch.equal(out[r, :n], ref[r])
        assert (out[r, n:] == fill).all()


def test_egress_rejects_bad_arguments(gpu):
    w = torch.zeros(2, 1, 16, device=gpu)
    with pytest.raises(ValueError):
        waveform_egress(w, format="mulaw")
    with pytest.raises(ValueError):
        waveform_egress(w.double())
    with pytest.raises(ValueError):
        waveform_egress(w, out=torch.empty(2, 8, device=gpu))
    lib = N.load_library()
    assert lib.omni_waveform_egress(w.data_ptr(), 2, 16, 8, None, 0, w.data_ptr(), 16,
                                    N.stream_handle(w.device)) == N.INVALID_ARG
    assert lib.omni_waveform_egress(w.data_ptr(), 2, 16, 16, None, 9, w.data_ptr(), 16,
                                    N.stream_handle(w.device)) == N.INVALID_ARG


@pytest.mark.parametrize("fmt", ["f32", "pcm16"])
def test_waveform_egress_steps(gpu, fmt):
    """Eight decode steps through a two-entry ring: every row's audio equals the oracle's
    encoding of the waveform that step produced, in step order, whether it left by poll, to
    free its ring entry for a later step, or at the final flush."""
    egress = WaveformEgress(gpu, format=fmt, depth=2)
    expected: dict[str, np.ndarray] = {}
    got: dict[str, np.ndarray] = {}
    order: list[str] = []
    for step in range(8):
        rows = 4 if step % 2 else 3
        w = _wave(rows, 1920 * 12, 100 + step)
        ids = [f"s{step}r{r}" for r in range(rows)]
        counts = [1920 * 12 - 7 * r for r in range(rows)]
        ref = O.waveform_egress_reference(w, counts, format=fmt)
        expected.update({i: ref[r].numpy() for r, i in enumerate(ids)})
        for rid, audio in egress.stage_step(ids, w.to(gpu), counts) + egress.poll():
            got[rid] = audio
            order.append(rid)
    for rid, audio in egress.flush():
        got[rid] = audio
        order.append(rid)
    assert set(got) == set(expected)
    assert order == sorted(order, key=lambda k: (int(k[1:k.index("r")]), int(k[k.index("r") + 1:])))
    for rid, audio in got.items():
        assert audio.dtype == (np.int16 if fmt == "pcm16" else np.float32)
        assert np.array_equal(audio.view(np.int16 if fmt == "pcm16" else np.int32),
                              expected[rid].view(np.int16 if fmt == "pcm16" else np.int32))
    assert egress.in_flight == 0 and egress.steps == egress.delivered == 8
    assert all(e.host is None or e.host.is_pinned() for e in egress.ring)


def test_waveform_egress_without_a_ring_copies_synchronously(gpu):
    egress = WaveformEgress(gpu, depth=0)
    w = _wave(2, 100, 3)
    ready = egress.stage_step(["a", "b"], w.to(gpu))
    assert [rid for rid, _ in ready] == ["a", "b"] and egress.in_flight == 0
    assert np.array_equal(ready[1][1].view(np.int32), w[1, 0].numpy().view(np.int32))


def test_a_ring_entry_is_reused_only_after_its_step_left(gpu):
    """Step n waits for step n - depth: with depth 3 the fourth step's staging delivers the
    first, and the buffers grow only between transfers."""
    egress = WaveformEgress(gpu, depth=3)
    waves = [_wave(2, 64 * (k + 1), 10 + k) for k in range(4)]
    assert egress.stage_step(["a0", "b0"], waves[0].to(gpu)) == []
    egress.stage_step(["a1", "b1"], waves[1].to(gpu))
    egress.stage_step(["a2", "b2"], waves[2].to(gpu))
    assert egress.in_flight == 3
    out = egress.stage_step(["a3", "b3"], waves[3].to(gpu))  # entry 0 again: step 0 leaves
    assert [rid for rid, _ in out] == ["a0", "b0"]
    assert np.array_equal(out[0][1].view(np.int32), waves[0][0, 0].numpy().view(np.int32))
    rest = egress.flush()
    assert [rid for rid, _ in rest] == ["a1", "b1", "a2", "b2", "a3", "b3"]
    assert np.array_equal(rest[-1][1].view(np.int32), waves[3][1, 0].numpy().view(np.int32))
    assert egress.ring[0].host.numel() >= 2 * 64 * 4


def test_a_failed_transfer_sets_its_buffer_aside_and_goes_synchronous(gpu, monkeypatch):
    """The failure is forced on the host (the event record raises): the step's buffer is kept
    out of the ring for good, the steps already in flight still arrive in order, and later steps
    are copied synchronously."""
    egress = WaveformEgress(gpu, depth=2)
    w = [_wave(1, 80, 20 + k) for k in range(3)]
    egress.stage_step(["x"], w[0].to(gpu))
    real_event = torch.cuda.Event

    class FailingEvent:
        def __init__(self, *args, **kwargs):
            pass

        def record(self, stream=None):
            raise RuntimeError("record refused")

    monkeypatch.setattr(torch.cuda, "Event", FailingEvent)
    with pytest.raises(RuntimeError, match="record refused"):
        egress.stage_step(["y"], w[1].to(gpu))
    monkeypatch.setattr(torch.cuda, "Event", real_event)
    assert not egress.overlapped and len(egress.set_aside) == 1
    assert egress.ring[1].host is None
    out = egress.stage_step(["z"], w[2].to(gpu))
    assert [rid for rid, _ in out] == ["x", "z"]
    assert np.array_equal(out[1][1].view(np.int32), w[2][0, 0].numpy().view(np.int32))
    assert egress.in_flight == 0


def test_audio_delivered_before_a_failed_transfer_is_kept(gpu, monkeypatch):
    """With one ring entry, staging step 1 first delivers step 0; when step 1's transfer then
    fails (forced on the host: the entry's event refuses to record), step 0's audio is not
    lost: the next poll returns it."""
    egress = WaveformEgress(gpu, depth=1)
    w = [_wave(2, 96, 30 + k) for k in range(2)]
    assert egress.stage_step(["a0", "b0"], w[0].to(gpu)) == []

    def refuse(stream=None):
        raise RuntimeError("record refused")

    monkeypatch.setattr(egress.ring[0].event, "record", refuse)
    with pytest.raises(RuntimeError, match="record refused"):
        egress.stage_step(["a1", "b1"], w[1].to(gpu))
    out = egress.poll()
    assert [rid for rid, _ in out] == ["a0", "b0"]
    assert np.array_equal(out[1][1].view(np.int32), w[0][1, 0].numpy().view(np.int32))
    assert egress.poll() == [] and egress.flush() == []
