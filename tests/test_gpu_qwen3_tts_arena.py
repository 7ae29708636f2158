"""The Qwen3-TTS decoder under its streaming scheduler's state API, on the GPU: the slot arena
(``Qwen3TTSCodecStateArena``: acquire / release / retire / gather / scatter / stage_index /
describe, sglang_omni/models/qwen3_tts/codec_state_arena.py:50-333) and the tail decode
(``tail_frames`` / ``decode_tail``, qwen3_tts/incremental_codec.py:1085-1135), restating the
reference's tests (tests/unit_test/qwen3_tts/test_incremental_codec.py:668-842):

* an arena slot decoded chunk by chunk equals a private state's decodes (a fresh arena slot is
  zeroed, so its warm decode at position 0 is the cold decode), bit for bit;
* a cohort of one cold and two warm streams at different positions equals each stream decoded
  on its own, bit for bit (every kernel's summation order is independent of the batch);
* a tail decode of rows of three widths equals each row decoded whole in its last frame's
  samples, leaves the same state (the next decode agrees), and sits within the oracle bounds.
"""

from __future__ import annotations

import pytest
import torch

from oracle import qwen3_code2wav_oracle as Q
from sglang_omni_amd.models import (
    Qwen3TTSCodecDecoder,
    Qwen3TTSCodecStateArena,
    make_qwen3_code2wav_weights,
)

from .test_gpu_qwen3_code2wav import TTS_SMALL, _codes, check_waveform, effective_weights

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def tts(gpu):
    state = make_qwen3_code2wav_weights(TTS_SMALL, seed=2, branch_scale=0.5,
                                        activation_spread=0.1)
    return state, Qwen3TTSCodecDecoder(state, TTS_SMALL, device=gpu)


def arena_decode(dec, arena, slots, positions, codes):
    """One cohort decode as the reference's vocoder runs it: gather, decode, scatter."""
    state = arena.gather(slots)
    state.frame_positions = positions
    wave = dec.decode(codes, state)
    arena.scatter(slots, state)
    return wave


def test_arena_slot_lifecycle(tts, gpu):
    _, dec = tts
    arena = Qwen3TTSCodecStateArena(dec, num_slots=3, device=gpu, dtype=torch.float32)
    assert arena.describe() == {"slots": 3, "active_slots": 0,
                                "bytes_per_slot": arena.bytes_per_slot,
                                "total_bytes": 3 * arena.bytes_per_slot, "exhausted": 0}
    slots = [arena.acquire() for _ in range(3)]
    assert sorted(slots) == [0, 1, 2] and arena.acquire() is None and arena.exhausted_count == 1
    arena.release(slots[0])
    with pytest.raises(RuntimeError, match="released twice"):
        arena.release(slots[0])
    arena.retire(slots[1])
    arena.release(slots[1])  # a retired slot stays out
    assert arena.active_slots() == 1
    assert arena.acquire() == slots[0] and arena.acquire() is None
    index = arena.stage_index([2, 0])
    assert index.tolist() == [2, 0] and index.device == dec.device


def test_arena_backed_decode_matches_the_lazy_state(tts, gpu):
    _, dec = tts
    arena = Qwen3TTSCodecStateArena(dec, num_slots=4, device=gpu)
    codes = _codes(TTS_SMALL, 1, 11, 13).to(gpu)
    lazy = dec.init_state(1)
    # a slot left dirty by an earlier stream: acquire zeroes it
    dirty = arena.acquire()
    arena_decode(dec, arena, [dirty], [0], _codes(TTS_SMALL, 1, 5, 14).to(gpu))
    arena.release(dirty)
    slot = arena.acquire()
    assert slot == dirty
    offset = 0
    for length in (2, 1, 5, 3):
        chunk = codes[..., offset:offset + length]
        expected = dec.decode(chunk, lazy)
        actual = arena_decode(dec, arena, [slot], [offset], chunk)
        assert torch.equal(actual, expected), offset
        offset += length
    assert arena.gather([slot]).frame_positions.tolist() == [11]


def test_arena_cohort_matches_per_stream_decodes(tts, gpu):
    _, dec = tts
    arena = Qwen3TTSCodecStateArena(dec, num_slots=8, device=gpu)
    warmups = [0, 3, 9]
    fresh = 2
    streams = [_codes(TTS_SMALL, 1, w + fresh, 20 + w).to(gpu) for w in warmups]
    cohort, solo = [], []
    for stream, warmup in zip(streams, warmups):
        c, s = arena.acquire(), arena.acquire()
        cohort.append(c)
        solo.append(s)
        for i in range(warmup):
            for slot in (c, s):
                arena_decode(dec, arena, [slot], [i], stream[..., i:i + 1])
    expected = [arena_decode(dec, arena, [s], [w], stream[..., w:])
                for s, w, stream in zip(solo, warmups, streams)]
    batched = arena_decode(dec, arena, cohort, warmups,
                           torch.cat([stream[..., w:] for stream, w in zip(streams, warmups)]))
    assert batched.shape[0] == 3
    for row, single in enumerate(expected):
        assert torch.equal(batched[row:row + 1], single), row
    assert arena.gather(cohort).frame_positions.tolist() == [w + fresh for w in warmups]


def test_a_private_state_scatters_into_arena_slots(tts, gpu):
    """scatter of a state that lives elsewhere (init_state) copies its rows into the slots: the
    slots then continue the stream as the private state does."""
    _, dec = tts
    arena = Qwen3TTSCodecStateArena(dec, num_slots=3, device=gpu)
    codes = _codes(TTS_SMALL, 2, 9, 30).to(gpu)
    private = dec.init_state(2)
    dec.decode(codes[..., :6], private)
    slots = [arena.acquire(), arena.acquire()]
    arena.scatter(slots, private)
    expected = dec.decode(codes[..., 6:], private)
    got = arena_decode(dec, arena, slots, [6, 6], codes[..., 6:])
    assert torch.equal(got, expected)


def test_tail_decode_matches_each_row_decoded_whole(tts, gpu):
    state, dec = tts
    arena = Qwen3TTSCodecStateArena(dec, num_slots=6, device=gpu)
    emit = 1
    tail = dec.tail_frames(emit)
    widths = [tail + 7, tail + 3, tail]
    codes_cpu = _codes(TTS_SMALL, 3, max(widths), 42)
    codes = codes_cpu.to(gpu)
    tail_slots = [arena.acquire() for _ in widths]
    alone_slots = [arena.acquire() for _ in widths]
    st = arena.gather(tail_slots)
    wave = dec.decode_tail(codes, torch.tensor(widths), st, emit)
    arena.scatter(tail_slots, st)
    samples = emit * TTS_SMALL.hop_length
    assert wave.shape == (3, 1, samples)
    follow = _codes(TTS_SMALL, 1, 2, 43).to(gpu)
    for row, (w, ts, al) in enumerate(zip(widths, tail_slots, alone_slots)):
        whole = arena_decode(dec, arena, [al], [0], codes[row:row + 1, :, :w])
        assert torch.equal(wave[row:row + 1], whole[..., -samples:]), row
        assert arena.gather([ts]).frame_positions.tolist() == [w]
        # the state the tail decode left continues the stream as the whole decode's does
        assert torch.equal(arena_decode(dec, arena, [ts], [w], follow),
                           arena_decode(dec, arena, [al], [w], follow)), row
    # one row against the oracle's whole-stream decode
    with torch.no_grad():
        ref = Q.qwen3_tts_decode(codes_cpu[:1, :, :widths[0]], effective_weights(state),
                                 TTS_SMALL)
    check_waveform(wave[:1], ref[..., -samples:])


def test_tail_decode_contract(tts, gpu):
    _, dec = tts
    codes = _codes(TTS_SMALL, 1, 30, 50).to(gpu)
    with pytest.raises(ValueError, match="per-row frame positions"):
        dec.decode_tail(codes, torch.tensor([30]), dec.init_state(1), 1)
    arena = Qwen3TTSCodecStateArena(dec, num_slots=1, device=gpu)
    st = arena.gather([arena.acquire()])
    with pytest.raises(ValueError, match="tail_frames"):
        dec.decode_tail(codes, torch.tensor([dec.tail_frames(1) - 1]), st, 1)
