"""The benchmarked workloads at their full sizes: the decode paths the throughput figures time,
with the tile configurations those shapes select, against the float32 oracle of the reference's
vocoder path on the same seeded inputs.

Bounds (the decode path's stated tolerances): waveform max|err| <= 2e-3 with bf16 weights (5e-3
with fp8 weights) and SNR >= 40 dB against the oracle evaluated with the weights the decoder
multiplies by; the output RMS is asserted non-trivial so the bound means something. The oracle
runs on the host's cores, so each test checks a few rows of the batch against it and the whole
batch through size-independent properties (streamed == whole decode bit for bit, one row
decoded alone == the same row decoded in the batch).
"""

from __future__ import annotations

import pytest
import torch

from oracle import codec_oracle as O
from sglang_omni_amd.kernels.conv import recording_plans
from sglang_omni_amd.models import (
    DacCodecDecoder,
    HifiGanVocoder,
    make_dac_weights,
    make_hifigan_weights,
)
from sglang_omni_amd.models.configs import CODEC_24K, CODEC_24K_LONG, HIFIGAN_24K
from sglang_omni_amd.quantization import reference_weights

pytestmark = pytest.mark.gpu


def check_waveform(actual: torch.Tensor, expected: torch.Tensor, max_abs: float,
                   min_snr: float = 40.0) -> None:
    actual = actual.cpu()
    assert actual.shape == expected.shape
    err = (actual.double() - expected.double()).abs().max().item()
    snr = O.snr_db(expected, actual)
    rms = expected.double().pow(2).mean().sqrt().item()
    print(f"max|err| {err:.3e}  SNR {snr:.2f} dB  output rms {rms:.4f}", flush=True)
    assert rms > 0.005, "the reference output is too quiet for the tolerance to mean anything"
    assert err <= max_abs, err
    assert snr >= min_snr, snr


@pytest.fixture(scope="module")
def codec24k(gpu):
    weights = make_dac_weights(CODEC_24K, seed=0)
    return weights, DacCodecDecoder(weights, CODEC_24K, device=gpu)


def test_streaming_64_streams_of_12_frame_chunks(gpu, codec24k):
    """The streaming serving step: 64 streams on shuffled slots of an 80-slot pool, three
    12-frame chunks each. Every stream's chunks equal its whole decode bit for bit; four streams
    (first, last and two between) against the oracle's whole-stream decode."""
    weights, decoder = codec24k
    gen = torch.Generator().manual_seed(31)
    streams, chunk, n_chunks = 64, 12, 3
    codes = torch.randint(0, 2048, (streams, 16, chunk * n_chunks), generator=gen)
    pool = decoder.new_state_pool(num_slots=80)
    slot_index = torch.randperm(80, generator=gen)[:streams].to(gpu)
    codes_d = codes.to(gpu)
    with recording_plans() as plans:
        parts = [decoder.decode_slots(codes_d[..., s:s + chunk].contiguous(), pool, slot_index,
                                      first_decode=s == 0)
                 for s in range(0, chunk * n_chunks, chunk)]
    streamed = torch.cat(parts, -1)
    # the step runs the large LDS-DMA tiles (entry 1 of their lists) the small tests never pick
    names = {p.name for p in plans}
    print("tiles:", sorted(names), flush=True)
    assert "dma#1" in names
    whole = decoder.from_indices(codes_d)
    assert torch.equal(streamed, whole)
    rows = [0, 21, 42, 63]
    expected = O.dac_from_indices(codes[rows], reference_weights(weights, "bf16"))
    check_waveform(streamed[rows], expected, 2e-3)


def test_single_utterance_of_250_frames(gpu, codec24k):
    """One 20 s utterance (250 frames), decoded whole, against the oracle."""
    weights, decoder = codec24k
    gen = torch.Generator().manual_seed(32)
    codes = torch.randint(0, 2048, (1, 16, 250), generator=gen)
    out = decoder.from_indices(codes.to(gpu))
    expected = O.dac_from_indices(codes, reference_weights(weights, "bf16"))
    check_waveform(out, expected, 2e-3)


def test_hifigan_16_clips_of_500_mel_frames(gpu):
    """The HiFiGAN vocoder on 16 clips of 10 s (500 log-mel frames ~ N(-5, 2)): two clips
    against the oracle, and a clip decoded alone equals the same clip in the batch."""
    weights = make_hifigan_weights(HIFIGAN_24K, seed=0)
    vocoder = HifiGanVocoder(weights, HIFIGAN_24K, device=gpu)
    gen = torch.Generator().manual_seed(33)
    mel = torch.randn(16, 80, 500, generator=gen) * 2 - 5
    with recording_plans() as plans:
        out = vocoder(mel.to(gpu))
    print("tiles:", sorted({p.name for p in plans}), flush=True)
    alone = vocoder(mel[5:6].to(gpu))
    assert torch.equal(alone, out[5:6])
    rows = [0, 15]
    expected = O.hifigan_generator(mel[rows], reference_weights(weights, "bf16"))
    check_waveform(out[rows], expected, 2e-3)


def test_fp8_long_form_8_utterances_of_1500_frames(gpu):
    """The fp8-weight long form (32 x 1024 x 512 tables, E4M3 conv weights with per-output-channel
    scales): 8 utterances of 120 s, decoded in frame chunks through slot state; one utterance
    against the oracle with the dequantized weights (5e-3), and an utterance decoded alone equals
    the same utterance in the batch."""
    weights = make_dac_weights(CODEC_24K_LONG, seed=0)
    decoder = DacCodecDecoder(weights, CODEC_24K_LONG, device=gpu, weight_format="fp8")
    gen = torch.Generator().manual_seed(34)
    codes = torch.randint(0, 1024, (8, 32, 1500), generator=gen)
    with recording_plans() as plans:
        out = decoder.from_indices(codes.to(gpu))
    print("tiles:", sorted({p.name for p in plans}), flush=True)
    assert out.shape == (8, 1, 1500 * 1920)
    # alone, the row decodes in other frame chunks with other tile configurations: neither
    # changes a bit
    alone = decoder.from_indices(codes[3:4].to(gpu))
    assert torch.equal(alone, out[3:4])
    expected = O.dac_from_indices(codes[:1], reference_weights(weights, "fp8"))
    check_waveform(out[:1], expected, 5e-3)
