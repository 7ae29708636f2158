"""Decoder-level GPU parity: the HIP decode path against the float32 oracle of the reference's
vocoder path on the same seeded inputs, and the streaming invariants of the reference's tests.

Tolerances (the decode path's stated bounds): waveform max|err| <= 2e-3 for bf16 weights (5e-3 for fp8
weights) and SNR >= 40 dB against the float32 oracle evaluated with the weights the decoder
multiplies by (bf16-rounded, or fp8-dequantized). Output RMS is asserted non-trivial so the
tolerance is not vacuous.
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from oracle import codec_oracle as O
from sglang_omni_amd.kernels.rvq import rvq_gather_sum
from sglang_omni_amd.models import (
    DacCodecDecoder,
    DacDecoderConfig,
    HifiGanVocoder,
    make_dac_weights,
    make_hifigan_weights,
)
from sglang_omni_amd.models.configs import CODEC_24K, CODEC_24K_LONG, HIFIGAN_24K
from sglang_omni_amd.quantization import reference_weights
from sglang_omni_amd.utils.channels_last_conv import channels_last_conv1d
from sglang_omni_amd.utils.snake_beta import snake1d

pytestmark = pytest.mark.gpu

TINY = DacDecoderConfig(n_codebooks=4, codebook_size=64, latent_dim=64, channels=128,
                        rates=(2, 4), conv_gain=0.85)
# 384 -> 192 -> 96 channels: both residual-unit stages run the fused (one-launch) unit kernel
TINY_FUSED = DacDecoderConfig(n_codebooks=4, codebook_size=64, latent_dim=64, channels=384,
                              rates=(2, 3), conv_gain=0.85)


def check_waveform(actual: torch.Tensor, expected: torch.Tensor, max_abs: float,
                   min_snr: float = 40.0) -> None:
    actual = actual.cpu()
    assert actual.shape == expected.shape
    err = (actual.double() - expected.double()).abs().max().item()
    snr = O.snr_db(expected, actual)
    rms = expected.double().pow(2).mean().sqrt().item()
    print(f"max|err| {err:.3e}  SNR {snr:.2f} dB  output rms {rms:.4f}")
    assert rms > 0.005, "the reference output is too quiet for the tolerance to mean anything"
    assert err <= max_abs, err
    assert snr >= min_snr, snr


@pytest.fixture(scope="module", params=[TINY, TINY_FUSED], ids=["unfused", "fused"])
def tiny(gpu, request):
    weights = make_dac_weights(request.param, seed=0)
    return weights, DacCodecDecoder(weights, request.param, device=gpu)


def test_single_conv_block_workload(gpu):
    """The fp32 single-block workload: RVQ (K=8, 1024 x 256 tables ~ N(0, 0.02), int32 codes,
    T=50) -> causal conv 256->256 k=7 -> Snake(alpha=1) -> + x, all in float32 on the GPU. The
    gather-sum is bit-exact; the conv is the direct-sum float32 kernel (the layer is fp32, so no
    bf16 operand is formed) and Snake the float32 kernel, held to float32-summation tolerance
    against the float32 oracle."""
    torch.manual_seed(0)
    tables = torch.randn(8, 1024, 256) * 0.02
    codes = torch.randint(0, 1024, (1, 8, 50), dtype=torch.int32)
    conv = torch.nn.Conv1d(256, 256, 7)
    w, b = conv.weight.detach(), conv.bias.detach()
    alpha = torch.ones(256)
    x_ref, y_ref = O.conv_block(codes, tables, w, b, alpha)
    x = rvq_gather_sum(codes.to(gpu), tables.to(gpu))  # [1, 50, 256] fp32
    assert torch.equal(x.cpu(), x_ref.transpose(1, 2))
    # the causal conv's input carries its left context (6 zero rows), as the reference's
    # channels-last API takes it
    padded = F.pad(x, (0, 0, 6, 0))
    c = channels_last_conv1d(padded, conv, w.to(gpu), b.to(gpu), 50)
    assert c.dtype == torch.float32 and c.shape == (1, 50, 256)
    y = x + snake1d(c, alpha.to(gpu))
    conv_ref = O.causal_conv1d(x_ref, w, b)
    scale = conv_ref.abs().max().item()
    torch.testing.assert_close(c.cpu().transpose(1, 2), conv_ref, rtol=1e-5, atol=1e-5 * scale)
    torch.testing.assert_close(y.cpu().transpose(1, 2), y_ref, rtol=1e-5, atol=1e-5 * scale)


def test_tiny_decoder_matches_the_oracle(gpu, tiny):
    weights, decoder = tiny
    gen = torch.Generator().manual_seed(1)
    codes = torch.randint(0, 64, (3, 4, 17), generator=gen)
    out = decoder.from_indices(codes.to(gpu))
    expected = O.dac_from_indices(codes, reference_weights(weights, "bf16"))
    check_waveform(out, expected, 2e-3)


@pytest.mark.parametrize("splits", [(4, 6, 7), (1,) * 17, (10, 7)])
def test_slot_decodes_in_any_split_equal_the_whole_decode_bitwise(gpu, tiny, splits):
    """Splits of tests/unit_test/qwen3_omni/test_code2wav.py:1170-1200; here the streamed waveform
    is bit-identical to the whole decode (same accumulation order per sample)."""
    weights, decoder = tiny
    gen = torch.Generator().manual_seed(2)
    codes = torch.randint(0, 64, (2, 4, sum(splits)), generator=gen).to(gpu)
    whole = decoder.from_indices(codes)
    pool = decoder.new_state_pool(num_slots=4)
    slot_index = torch.tensor([2, 0], device=gpu)
    parts, start = [], 0
    for i, n in enumerate(splits):
        parts.append(decoder.decode_slots(codes[..., start:start + n], pool, slot_index,
                                          first_decode=i == 0))
        start += n
    assert torch.equal(torch.cat(parts, dim=-1), whole)


def test_a_reused_slot_decodes_like_a_fresh_pool(gpu, tiny):
    """tests/unit_test/qwen3_omni/test_code2wav.py:1242-1257: a slot that held another stream
    decodes a new stream exactly as a fresh pool does."""
    weights, decoder = tiny
    gen = torch.Generator().manual_seed(3)
    old = torch.randint(0, 64, (1, 4, 9), generator=gen).to(gpu)
    new = torch.randint(0, 64, (1, 4, 8), generator=gen).to(gpu)
    used = decoder.new_state_pool(num_slots=2)
    idx = torch.tensor([1], device=gpu)
    decoder.decode_slots(old[..., :5], used, idx, first_decode=True)
    decoder.decode_slots(old[..., 5:], used, idx, first_decode=False)
    fresh = decoder.new_state_pool(num_slots=2)
    a = [decoder.decode_slots(new[..., :3], used, idx, first_decode=True),
         decoder.decode_slots(new[..., 3:], used, idx, first_decode=False)]
    b = [decoder.decode_slots(new[..., :3], fresh, idx, first_decode=True),
         decoder.decode_slots(new[..., 3:], fresh, idx, first_decode=False)]
    assert torch.equal(torch.cat(a, -1), torch.cat(b, -1))


def test_rows_at_different_positions_keep_their_streams(gpu, tiny):
    """tests/unit_test/qwen3_omni/test_code2wav.py:1262-1297: one batched step serves rows that
    are at different points of their streams."""
    weights, decoder = tiny
    gen = torch.Generator().manual_seed(4)
    a = torch.randint(0, 64, (1, 4, 10), generator=gen).to(gpu)
    b = torch.randint(0, 64, (1, 4, 6), generator=gen).to(gpu)
    pool = decoder.new_state_pool(num_slots=3)
    ia = torch.tensor([0], device=gpu)
    ib = torch.tensor([2], device=gpu)
    a0 = decoder.decode_slots(a[..., :4], pool, ia, first_decode=True)
    b0 = decoder.decode_slots(b[..., :3], pool, ib, first_decode=True)
    both = decoder.decode_slots(torch.cat([a[..., 4:7], b[..., 3:6]]), pool,
                                torch.tensor([0, 2], device=gpu), first_decode=False)
    a_whole = decoder.from_indices(a[..., :7])
    b_whole = decoder.from_indices(b)
    hop = decoder.frame_length
    assert torch.equal(torch.cat([a0, both[:1]], -1), a_whole)
    assert torch.equal(torch.cat([b0, both[1:]], -1), b_whole)
    assert pool.parity.tolist() == [2, 0, 2]
    assert a0.shape[-1] == 4 * hop


def test_graph_captured_slot_decode_replays_like_eager(gpu, tiny):
    """A decode step captured in a HIP graph with a static slot index replays like the eager
    decode, every replay, with eager work and synchronisations between replays (the check of
    sglang_omni/models/qwen3_omni/components/code2wav_cuda_graph.py:750-763)."""
    weights, decoder = tiny
    gen = torch.Generator().manual_seed(5)
    codes = torch.randint(0, 64, (2, 4, 18), generator=gen).to(gpu)
    idx = torch.tensor([1, 0], device=gpu)
    eager_pool = decoder.new_state_pool(num_slots=2)
    eager = [decoder.decode_slots(codes[..., :6], eager_pool, idx, first_decode=True)]
    for s in (6, 12):
        eager.append(decoder.decode_slots(codes[..., s:s + 6], eager_pool, idx, first_decode=False))

    pool = decoder.new_state_pool(num_slots=2)
    static_codes = codes[..., :6].clone()
    first = decoder.decode_slots(static_codes, pool, idx, first_decode=True)
    assert torch.equal(first, eager[0])
    static_codes.copy_(codes[..., 6:12])
    decoder.decode_slots(static_codes, pool, idx, first_decode=False)  # warm the workspace
    pool.zero_slots(torch.tensor([0, 1], device=gpu))
    decoder.decode_slots(codes[..., :6], pool, idx, first_decode=True)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            static_out = decoder.decode_slots(static_codes, pool, idx, first_decode=False)
    torch.cuda.current_stream().wait_stream(stream)
    # capture does not execute: the pool still holds the state after chunk 0
    for step, s in enumerate((6, 12)):
        static_codes.copy_(codes[..., s:s + 6])
        graph.replay()
        torch.cuda.synchronize()
        _ = torch.randn(1000, device=gpu).sum().item()  # eager work between replays
        assert torch.equal(static_out, eager[step + 1]), f"replay {step}"


def test_codec_24k_decoder_matches_the_oracle(gpu):
    """The 24 kHz codec (16 x 2048 x 512 tables, 1536 channels, strides 8/8/5/6) on 40 frames
    (3.2 s) of uniform random codes, batch 1."""
    weights = make_dac_weights(CODEC_24K, seed=0)
    decoder = DacCodecDecoder(weights, CODEC_24K, device=gpu)
    gen = torch.Generator().manual_seed(0)
    codes = torch.randint(0, 2048, (1, 16, 40), generator=gen)
    out = decoder.from_indices(codes.to(gpu))
    expected = O.dac_from_indices(codes, reference_weights(weights, "bf16"))
    check_waveform(out, expected, 2e-3)


def test_streaming_24k_chunks_equal_whole_stream_and_oracle(gpu):
    """The streaming pattern: 4 streams, 12-frame chunks, 3 chunks each, per-layer states in the
    slot pool; every chunk's samples equal the whole-stream decode bitwise and the oracle within
    tolerance."""
    weights = make_dac_weights(CODEC_24K, seed=0)
    decoder = DacCodecDecoder(weights, CODEC_24K, device=gpu)
    gen = torch.Generator().manual_seed(7)
    codes = torch.randint(0, 2048, (4, 16, 36), generator=gen)
    pool = decoder.new_state_pool(num_slots=8)
    idx = torch.tensor([5, 0, 7, 2], device=gpu)
    parts = [decoder.decode_slots(codes[..., s:s + 12].to(gpu), pool, idx, first_decode=s == 0)
             for s in (0, 12, 24)]
    streamed = torch.cat(parts, -1)
    whole = decoder.from_indices(codes.to(gpu))
    assert torch.equal(streamed, whole)
    expected = O.dac_from_indices(codes[:1], reference_weights(weights, "bf16"))
    check_waveform(streamed[:1], expected, 2e-3)


def test_fp8_weight_decoder_matches_the_dequantized_oracle(gpu):
    """The long-form fp8-weight decoder (32 x 1024 x 512 tables, E4M3 conv weights with fp32
    per-output-channel scales) on 24 frames, batch 2, against the float32 oracle with the
    dequantized weights; tolerance 5e-3."""
    weights = make_dac_weights(CODEC_24K_LONG, seed=0)
    decoder = DacCodecDecoder(weights, CODEC_24K_LONG, device=gpu, weight_format="fp8")
    gen = torch.Generator().manual_seed(9)
    codes = torch.randint(0, 1024, (2, 32, 24), generator=gen)
    out = decoder.from_indices(codes.to(gpu))
    expected = O.dac_from_indices(codes, reference_weights(weights, "fp8"))
    check_waveform(out, expected, 5e-3)


@pytest.mark.parametrize("residual_dtype", [torch.float16, torch.float32])
def test_hifigan_matches_the_oracle(gpu, residual_dtype):
    """The HiFiGAN body (80 mels, 512 channels, rates 8/5/3/4, MRF k 3/7/11 d 1/3/5) on 20 mel
    frames of log-mel ~ N(-5, 2), batch 2, with float16 (the default) or float32 residual
    streams."""
    weights = make_hifigan_weights(HIFIGAN_24K, seed=0)
    vocoder = HifiGanVocoder(weights, HIFIGAN_24K, device=gpu, residual_dtype=residual_dtype)
    gen = torch.Generator().manual_seed(0)
    mel = torch.randn(2, 80, 20, generator=gen) * 2 - 5
    out = vocoder(mel.to(gpu))
    expected = O.hifigan_generator(mel, reference_weights(weights, "bf16"))
    check_waveform(out, expected, 2e-3)


@pytest.mark.parametrize("residual_dtype", [torch.float32, torch.float16])
@pytest.mark.parametrize("config", [TINY_FUSED, CODEC_24K], ids=["tiny", "codec24k"])
def test_residual_stacks_decode_like_one_launch_per_unit(gpu, config, residual_dtype):
    """The 96-channel stage as one residual-stack launch per block (the final conv to one
    channel inside it) against one fused launch per residual unit and a separate final conv. With
    a float32 residual stream the residual units give the same bits, and the final conv's two
    forms sum the same products in different float32 orders, so the waveforms agree to float32
    summation error; with a float16 stream the per-unit launches round x between the units, which
    the stack (x in float32 registers) does not, so they agree to that rounding. Streamed decodes
    give each decoder's whole-decode bits."""
    weights = make_dac_weights(config, seed=0)
    stacked = DacCodecDecoder(weights, config, device=gpu, residual_dtype=residual_dtype)
    per_unit = DacCodecDecoder(weights, config, device=gpu, residual_stacks=False,
                               residual_dtype=residual_dtype)
    assert any(b.stack for b in stacked.blocks) and not any(b.stack for b in per_unit.blocks)
    assert stacked.final_in_stack and not per_unit.final_in_stack
    gen = torch.Generator().manual_seed(4)
    codes = torch.randint(0, config.codebook_size, (3, config.n_codebooks, 24), generator=gen)
    codes = codes.to(gpu)
    wholes = [stacked.from_indices(codes), per_unit.from_indices(codes)]
    # float16: x rounded between the units (|x| up to a few units: 2^-11 relative) moves the
    # tiny decoder's waveform by up to ~5e-4, well inside the oracle bound of 2e-3
    atol = 2e-6 if residual_dtype == torch.float32 else 1e-3
    torch.testing.assert_close(wholes[0], wholes[1], rtol=0, atol=atol)
    idx = torch.tensor([2, 0, 1], device=gpu)
    for dec, whole in zip((stacked, per_unit), wholes):
        pool = dec.new_state_pool(num_slots=3)
        streamed = torch.cat([dec.decode_slots(codes[..., s:s + 8], pool, idx, first_decode=s == 0)
                              for s in (0, 8, 16)], -1)
        assert torch.equal(streamed, whole)


def test_long_inputs_decode_in_chunks_with_the_whole_decodes_bits(gpu):
    """from_indices splits inputs longer than its buffers allow into frame chunks through slot
    state; forcing small chunks gives the single call's bits."""
    weights = make_dac_weights(TINY_FUSED, seed=0)
    decoder = DacCodecDecoder(weights, TINY_FUSED, device=gpu)
    gen = torch.Generator().manual_seed(11)
    codes = torch.randint(0, 64, (3, 4, 23), generator=gen).to(gpu)
    whole = decoder.from_indices(codes)
    per_frame, samples = 0, 1  # bytes of the largest float32 activation per frame
    for rate, channels in zip(TINY_FUSED.rates, TINY_FUSED.stage_channels()[1:]):
        samples *= rate
        per_frame = max(per_frame, samples * channels * 4)
    for frames in (1, 6):
        decoder.MAX_BUFFER_BYTES = 3 * frames * per_frame
        assert decoder.frames_per_call(3) == frames
        assert torch.equal(decoder.from_indices(codes), whole)
