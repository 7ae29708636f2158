"""GPU parity of the RVQ gather-sum, the state-exchange kernels, the single-output conv and the
Snake-family elementwise kernels, each against the oracle or the reference's own test
expectations, called through the C ABI."""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from sglang_omni_amd import _native as N
from sglang_omni_amd.kernels import (
    SnakeBetaCoefficients,
    clamped_single_output_conv,
    fused_bias_snake_beta,
    history_exchange,
    overlap_exchange,
    rvq_gather_sum,
)
from sglang_omni_amd.utils.snake_beta import snake1d
from oracle import codec_oracle as O

pytestmark = pytest.mark.gpu


# ------------------------------------------------------------------------------------- RVQ


@pytest.mark.parametrize(
    "batch,k,v,d,t,code_dtype",
    [
        (1, 8, 1024, 256, 50, torch.int32),     # the single-block workload
        (1, 16, 2048, 512, 250, torch.int64),   # the 24 kHz codec's quantizer
        (3, 32, 1024, 512, 37, torch.int64),
        (2, 1, 64, 24, 5, torch.int32),
        (2, 9, 33, 520, 3, torch.int64),         # K not a multiple of 8, D past one wave
        (1, 40, 64, 128, 9, torch.int32),        # K > 32: the four-frame kernel
        (3, 4, 256, 64, 2900, torch.int64),      # > 8192 frames: the four-frame kernel
    ],
)
def test_rvq_gather_sum_is_bit_exact_in_fp32(gpu, batch, k, v, d, t, code_dtype):
    gen = torch.Generator().manual_seed(batch * 1000 + k)
    tables = torch.randn(k, v, d, generator=gen) * 0.02
    codes = torch.randint(0, v, (batch, k, t), generator=gen).to(code_dtype)
    expected = O.rvq_gather_sum(codes, tables)  # [B, D, T]
    got = rvq_gather_sum(codes.to(gpu), tables.to(gpu), channels_last=False)
    assert torch.equal(got.cpu(), expected)
    got_cl = rvq_gather_sum(codes.to(gpu), tables.to(gpu))
    assert torch.equal(got_cl.cpu(), expected.transpose(1, 2))


def test_rvq_bf16_tables_sum_in_fp32_and_round_once(gpu):
    gen = torch.Generator().manual_seed(3)
    tables = (torch.randn(16, 2048, 512, generator=gen) * 0.02).to(torch.bfloat16)
    codes = torch.randint(0, 2048, (2, 16, 20), generator=gen)
    expected = O.rvq_gather_sum(codes, tables.float())
    got32 = rvq_gather_sum(codes.to(gpu), tables.to(gpu), out_dtype=torch.float32,
                           channels_last=False)
    assert torch.equal(got32.cpu(), expected)
    got16 = rvq_gather_sum(codes.to(gpu), tables.to(gpu), channels_last=False)
    assert got16.dtype == torch.bfloat16
    assert torch.equal(got16.cpu(), expected.to(torch.bfloat16))


def test_rvq_mean_form_and_code_clamping(gpu):
    gen = torch.Generator().manual_seed(4)
    tables = torch.randn(4, 100, 64, generator=gen)
    codes = torch.randint(0, 100, (2, 4, 9), generator=gen)
    mean = rvq_gather_sum(codes.to(gpu), tables.to(gpu), mean=True, channels_last=False)
    assert torch.equal(mean.cpu(), O.rvq_gather_sum(codes, tables, mean=True))
    big = codes.clone()
    big[0, 1, 2] = 5000
    big[1, 3, 0] = 100
    clamped = rvq_gather_sum(big.to(gpu), tables.to(gpu), channels_last=False)
    assert torch.equal(clamped.cpu(), O.rvq_gather_sum(O.clamp_codes(big, 100), tables))
    # without clamping an out-of-range code adds nothing (the ordered gather-sum convention)
    dropped = rvq_gather_sum(big.to(gpu), tables.to(gpu), clamp=False, channels_last=False)
    keep = codes.clone()
    expected = O.rvq_gather_sum(keep, tables)
    for (b, k, t) in [(0, 1, 2), (1, 3, 0)]:  # the two frames that lost one codebook
        total = torch.zeros(64)
        for kk in range(4):
            if kk != k:
                total = total + tables[kk, codes[b, kk, t]]
        expected[b, :, t] = total
    assert torch.equal(dropped.cpu(), expected)


def test_rvq_rejects_bad_shapes(gpu):
    tables = torch.zeros(4, 10, 64, device=gpu)
    with pytest.raises(ValueError):
        rvq_gather_sum(torch.zeros(2, 3, 5, dtype=torch.int64, device=gpu), tables)
    with pytest.raises(N.OmniCodecError):
        rvq_gather_sum(torch.zeros(1, 4, 5, dtype=torch.int64, device=gpu),
                       torch.zeros(4, 10, 6, device=gpu))  # D not a multiple of 4


# ------------------------------------------------------------------ state exchange kernels


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("is_channels_first", [False, True])
@pytest.mark.parametrize("is_cold", [False, True])
@pytest.mark.parametrize(
    "history_samples,new_samples,tail_samples",
    [(2, 1, 0), (6, 2, 0), (6, 4, 0), (6, 40, 2), (18, 320, 0), (54, 32, 2), (54, 320, 8)],
)
def test_history_exchange_kernel_equals_the_reference(
    gpu, dtype, is_channels_first, is_cold, history_samples, new_samples, tail_samples
):
    """The case grid of tests/unit_test/kernels/test_codec_state.py:133-176."""
    torch.manual_seed(history_samples * new_samples)
    channels = 200
    slot_index = torch.tensor([4, 1, 6], device=gpu)
    history_pool = torch.randn(8, history_samples, channels, device=gpu).to(dtype)
    samples = history_samples + new_samples + tail_samples
    if is_channels_first:
        padded = torch.randn(3, channels, samples, device=gpu).to(dtype).transpose(1, 2)
    else:
        padded = torch.randn(3, samples, channels, device=gpu).to(dtype)
    expected_padded, expected_pool = padded.clone(), history_pool.clone()
    O.history_exchange_reference(expected_padded, expected_pool, slot_index, new_samples, is_cold)
    history_exchange(padded, history_pool, slot_index, new_samples, is_cold)
    assert torch.equal(padded, expected_padded)
    assert torch.equal(history_pool, expected_pool)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("is_channels_first", [False, True])
@pytest.mark.parametrize("is_cold", [False, True])
@pytest.mark.parametrize(
    "overlap_samples,emitted_samples", [(3, 3), (4, 640), (5, 160), (8, 32), (8, 320)]
)
def test_overlap_exchange_kernel_equals_the_reference(
    gpu, dtype, is_channels_first, is_cold, overlap_samples, emitted_samples
):
    """The case grid of tests/unit_test/kernels/test_codec_state.py:179-214."""
    torch.manual_seed(overlap_samples * emitted_samples)
    channels = 200
    slot_index = torch.tensor([4, 1, 6], device=gpu)
    overlap_pool = torch.randn(8, overlap_samples, channels, device=gpu).to(dtype)
    samples = emitted_samples + overlap_samples
    if is_channels_first:
        output = torch.randn(3, channels, samples, device=gpu).to(dtype).transpose(1, 2)
    else:
        output = torch.randn(3, samples, channels, device=gpu).to(dtype)
    expected_output, expected_pool = output.clone(), overlap_pool.clone()
    O.overlap_exchange_reference(expected_output, expected_pool, slot_index, emitted_samples,
                                 is_cold)
    overlap_exchange(output, overlap_pool, slot_index, emitted_samples, is_cold)
    assert torch.equal(output, expected_output)
    assert torch.equal(overlap_pool, expected_pool)


@pytest.mark.parametrize("history_samples", [2, 6, 54])
@pytest.mark.parametrize("chunks", [(10, 10, 7), (1, 2, 1, 3, 40), (32, 1, 32)])
def test_history_exchange_builds_the_causal_window_of_the_whole_stream(gpu, history_samples,
                                                                       chunks):
    """tests/unit_test/kernels/test_codec_state.py:52-94, on the HIP exchange kernel."""
    torch.manual_seed(history_samples + len(chunks))
    slots, channels = 5, 3
    slot_index = torch.tensor([3, 1], device=gpu)
    history_pool = torch.randn(slots, history_samples, channels, device=gpu)
    untouched = history_pool[[0, 2, 4]].clone()
    stream = torch.randn(2, sum(chunks), channels, device=gpu)
    whole = F.pad(stream, (0, 0, history_samples, 0))
    start = 0
    for index, new_samples in enumerate(chunks):
        padded = torch.full((2, history_samples + new_samples + 2, channels), 7.0, device=gpu)
        padded[:, history_samples:history_samples + new_samples] = stream[:, start:start + new_samples]
        history_exchange(padded, history_pool, slot_index, new_samples=new_samples,
                         is_cold=index == 0)
        torch.testing.assert_close(padded[:, :history_samples + new_samples],
                                   whole[:, start:start + history_samples + new_samples],
                                   rtol=0, atol=0)
        assert not padded[:, history_samples + new_samples:].any()
        start += new_samples
    torch.testing.assert_close(history_pool[slot_index], whole[:, -history_samples:], rtol=0,
                               atol=0)
    torch.testing.assert_close(history_pool[[0, 2, 4]], untouched, rtol=0, atol=0)


# ------------------------------------------------------------------ single-output conv


def make_conv(channels: int, dtype: torch.dtype, device) -> torch.nn.Conv1d:
    conv = torch.nn.Conv1d(channels, 1, 7).to(device=device, dtype=dtype)
    return conv


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("channels", [8, 96])
def test_single_output_conv_is_the_clamped_conv_rounded_once(gpu, dtype, channels):
    """tests/unit_test/kernels/test_single_output_conv.py:19-44."""
    torch.manual_seed(0)
    conv = make_conv(channels, dtype, gpu)
    padded = torch.randn(3, 300 + 6, channels, device=gpu, dtype=dtype)
    with torch.inference_mode():
        actual = clamped_single_output_conv(padded, conv, 300)
        expected = O.clamped_single_output_conv(padded.cpu(), conv.weight.cpu(), conv.bias.cpu(),
                                                300).to(dtype)
    assert actual.shape == (3, 1, 300) and actual.is_contiguous()
    assert (expected.abs() == 1).any() and (expected.abs() < 1).any()
    torch.testing.assert_close(actual.cpu(), expected)


def test_single_output_conv_gives_a_position_the_same_bits_in_any_split(gpu):
    """tests/unit_test/kernels/test_single_output_conv.py:47-66."""
    torch.manual_seed(0)
    conv = make_conv(96, torch.bfloat16, gpu)
    padded = torch.randn(3, 1000 + 6, 96, device=gpu, dtype=torch.bfloat16)
    with torch.inference_mode():
        whole = clamped_single_output_conv(padded, conv, 1000)
        parts = torch.cat(
            [clamped_single_output_conv(padded[:, :417 + 6], conv, 417),
             clamped_single_output_conv(padded[:, 417:], conv, 583)],
            dim=-1,
        )
        row = clamped_single_output_conv(padded[1:2], conv, 1000)
    assert torch.equal(parts, whole)
    assert torch.equal(row, whole[1:2])


@pytest.mark.parametrize("channels", [32, 64, 96, 128, 136])
@pytest.mark.parametrize("taps", [7, 8])
def test_decoder_form_single_output_conv_streams_like_the_whole_row(gpu, channels, taps):
    """The decoder's last layer: causal conv of bf16 operands to one channel + tanh. The whole
    rows match a float64 direct sum, and decoding them in chunks (some shorter than the context)
    through the slot history gives the whole decode's bits."""
    from sglang_omni_amd.kernels.single_output_conv import single_output_conv

    gen = torch.Generator().manual_seed(channels + taps)
    batch, length, ctx = 3, 700, taps - 1
    x = (torch.randn(batch, length, channels, generator=gen) * 0.5).to(torch.bfloat16)
    w = torch.randn(taps, channels, generator=gen) / (taps * channels) ** 0.5
    bias = torch.tensor([0.05])
    xg, wg, bg = x.to(gpu), w.to(gpu), bias.to(gpu)
    whole = torch.empty(batch, 1, length, device=gpu)
    single_output_conv(xg, wg, bg, whole, activation=N.ACT_TANH, left_pad=ctx)
    padded = F.pad(x.double(), (0, 0, ctx, 0))
    ref = sum(padded[:, j:j + length] @ w[j].double() for j in range(taps)) + 0.05
    assert (whole.cpu()[:, 0].double() - torch.tanh(ref)).abs().max().item() < 2e-6

    slots = 5
    history = torch.zeros(slots, 2 * ctx * channels, dtype=torch.bfloat16, device=gpu)
    parity = torch.zeros(slots, dtype=torch.int64, device=gpu)
    slot_index = torch.tensor([4, 0, 2], device=gpu)
    pieces, start = [], 0
    for n, size in enumerate([5, 300, 1, 3, 391]):
        out = torch.empty(batch, 1, size, device=gpu)
        single_output_conv(xg[:, start:start + size].contiguous(), wg, bg, out,
                           activation=N.ACT_TANH, left_pad=ctx, history=history,
                           slot_index=slot_index, slot_parity=parity, history_cold=n == 0)
        parity[slot_index] += 1
        pieces.append(out)
        start += size
    assert start == length
    assert torch.equal(torch.cat(pieces, dim=-1), whole)


# ------------------------------------------------------------------ Snake family


def eager_bias_snake_beta(conv, bias, alpha_scale, inverse_beta, residual=None):
    """The eager op chain (every op in the activations' dtype) the reference's fused kernel
    equals bitwise, evaluated on the CPU."""
    total = conv + bias
    if residual is not None:
        total = total + residual
    phase = total * alpha_scale
    sine = torch.sin(phase)
    sq = sine * sine
    return total, total + inverse_beta * sq


def ulp_mismatch_fraction(a: torch.Tensor, b: torch.Tensor) -> tuple[float, int]:
    """Fraction of elements that differ, and the largest difference in units of the dtype's ulp."""
    ai = a.view(torch.int16).to(torch.int32)
    bi = b.view(torch.int16).to(torch.int32)
    diff = (ai - bi).abs()
    return (diff > 0).float().mean().item(), int(diff.max().item())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("channels", [96, 1536])
@pytest.mark.parametrize("has_residual", [False, True])
def test_fused_bias_snake_beta_matches_the_eager_chain(gpu, dtype, channels, has_residual):
    """tests/unit_test/kernels/test_bias_snake_beta.py:17-56 restated: the sums bitwise, the
    activation bitwise except where the device sinf and the CPU sin disagree in the last float32
    bit at a rounding boundary (at most one ulp of the dtype, on a tiny fraction)."""
    gen = torch.Generator().manual_seed(channels)
    batch, length = 2, 64
    conv = (torch.randn(batch, length + 3, channels, generator=gen)).to(dtype)
    bias = torch.randn(channels, generator=gen).to(dtype)
    alpha = (torch.randn(channels, generator=gen) * 0.3).to(dtype)
    beta = (torch.randn(channels, generator=gen) * 0.3).to(dtype)
    residual = torch.randn(batch, length, channels, generator=gen).to(dtype) if has_residual else None
    coeff = SnakeBetaCoefficients(alpha_scale=torch.exp(alpha), inverse_beta=1.0 / (torch.exp(beta) + 1e-9))
    exp_sum, exp_out = eager_bias_snake_beta(conv[:, :length], bias, coeff.alpha_scale,
                                             coeff.inverse_beta, residual)
    d_coeff = SnakeBetaCoefficients(alpha_scale=coeff.alpha_scale.to(gpu),
                                    inverse_beta=coeff.inverse_beta.to(gpu))
    out_buf = torch.zeros(batch, length + 5, channels, dtype=dtype, device=gpu)
    out = out_buf[:, 2:2 + length]
    sum_out = torch.empty(batch, length, channels, dtype=dtype, device=gpu)
    fused_bias_snake_beta(conv.to(gpu)[:, :length], bias.to(gpu), d_coeff, out,
                          residual=None if residual is None else residual.to(gpu), sum_out=sum_out)
    assert torch.equal(sum_out.cpu(), exp_sum)
    frac, worst = ulp_mismatch_fraction(out.cpu(), exp_out)
    assert worst <= 1 and frac < 2e-3, (frac, worst)
    assert not out_buf[:, :2].any() and not out_buf[:, 2 + length:].any()


def test_snake1d_follows_the_float64_formula(gpu):
    """tests/unit_test/fishaudio_drama3/test_vocoder.py:467-500 restated for bf16 and fp32."""
    gen = torch.Generator().manual_seed(0)
    c = 96
    alpha = torch.rand(c, generator=gen) * 4 + 0.05
    for dtype in (torch.float32, torch.bfloat16):
        x = torch.randn(3, 125, c, generator=gen).to(dtype)
        y = snake1d(x.to(gpu), alpha.to(gpu))
        exact = O.snake(x.double().transpose(1, 2), alpha.double()).transpose(1, 2)
        torch.testing.assert_close(y.cpu(), exact.to(dtype))
