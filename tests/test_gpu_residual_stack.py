"""The residual-stack kernel (every residual unit of a decoder block in one launch) against the
same units run one omni_conv1d_fused launch each — bit for bit, since the kernel repeats their
arithmetic — on long rows, short rows (several stream rows per tile), ragged tails, one to four
units and bf16 / fp8 weights; and its streaming form (per-unit slot histories, chunks shorter
than the receptive field) against the whole-row launch. The decoder's final conv to one channel,
fused behind the stack, against omni_single_output_conv over the stack's output, bit for bit,
whole and streamed."""

from __future__ import annotations

import pytest
import torch

from sglang_omni_amd import _native as N
from sglang_omni_amd.kernels.conv import (
    FinalConv,
    ResidualUnitWeights,
    fused_conv,
    pack_conv1d,
    residual_stack,
    stack_coefficients,
)
from sglang_omni_amd.kernels.single_output_conv import single_output_conv

pytestmark = pytest.mark.gpu

C = 96


def make_units(dilations, device, *, fp8=False, seed=0):
    gen = torch.Generator().manual_seed(seed)

    def snake():
        alpha = 0.5 + torch.rand(C, generator=gen)
        return alpha.to(device), (alpha + 1e-9).reciprocal().to(device)

    units = []
    for d in dilations:
        w1 = torch.randn(C, C, 7, generator=gen) / (C * 7) ** 0.5
        w2 = torch.randn(C, C, 1, generator=gen) / C ** 0.5 * 0.5
        b1 = torch.randn(C, generator=gen) * 0.1
        b2 = torch.randn(C, generator=gen) * 0.1
        conv1 = pack_conv1d(w1, b1, dilation=d, fp8=fp8).to(device)
        conv2 = pack_conv1d(w2, b2, fp8=fp8).to(device)
        (ia, ib), (ma, mb) = snake(), snake()
        units.append(ResidualUnitWeights(conv1, conv2, ia, ib, ma, mb))
    out_a, out_b = snake()
    return units, out_a, out_b


def identity_operand(x, a, b):
    """bf16(Snake(a, b)(x)) computed as the conv kernels stage it: an identity k = 1 conv whose
    staging applies the Snake to the float32 input (the products are exact)."""
    eye = pack_conv1d(torch.eye(C).unsqueeze(-1), None).to(x.device)
    u = torch.empty(x.shape, dtype=torch.bfloat16, device=x.device)
    fused_conv(x, eye, u, in_activation=N.ACT_SNAKE, in_a=a, in_b=b)
    return u


def unit_by_unit(x, units, out_a, out_b):
    x = x.clone()
    u = identity_operand(x, units[0].in_a, units[0].in_b)
    for k, un in enumerate(units):
        na, nb = (units[k + 1].in_a, units[k + 1].in_b) if k + 1 < len(units) else (out_a, out_b)
        nxt = torch.empty_like(u)
        fused_conv(u, un.conv1, nxt, second=un.conv2, mid_activation=N.ACT_SNAKE,
                   mid_a=un.mid_a, mid_b=un.mid_b, residual=x, sum_out=x,
                   activation=N.ACT_SNAKE, act_a=na, act_b=nb)
        u = nxt
    return u, x


@pytest.mark.parametrize("batch,length", [(2, 1000), (3, 37), (1, 5), (5, 179), (64, 12), (1, 2000)])
@pytest.mark.parametrize("dilations", [(1, 3, 9), (2,), (1, 1, 3, 10)])
def test_residual_stack_equals_one_launch_per_unit_bitwise(gpu, batch, length, dilations):
    units, out_a, out_b = make_units(dilations, gpu, seed=batch + length)
    gen = torch.Generator().manual_seed(length)
    x = (torch.randn(batch, length, C, generator=gen) * 0.3).to(gpu)
    out = torch.empty(batch, length, C, dtype=torch.bfloat16, device=gpu)
    x_out = torch.empty_like(x)
    residual_stack(x, units, out, out_a, out_b, x_out=x_out)
    ref_u, ref_x = unit_by_unit(x, units, out_a, out_b)
    assert torch.equal(x_out, ref_x)
    assert torch.equal(out, ref_u)
    assert ref_x.abs().max().item() > 0.5  # the units change x


@pytest.mark.parametrize("batch,length", [(4, 700), (64, 12), (3, 37), (1, 2000), (2, 1000)])
@pytest.mark.parametrize("dilations", [(1, 3, 9), (2,)])
def test_residual_stack_fp8_weights_equal_one_launch_per_unit_bitwise(gpu, batch, length,
                                                                      dilations):
    """E4M3 weights: the stack (tiled form for short rows, the sweep for long ones, the weights'
    bytes staged by LDS DMA and widened when read) against one launch per unit."""
    units, out_a, out_b = make_units(dilations, gpu, fp8=True, seed=3 + length)
    gen = torch.Generator().manual_seed(1)
    x = (torch.randn(batch, length, C, generator=gen) * 0.3).to(gpu)
    out = torch.empty(batch, length, C, dtype=torch.bfloat16, device=gpu)
    x_out = torch.empty_like(x)
    residual_stack(x, units, out, out_a, out_b, x_out=x_out)
    ref_u, ref_x = unit_by_unit(x, units, out_a, out_b)
    assert torch.equal(x_out, ref_x) and torch.equal(out, ref_u)


@pytest.mark.parametrize("splits", [(5, 300, 1, 700, 994), (2000,), (60, 60, 1880)])
def test_residual_stack_chunks_through_slot_histories_equal_the_whole_rows(gpu, splits):
    """Rows decoded chunk by chunk (chunks shorter than each unit's context included), each
    unit's conv keeping its own slot history, give the whole rows' bits."""
    dilations = (1, 3, 9)
    units, out_a, out_b = make_units(dilations, gpu, seed=11)
    batch, length = 3, sum(splits)
    gen = torch.Generator().manual_seed(5)
    x = (torch.randn(batch, length, C, generator=gen) * 0.3).to(gpu)
    whole = torch.empty(batch, length, C, dtype=torch.bfloat16, device=gpu)
    residual_stack(x, units, whole, out_a, out_b)
    slots = 6
    hists = [torch.zeros(slots, 2, 6 * d, C, dtype=torch.bfloat16, device=gpu) for d in dilations]
    parity = torch.zeros(slots, dtype=torch.int64, device=gpu)
    slot_index = torch.tensor([3, 5, 0], device=gpu)
    parts, start = [], 0
    for n, size in enumerate(splits):
        xc = x[:, start:start + size].contiguous()
        out = torch.empty(batch, size, C, dtype=torch.bfloat16, device=gpu)
        residual_stack(xc, units, out, out_a, out_b, histories=hists, slot_index=slot_index,
                       slot_parity=parity, history_cold=n == 0)
        parity[slot_index] += 1
        parts.append(out)
        start += size
    assert torch.equal(torch.cat(parts, dim=1), whole)


def test_residual_stack_rejects_what_it_has_no_kernel_for(gpu):
    units, out_a, out_b = make_units((1,), gpu)
    x = torch.zeros(1, 8, C, device=gpu)
    out = torch.empty(1, 8, C, dtype=torch.bfloat16, device=gpu)
    with pytest.raises(ValueError):
        residual_stack(x, [], out, out_a, out_b)
    with pytest.raises(ValueError):
        residual_stack(x.to(torch.bfloat16), units, out, out_a, out_b)
    big, _, _ = make_units((11,), gpu)  # context 66 rows: past the kernel's guard rows
    with pytest.raises(N.OmniCodecError):
        residual_stack(x, big, out, out_a, out_b)


def final_conv_weights(device, taps=7, seed=7):
    """bf16-valued weights, as the decoder's (the fused form multiplies bf16 weights)."""
    gen = torch.Generator().manual_seed(seed)
    w = (torch.randn(taps, C, generator=gen) / (C * taps) ** 0.5).to(torch.bfloat16).float().to(device)
    b = (torch.randn(1, generator=gen) * 0.05).to(device)
    return w, b


@pytest.mark.parametrize("batch,length", [(2, 1000), (3, 37), (1, 5), (64, 12), (5, 179), (1, 2000)])
def test_residual_stack_final_conv_matches_the_separate_launch(gpu, batch, length):
    """The decoder's conv to one channel fused behind the stack (on MFMA) against
    omni_single_output_conv over the stack's bf16 output: the same products, summed in another
    float32 order, so within float32 summation error (672 terms, outputs of order 0.1)."""
    units, out_a, out_b = make_units((1, 3, 9), gpu, seed=batch * 7 + length)
    gen = torch.Generator().manual_seed(length + 1)
    x = (torch.randn(batch, length, C, generator=gen) * 0.3).to(gpu)
    w, b = final_conv_weights(gpu)
    u = torch.empty(batch, length, C, dtype=torch.bfloat16, device=gpu)
    residual_stack(x, units, u, out_a, out_b)
    expected = torch.empty(batch, 1, length, dtype=torch.float32, device=gpu)
    single_output_conv(u, w, b, expected, activation=N.ACT_TANH, left_pad=6)
    wave = torch.full((batch, 1, length), float("nan"), device=gpu)
    got = residual_stack(x, units, None, out_a, out_b,
                         final=FinalConv(w, b, N.ACT_TANH, wave))
    assert got is wave
    torch.testing.assert_close(wave, expected, rtol=0, atol=2e-6)
    assert expected.abs().max().item() > 0.05


@pytest.mark.parametrize("splits", [(5, 300, 1, 700, 994), (3, 3, 1994), (60, 60, 1880)])
def test_residual_stack_final_conv_streams_through_its_slot_history(gpu, splits):
    """Chunked decode with every unit's history and the final conv's own history (chunks shorter
    than its six-sample context included) equals the whole rows, bit for bit."""
    dilations = (1, 3, 9)
    units, out_a, out_b = make_units(dilations, gpu, seed=13)
    w, b = final_conv_weights(gpu, seed=3)
    batch, length = 3, sum(splits)
    gen = torch.Generator().manual_seed(9)
    x = (torch.randn(batch, length, C, generator=gen) * 0.3).to(gpu)
    whole = torch.empty(batch, 1, length, device=gpu)
    residual_stack(x, units, None, out_a, out_b, final=FinalConv(w, b, N.ACT_TANH, whole))
    slots = 5
    hists = [torch.zeros(slots, 2, 6 * d, C, dtype=torch.bfloat16, device=gpu) for d in dilations]
    fhist = torch.randn(slots, 2, 6, C, device=gpu).to(torch.bfloat16)  # cold start ignores it
    parity = torch.zeros(slots, dtype=torch.int64, device=gpu)
    slot_index = torch.tensor([4, 1, 2], device=gpu)
    parts, start = [], 0
    for n, size in enumerate(splits):
        xc = x[:, start:start + size].contiguous()
        wave = torch.empty(batch, 1, size, device=gpu)
        residual_stack(xc, units, None, out_a, out_b, histories=hists, slot_index=slot_index,
                       slot_parity=parity, history_cold=n == 0,
                       final=FinalConv(w, b, N.ACT_TANH, wave, fhist))
        parity[slot_index] += 1
        parts.append(wave)
        start += size
    assert torch.equal(torch.cat(parts, dim=-1), whole)


@pytest.mark.parametrize("fp8", [False, True])
@pytest.mark.parametrize("dilations", [(1, 3, 9), (4,)])
def test_residual_stack_precomputed_coefficients_give_the_same_bits(gpu, fp8, dilations):
    """The coefficient rows computed once (omni_residual_stack_coefficients) and passed as
    coef_table give exactly the launch that computes them per workgroup."""
    units, out_a, out_b = make_units(dilations, gpu, fp8=fp8, seed=11)
    table = stack_coefficients(units, out_a, out_b)
    assert table.numel() == (8 * len(units) + 2) * C
    gen = torch.Generator().manual_seed(5)
    x = (torch.randn(3, 700, C, generator=gen) * 0.5).to(gpu)
    outs = []
    for coef in (None, table):
        out = torch.empty(3, 700, C, dtype=torch.bfloat16, device=gpu)
        x_out = torch.empty_like(x)
        residual_stack(x, units, out, out_a, out_b, x_out=x_out, coef_table=coef)
        outs.append((out, x_out))
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])
    with pytest.raises(ValueError):
        residual_stack(x, units, torch.empty_like(outs[0][0]), out_a, out_b,
                       coef_table=table[:-1])
