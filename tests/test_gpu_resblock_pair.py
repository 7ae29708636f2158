"""``omni_resblock_pair`` (kernels/conv.py ``resblock_pair``): a 32-channel HiFiGAN ResBlock pair
in one launch equals its two ``omni_conv1d_fused`` launches (c1 into a bf16 h, then c2 with the
residual / sum_out / mix epilogue) bit for bit, for every kernel size and dilation of the
multi-receptive-field blocks (k 3 / 7 / 11, d 1 / 3 / 5), rows shorter and longer than a tile,
float16 and float32 residual streams; and the whole vocoder gives the same bits with and without
pairs (restating hift_layers.py:95-110's pair: xt = c2(act(c1(act(x)))) + x)."""

from __future__ import annotations

import math

import pytest
import torch

from sglang_omni_amd import _native as N
from sglang_omni_amd.kernels.conv import fused_conv, pack_conv1d, resblock_pair
from sglang_omni_amd.models import HifiGanVocoder
from sglang_omni_amd.models.configs import HIFIGAN_24K, make_hifigan_weights

pytestmark = pytest.mark.gpu

SLOPE = 0.1


def _pair(k, d, seed, gpu):
    g = torch.Generator().manual_seed(seed)
    c1 = pack_conv1d(torch.randn(32, 32, k, generator=g) / math.sqrt(32 * k),
                     torch.randn(32, generator=g) * 0.1, dilation=d, causal=False).to(gpu)
    c2 = pack_conv1d(torch.randn(32, 32, k, generator=g) / math.sqrt(32 * k),
                     torch.randn(32, generator=g) * 0.1, causal=False).to(gpu)
    return c1, c2


def _two_launches(x, c1, c2, out, **kw):
    h = torch.empty(x.shape, dtype=torch.bfloat16, device=x.device)
    fused_conv(x, c1, h, activation=N.ACT_LEAKY_RELU, slope=SLOPE)
    return fused_conv(h, c2, out, **kw)


@pytest.mark.parametrize("k", [3, 7, 11])
@pytest.mark.parametrize("d", [1, 3, 5])
@pytest.mark.parametrize("batch,length", [(3, 1000), (2, 60)])
def test_pair_equals_two_launches(gpu, k, d, batch, length):
    c1, c2 = _pair(k, d, 10 * k + d, gpu)
    g = torch.Generator().manual_seed(k * d + length)
    x = torch.randn(batch, length, 32, generator=g).to(torch.bfloat16).to(gpu)
    resid = (torch.randn(batch, length, 32, generator=g) * 2).half().to(gpu)
    outs = []
    for run in (_two_launches, lambda *a, **kw: resblock_pair(*a, slope1=SLOPE, **kw)):
        out = torch.full((batch, length, 32), float("nan"), dtype=torch.bfloat16, device=gpu)
        s = torch.full((batch, length, 32), float("nan"), dtype=torch.float16, device=gpu)
        run(x, c1, c2, out, residual=resid, sum_out=s, activation=N.ACT_LEAKY_RELU, slope=SLOPE)
        outs.append((out, s))
    (o_ref, s_ref), (o, s) = outs
    assert torch.equal(o, o_ref) and torch.equal(s, s_ref)


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_pair_with_the_three_block_mix(gpu, dtype):
    """The stage's last pair: residual, the other blocks' streams mixed in (mean of three), the
    next stage's operand out; and a block's last pair: no out, the stream only."""
    c1, c2 = _pair(11, 5, 3, gpu)
    g = torch.Generator().manual_seed(4)
    batch, length = 2, 3000
    x = torch.randn(batch, length, 32, generator=g).to(torch.bfloat16).to(gpu)
    r, a, b = ((torch.randn(batch, length, 32, generator=g) * 2).to(dtype).to(gpu)
               for _ in range(3))
    results = []
    for run in (_two_launches, lambda *p, **kw: resblock_pair(*p, slope1=SLOPE, **kw)):
        out = torch.empty(batch, length, 32, dtype=torch.bfloat16, device=gpu)
        run(x, c1, c2, out, residual=r, mix=(a, b, 1.0 / 3.0), activation=N.ACT_LEAKY_RELU,
            slope=0.01)
        s = torch.empty(batch, length, 32, dtype=dtype, device=gpu)
        run(x, c1, c2, None, residual=r, sum_out=s)
        results.append((out, s))
    assert torch.equal(results[0][0], results[1][0])
    assert torch.equal(results[0][1], results[1][1])


def test_vocoder_with_and_without_pairs(gpu):
    weights = make_hifigan_weights(HIFIGAN_24K, seed=1)
    g = torch.Generator().manual_seed(5)
    mel = (torch.randn(2, 80, 40, generator=g) * 2 - 5).to(gpu)
    paired = HifiGanVocoder(weights, HIFIGAN_24K, device=gpu)(mel)
    plain = HifiGanVocoder(weights, HIFIGAN_24K, device=gpu, resblock_pairs=False)(mel)
    assert torch.equal(paired, plain)


def test_pair_contract(gpu):
    c1, c2 = _pair(3, 1, 1, gpu)
    x = torch.zeros(1, 64, 32, dtype=torch.bfloat16, device=gpu)
    out = torch.empty_like(x)
    wide = pack_conv1d(torch.randn(64, 32, 3), None, causal=False).to(gpu)
    with pytest.raises(ValueError, match="32-channel"):
        resblock_pair(x, wide, c2, out, slope1=SLOPE)
    with pytest.raises(ValueError, match="bf16"):
        resblock_pair(x.float(), c1, c2, out, slope1=SLOPE)
