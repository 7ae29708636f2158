"""The float16 residual stream (``residual_dtype`` of omni_conv1d_fused, ``x_dtype`` of
omni_residual_stack): the kernels widen a float16 stream exactly, add in float32 and round the
stored sum once to float16 (nearest even). So every launch with a float16 stream equals the same
launch with the float32 widening of that stream bit for bit, its stored sum being the float16
rounding of the float32 one: the LDS-DMA k = 1 conv, the register-staged k = 7 conv, the fused
residual unit (LDS-DMA with bf16 weights, register-staged with E4M3 weights), the transposed
conv's stream store and the residual stack (x read as float16, x_last stored as float16)."""

from __future__ import annotations

import ctypes
import math

import pytest
import torch

from sglang_omni_amd import _native as N
from sglang_omni_amd.kernels.conv import (
    FinalConv,
    _conv_args,
    fused_conv,
    pack_conv1d,
    pack_conv_transpose1d,
    residual_stack,
)

from .test_gpu_residual_stack import make_units

pytestmark = pytest.mark.gpu


def _snake(c, gen, device):
    a = 0.5 + torch.rand(c, generator=gen)
    return a.to(device), (a + 1e-9).reciprocal().to(device)


def _both(run, x16):
    """run(residual, sum_out) with the float16 stream and with its float32 widening."""
    s16 = torch.full_like(x16, float("nan"))
    s32 = torch.full(x16.shape, float("nan"), dtype=torch.float32, device=x16.device)
    o16 = run(x16, s16)
    o32 = run(x16.float(), s32)
    return (o16, s16), (o32, s32)


def _assert_same(half, full):
    (o16, s16), (o32, s32) = half, full
    assert torch.equal(s16, s32.half()), "the float16 store is not the rounded float32 sum"
    if o16 is not None:
        assert torch.equal(o16, o32), "the next operand differs"


@pytest.mark.parametrize("c_in,c_out,rows", [(384, 384, 3000), (768, 768, 700)])
def test_k1_conv_with_a_float16_stream(gpu, c_in, c_out, rows):
    gen = torch.Generator().manual_seed(c_in + rows)
    h = torch.randn(1, rows, c_in, generator=gen).to(torch.bfloat16).to(gpu)
    conv = pack_conv1d(torch.randn(c_out, c_in, 1, generator=gen) / math.sqrt(c_in),
                       torch.randn(c_out, generator=gen) * 0.1).to(gpu)
    x16 = (torch.randn(1, rows, c_out, generator=gen) * 3).half().to(gpu)
    a, b = _snake(c_out, gen, gpu)

    def run(res, s):
        out = torch.empty(1, rows, c_out, dtype=torch.bfloat16, device=gpu)
        fused_conv(h, conv, out, residual=res, sum_out=s, activation=N.ACT_SNAKE, act_a=a, act_b=b,
                   kernel=N.CONV_KERNEL_DMA, config=1)
        return out

    _assert_same(*_both(run, x16))


def test_staged_k7_conv_with_a_float16_stream(gpu):
    gen = torch.Generator().manual_seed(7)
    c, rows = 192, 900
    x = torch.randn(2, rows, c, generator=gen).to(gpu)  # float32 operand: the staged kernel
    conv = pack_conv1d(torch.randn(c, c, 7, generator=gen) / math.sqrt(7 * c),
                       torch.randn(c, generator=gen) * 0.1, dilation=3).to(gpu)
    x16 = torch.randn(2, rows, c, generator=gen).half().to(gpu)
    a, b = _snake(c, gen, gpu)

    def run(res, s):
        out = torch.empty(2, rows, c, dtype=torch.bfloat16, device=gpu)
        fused_conv(x, conv, out, residual=res, sum_out=s, in_activation=N.ACT_SNAKE, in_a=a,
                   in_b=b, activation=N.ACT_SNAKE, act_a=a, act_b=b)
        return out

    _assert_same(*_both(run, x16))


@pytest.mark.parametrize("fp8", [False, True])
def test_fused_unit_with_a_float16_stream(gpu, fp8):
    gen = torch.Generator().manual_seed(11 + fp8)
    c, batch, length = 192, 8, 240
    u = torch.randn(batch, length, c, generator=gen).to(torch.bfloat16).to(gpu)
    p1 = pack_conv1d(torch.randn(c, c, 7, generator=gen) / math.sqrt(7 * c),
                     torch.randn(c, generator=gen) * 0.1, dilation=9, fp8=fp8).to(gpu)
    p2 = pack_conv1d(torch.randn(c, c, 1, generator=gen) / math.sqrt(c),
                     torch.randn(c, generator=gen) * 0.1, fp8=fp8).to(gpu)
    x16 = torch.randn(batch, length, c, generator=gen).half().to(gpu)
    (ma, mb), (na, nb) = _snake(c, gen, gpu), _snake(c, gen, gpu)

    def run(res, s):
        out = torch.empty(batch, length, c, dtype=torch.bfloat16, device=gpu)
        fused_conv(u, p1, out, second=p2, mid_activation=N.ACT_SNAKE, mid_a=ma, mid_b=mb,
                   residual=res, sum_out=s, activation=N.ACT_SNAKE, act_a=na, act_b=nb)
        return out

    _assert_same(*_both(run, x16))


def test_transposed_conv_stores_a_float16_stream(gpu):
    gen = torch.Generator().manual_seed(13)
    c_in, c_out, s, rows = 192, 96, 6, 400
    u = torch.randn(4, rows, c_in, generator=gen).to(torch.bfloat16).to(gpu)
    conv = pack_conv_transpose1d(torch.randn(c_in, c_out, 2 * s, generator=gen) / math.sqrt(c_in),
                                 torch.randn(c_out, generator=gen) * 0.1, stride=s).to(gpu)
    x32 = torch.empty(4, rows, s * c_out, device=gpu)
    x16 = torch.empty(4, rows, s * c_out, dtype=torch.float16, device=gpu)
    fused_conv(u, conv, None, sum_out=x32)
    fused_conv(u, conv, None, sum_out=x16)
    assert torch.equal(x16, x32.half())


@pytest.mark.parametrize("batch,length,final", [(2, 1000, False), (64, 12, False), (3, 700, True)])
def test_residual_stack_reads_and_writes_a_float16_stream(gpu, batch, length, final):
    units, out_a, out_b = make_units((1, 3, 9), gpu, seed=21)
    gen = torch.Generator().manual_seed(22)
    x16 = torch.randn(batch, length, 96, generator=gen).half().to(gpu)
    fw = (torch.randn(7, 96, generator=gen) / 30).to(gpu)
    fb = torch.zeros(1, device=gpu)
    results = []
    for x in (x16, x16.float()):
        out = torch.empty(batch, length, 96, dtype=torch.bfloat16, device=gpu)
        x_out = torch.empty_like(x)
        fin = FinalConv(fw, fb, N.ACT_TANH, torch.empty(batch, 1, length, device=gpu),
                        None) if final else None
        residual_stack(x, units, out, out_a, out_b, x_out=x_out, final=fin)
        results.append((out, x_out, fin.out if final else None))
    (o16, xo16, f16), (o32, xo32, f32) = results
    assert torch.equal(o16, o32)
    assert torch.equal(xo16, xo32.half())
    if final:
        assert torch.equal(f16, f32)


def test_mix_of_float16_streams(gpu):
    """The mean of three float16 streams (HiFiGAN's multi-receptive-field mix): each stream
    widened exactly, the same float32 sum as with the widened streams, rounded once."""
    gen = torch.Generator().manual_seed(33)
    c, rows = 128, 1500
    h = torch.randn(2, rows, c, generator=gen).to(torch.bfloat16).to(gpu)
    conv = pack_conv1d(torch.randn(c, c, 7, generator=gen) / math.sqrt(7 * c),
                       torch.randn(c, generator=gen) * 0.1, dilation=5).to(gpu)
    x16, a16, b16 = ((torch.randn(2, rows, c, generator=gen) * 2).half().to(gpu)
                     for _ in range(3))
    outs = []
    for dt in (torch.float16, torch.float32):
        s = torch.full((2, rows, c), float("nan"), dtype=dt, device=gpu)
        out = torch.empty(2, rows, c, dtype=torch.bfloat16, device=gpu)
        fused_conv(h, conv, out, residual=x16.to(dt), sum_out=s, activation=N.ACT_LEAKY_RELU,
                   slope=0.01, mix=(a16.to(dt), b16.to(dt), 1.0 / 3.0))
        outs.append((out, s))
    (o16, s16), (o32, s32) = outs
    assert torch.equal(o16, o32)
    assert torch.equal(s16, s32.half())


def test_float16_streams_refuse_a_dtype_mix_and_misaligned_rows(gpu):
    gen = torch.Generator().manual_seed(31)
    h = torch.randn(1, 64, 128, generator=gen).to(torch.bfloat16).to(gpu)
    conv = pack_conv1d(torch.randn(128, 128, 1, generator=gen) / 12, None).to(gpu)
    x16 = torch.zeros(1, 64, 128, dtype=torch.float16, device=gpu)
    m = torch.zeros(1, 64, 128, device=gpu)
    with pytest.raises(ValueError, match="share one dtype"):
        fused_conv(h, conv, None, sum_out=x16, mix=(m, m, 0.5))
    # an 8-byte-misaligned float16 stream is refused by the library before any launch
    buf = torch.zeros(64 * 128 + 2, dtype=torch.float16, device=gpu)
    odd = buf[2:].view(1, 64, 128)
    args = _conv_args(h, conv, None, sum_out=odd)
    lib = N.load_library()
    assert lib.omni_conv1d_fused(ctypes.byref(args), N.stream_handle(gpu)) == N.INVALID_ARG
