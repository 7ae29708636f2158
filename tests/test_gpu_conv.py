"""GPU parity of the fused MFMA conv against float64 references of the same ops.

Each case packs a reference-layout weight (Conv1d [C_out, C_in, k] / ConvTranspose1d
[C_in, C_out, k]), runs ``omni_conv1d_fused`` through the C ABI, and compares with ``F.conv1d`` /
``F.conv_transpose1d`` in float64 on the CPU over the same bf16-rounded inputs and weights
(the restatements of channels_last_conv.py:45-120 in tests/unit_test/utils/
test_channels_last_conv.py:18-115). The kernel accumulates in float32, so the bound is float32
summation error, far below one bf16 ulp of the outputs; bf16 outputs are compared within one
bf16 ulp (rtol 2^-8).
"""

from __future__ import annotations

import math

import pytest
import torch
import torch.nn.functional as F

from sglang_omni_amd import _native as N
from sglang_omni_amd.kernels.conv import fused_conv, pack_conv1d, pack_conv_transpose1d
from oracle import codec_oracle as O

pytestmark = pytest.mark.gpu


def bf(t: torch.Tensor) -> torch.Tensor:
    return t.to(torch.bfloat16).float()


def rand(*shape: int, gen: torch.Generator, scale: float = 1.0) -> torch.Tensor:
    return torch.randn(*shape, generator=gen) * scale


def conv_ref64(x, w, b, *, dilation=1, causal=True):
    """x [B, L, C_in] float; w [C_out, C_in, k]; float64 conv -> [B, L, C_out]."""
    k = w.shape[-1]
    xc = x.double().transpose(1, 2)
    if causal:
        y = F.conv1d(F.pad(xc, ((k - 1) * dilation, 0)), w.double(), None if b is None else b.double(),
                     dilation=dilation)
    else:
        pad = (k * dilation - dilation) // 2
        y = F.conv1d(xc, w.double(), None if b is None else b.double(), dilation=dilation, padding=pad)
    return y.transpose(1, 2)


def convt_ref64(x, w, b, *, stride, padding=0):
    """x [B, L, C_in]; w [C_in, C_out, k] -> [B, L*stride, C_out] (right-trimmed when padding=0)."""
    y = F.conv_transpose1d(x.double().transpose(1, 2), w.double(),
                           None if b is None else b.double(), stride=stride, padding=padding)
    length = x.shape[1] * stride
    return y[..., :length].transpose(1, 2)


def close(actual: torch.Tensor, expected: torch.Tensor, rtol: float, atol: float) -> None:
    torch.testing.assert_close(actual.double().cpu(), expected.double(), rtol=rtol, atol=atol)


CAUSAL_CASES = [
    # (B, L, C_in, C_out, k, dilation)
    (1, 1, 96, 96, 7, 1),
    (2, 5, 96, 96, 7, 3),
    (1, 16, 512, 256, 7, 1),
    (3, 12, 256, 256, 7, 9),
    (2, 50, 256, 256, 7, 1),
    (2, 130, 192, 192, 7, 9),
    (1, 300, 96, 96, 7, 3),
    (2, 1000, 96, 96, 7, 9),
    (2, 700, 192, 192, 1, 1),
    (1, 257, 384, 384, 7, 1),
    (1, 33, 768, 768, 7, 3),
    (2, 40, 80, 64, 7, 1),
]


@pytest.mark.parametrize("case", CAUSAL_CASES, ids=lambda c: "B{}L{}ci{}co{}k{}d{}".format(*c))
def test_causal_conv_matches_float64(gpu, case):
    batch, length, c_in, c_out, k, d = case
    gen = torch.Generator().manual_seed(length * 31 + k + d)
    x = bf(rand(batch, length, c_in, gen=gen))
    w = bf(rand(c_out, c_in, k, gen=gen, scale=1 / math.sqrt(c_in * k)))
    b = bf(rand(c_out, gen=gen, scale=0.1))
    packed = pack_conv1d(w, b, dilation=d).to(gpu)
    out = torch.empty(batch, length, c_out, dtype=torch.float32, device=gpu)
    fused_conv(x.to(gpu, torch.bfloat16), packed, out)
    close(out, conv_ref64(x, w, b, dilation=d), rtol=1e-5, atol=1e-5)


SAME_CASES = [
    # (B, L, C, k, dilation)
    (2, 37, 64, 3, 1),
    (1, 300, 32, 11, 5),
    (2, 129, 128, 7, 3),
    (1, 500, 64, 11, 3),
    (3, 20, 32, 3, 5),
]


@pytest.mark.parametrize("case", SAME_CASES, ids=lambda c: "B{}L{}C{}k{}d{}".format(*c))
def test_same_padded_conv_matches_float64(gpu, case):
    batch, length, c, k, d = case
    gen = torch.Generator().manual_seed(length + 7 * k + d)
    x = bf(rand(batch, length, c, gen=gen))
    w = bf(rand(c, c, k, gen=gen, scale=1 / math.sqrt(c * k)))
    b = bf(rand(c, gen=gen, scale=0.1))
    packed = pack_conv1d(w, b, dilation=d, causal=False).to(gpu)
    out = torch.empty(batch, length, c, dtype=torch.float32, device=gpu)
    fused_conv(x.to(gpu, torch.bfloat16), packed, out)
    close(out, conv_ref64(x, w, b, dilation=d, causal=False), rtol=1e-5, atol=1e-5)


TRANSPOSE_CASES = [
    # (B, L, C_in, C_out, stride, k, padding)
    (1, 1, 192, 96, 6, 12, 0),
    (2, 12, 1536, 768, 8, 16, 0),
    (2, 40, 384, 192, 5, 10, 0),
    (1, 100, 192, 96, 6, 12, 0),
    (3, 7, 768, 384, 8, 16, 0),
    (2, 30, 512, 256, 8, 16, 4),
    (2, 50, 256, 128, 5, 11, 3),
    (1, 64, 128, 64, 3, 7, 2),
    (2, 90, 64, 32, 4, 8, 2),
]


@pytest.mark.parametrize("case", TRANSPOSE_CASES,
                         ids=lambda c: "B{}L{}ci{}co{}s{}k{}p{}".format(*c))
def test_polyphase_transposed_conv_matches_float64(gpu, case):
    batch, length, c_in, c_out, s, k, pad = case
    gen = torch.Generator().manual_seed(length * 13 + s + k)
    x = bf(rand(batch, length, c_in, gen=gen))
    w = bf(rand(c_in, c_out, k, gen=gen, scale=1 / math.sqrt(c_in * 2)))
    b = bf(rand(c_out, gen=gen, scale=0.1))
    packed = pack_conv_transpose1d(w, b, stride=s, padding=pad).to(gpu)
    out = torch.empty(batch, length * s, c_out, dtype=torch.float32, device=gpu)
    fused_conv(x.to(gpu, torch.bfloat16), packed, out.view(batch, length, s * c_out))
    close(out, convt_ref64(x, w, b, stride=s, padding=pad), rtol=1e-5, atol=1e-5)


def test_epilogue_snake_residual_sum_out_bf16(gpu):
    """v = conv + bias + residual; sum_out = v (float32); out = Snake(v) in bf16, Snake from the
    oracle's closed form in float64."""
    gen = torch.Generator().manual_seed(5)
    batch, length, c = 2, 333, 96
    x = bf(rand(batch, length, c, gen=gen))
    w = bf(rand(c, c, 7, gen=gen, scale=1 / math.sqrt(c * 7)))
    b = bf(rand(c, gen=gen, scale=0.1))
    resid = rand(batch, length, c, gen=gen)
    alpha = torch.rand(c, generator=gen) * 4 + 0.05
    packed = pack_conv1d(w, b, dilation=3).to(gpu)
    out = torch.empty(batch, length, c, dtype=torch.bfloat16, device=gpu)
    sum_out = torch.empty(batch, length, c, dtype=torch.float32, device=gpu)
    a_d = alpha.to(gpu)
    b_d = (alpha + 1e-9).reciprocal().to(gpu)
    fused_conv(x.to(gpu, torch.bfloat16), packed, out, activation=N.ACT_SNAKE, act_a=a_d,
               act_b=b_d, residual=resid.to(gpu), sum_out=sum_out)
    v = conv_ref64(x, w, b, dilation=3) + resid.double()
    close(sum_out, v, rtol=1e-5, atol=1e-5)
    expected = O.snake(v.transpose(1, 2), alpha.double()).transpose(1, 2)
    close(out.float(), expected, rtol=2**-8, atol=1e-5)


def test_epilogue_leaky_relu_mix_and_fp32_out(gpu):
    gen = torch.Generator().manual_seed(6)
    batch, length, c = 2, 200, 64
    x = bf(rand(batch, length, c, gen=gen))
    w = bf(rand(c, c, 3, gen=gen, scale=1 / math.sqrt(c * 3)))
    b = bf(rand(c, gen=gen, scale=0.1))
    resid, ma, mb = (rand(batch, length, c, gen=gen) for _ in range(3))
    packed = pack_conv1d(w, b, dilation=5, causal=False).to(gpu)
    out = torch.empty(batch, length, c, dtype=torch.float32, device=gpu)
    fused_conv(x.to(gpu, torch.bfloat16), packed, out, activation=N.ACT_LEAKY_RELU, slope=0.1,
               residual=resid.to(gpu), mix=(ma.to(gpu), mb.to(gpu), 1.0 / 3.0))
    v = ((ma.double() + mb.double()) + conv_ref64(x, w, b, dilation=5, causal=False)
         + resid.double()) / 3.0
    close(out, F.leaky_relu(v, 0.1), rtol=1e-5, atol=1e-5)


def test_fp8_weights_match_dequantized_reference(gpu):
    """W8A16: E4M3 weights with per-output-channel scales dequantized in LDS; the result equals the
    float64 conv with the dequantized weights (float32-accumulation tolerance)."""
    from sglang_omni_amd.quantization import dequantize_fp8, quantize_fp8

    gen = torch.Generator().manual_seed(8)
    batch, length, c_in, c_out = 2, 150, 192, 96
    x = bf(rand(batch, length, c_in, gen=gen))
    w = rand(c_out, c_in, 7, gen=gen, scale=1 / math.sqrt(c_in * 7))
    b = bf(rand(c_out, gen=gen, scale=0.1))
    q, s = quantize_fp8(w, 0)
    w_deq = dequantize_fp8(q, s, 0)
    packed = pack_conv1d(w, b, dilation=9, fp8=True).to(gpu)
    assert packed.weight.dtype == torch.float8_e4m3fn
    out = torch.empty(batch, length, c_out, dtype=torch.float32, device=gpu)
    fused_conv(x.to(gpu, torch.bfloat16), packed, out)
    close(out, conv_ref64(x, w_deq, b, dilation=9), rtol=1e-5, atol=1e-5)

    wt = rand(c_in, c_out, 12, gen=gen, scale=1 / math.sqrt(c_in * 2))
    qt, st = quantize_fp8(wt, 1)
    packed_t = pack_conv_transpose1d(wt, b, stride=6, fp8=True).to(gpu)
    out_t = torch.empty(batch, length * 6, c_out, dtype=torch.float32, device=gpu)
    fused_conv(x.to(gpu, torch.bfloat16), packed_t, out_t.view(batch, length, 6 * c_out))
    close(out_t, convt_ref64(x, dequantize_fp8(qt, st, 1), b, stride=6), rtol=1e-5, atol=1e-5)


def test_fp8_weight_decode_is_exact_for_every_encoding(gpu):
    """Every finite E4M3 encoding, at every byte position of the packed weights, reaches the MFMA
    as its exact value: a k = 1 conv with one-hot inputs returns one weight per output, which
    must equal torch's float8_e4m3fn -> float32 conversion times the channel's scale (a power of
    two, so the product is exact too)."""
    c_in, c_out = 32, 256
    codes = (torch.arange(c_out * c_in) * 37 % 256).to(torch.uint8)  # every byte, shuffled
    codes[(codes == 0x7F) | (codes == 0xFF)] = 0  # the two NaN encodings
    assert codes.unique().numel() == 254
    q = codes.view(torch.float8_e4m3fn).view(c_out, c_in, 1)
    scale = 2.0 ** torch.randint(-3, 4, (c_out,), generator=torch.Generator().manual_seed(3))
    packed = pack_conv1d(q, None, fp8=True, scale=scale.float()).to(gpu)
    x = torch.eye(c_in).view(1, c_in, c_in)  # position p holds channel p
    out = torch.empty(1, c_in, c_out, dtype=torch.float32, device=gpu)
    fused_conv(x.to(gpu, torch.bfloat16), packed, out)
    expect = (q.float()[:, :, 0] * scale[:, None]).t()  # [position = c_in, c_out]
    assert torch.equal(out[0].cpu(), expect)


@pytest.mark.parametrize("dilation", [1, 3, 9])
@pytest.mark.parametrize("chunks", [(10, 10, 7), (1, 2, 1, 3, 40), (32, 1, 32)])
def test_streamed_causal_conv_equals_the_whole_stream_bitwise(gpu, dilation, chunks):
    """Decoding a stream chunk by chunk with the slot history gives the same bits as one decode of
    the whole stream (the invariant of tests/unit_test/kernels/test_codec_state.py:52-94)."""
    gen = torch.Generator().manual_seed(dilation * 100 + len(chunks))
    batch, c = 2, 96
    total = sum(chunks)
    x = bf(rand(batch, total, c, gen=gen)).to(gpu, torch.bfloat16)
    w = bf(rand(c, c, 7, gen=gen, scale=1 / math.sqrt(c * 7)))
    packed = pack_conv1d(w, None, dilation=dilation).to(gpu)
    whole = torch.empty(batch, total, c, dtype=torch.float32, device=gpu)
    fused_conv(x, packed, whole)
    slots = 5
    hist = torch.randn(slots, 2, packed.left_pad, c, device=gpu).to(torch.bfloat16)
    untouched = hist[[0, 2, 4]].clone()
    slot_index = torch.tensor([3, 1], device=gpu)
    parity = torch.zeros(slots, dtype=torch.int64, device=gpu)
    lib = N.load_library()
    start = 0
    for i, n in enumerate(chunks):
        out = torch.empty(batch, n, c, dtype=torch.float32, device=gpu)
        fused_conv(x[:, start:start + n].contiguous(), packed, out, history=hist,
                   slot_index=slot_index, slot_parity=parity, history_cold=i == 0)
        N.check(lib.omni_advance_slots(parity.data_ptr(), parity.shape[0], slot_index.data_ptr(), batch,
                                       N.stream_handle()), "advance")
        assert torch.equal(out, whole[:, start:start + n]), f"chunk {i}"
        start += n
    torch.cuda.synchronize()
    assert torch.equal(hist[[0, 2, 4]], untouched)
    assert parity.tolist() == [0, len(chunks), 0, len(chunks), 0]
    # the slot's live copy holds the last left_pad samples of the zero-started stream
    context = F.pad(x.float(), (0, 0, packed.left_pad, 0)).to(torch.bfloat16)
    for row, slot in enumerate(slot_index.tolist()):
        live = hist[slot, parity[slot].item() & 1]
        assert torch.equal(live, context[row, -packed.left_pad:])


@pytest.mark.parametrize("stride", [5, 6, 8])
@pytest.mark.parametrize("chunks", [(4, 4, 2), (1, 1, 1, 5)])
def test_streamed_transposed_conv_equals_the_whole_stream_bitwise(gpu, stride, chunks):
    """The polyphase transposed conv's one-sample history reproduces the reference's overlap-add
    across chunks (tests/unit_test/kernels/test_codec_state.py:97-130), here bitwise."""
    gen = torch.Generator().manual_seed(stride + len(chunks))
    batch, c_in, c_out = 2, 192, 96
    total = sum(chunks)
    x = bf(rand(batch, total, c_in, gen=gen)).to(gpu, torch.bfloat16)
    w = bf(rand(c_in, c_out, 2 * stride, gen=gen, scale=0.05))
    packed = pack_conv_transpose1d(w, None, stride=stride).to(gpu)
    whole = torch.empty(batch, total * stride, c_out, dtype=torch.float32, device=gpu)
    fused_conv(x, packed, whole.view(batch, total, stride * c_out))
    close(whole, convt_ref64(x.float().cpu(), w, None, stride=stride), rtol=1e-5, atol=1e-5)
    hist = torch.zeros(4, 2, 1, c_in, dtype=torch.bfloat16, device=gpu)
    slot_index = torch.tensor([2, 0], device=gpu)
    parity = torch.zeros(4, dtype=torch.int64, device=gpu)
    lib = N.load_library()
    start = 0
    for i, n in enumerate(chunks):
        out = torch.empty(batch, n * stride, c_out, dtype=torch.float32, device=gpu)
        fused_conv(x[:, start:start + n].contiguous(), packed, out.view(batch, n, stride * c_out),
                   history=hist, slot_index=slot_index, slot_parity=parity, history_cold=i == 0)
        N.check(lib.omni_advance_slots(parity.data_ptr(), parity.shape[0], slot_index.data_ptr(), batch,
                                       N.stream_handle()), "advance")
        assert torch.equal(out, whole[:, start * stride:(start + n) * stride])
        start += n


def test_invalid_arguments_raise_before_launch(gpu):
    gen = torch.Generator().manual_seed(1)
    w = bf(rand(96, 96, 7, gen=gen))
    packed = pack_conv1d(w, None, dilation=1).to(gpu)
    x = torch.zeros(1, 10, 96, dtype=torch.bfloat16, device=gpu)
    with pytest.raises(ValueError):
        fused_conv(x, packed, torch.empty(1, 10, 64, device=gpu))
    with pytest.raises(ValueError):
        fused_conv(x.half(), packed, torch.empty(1, 10, 96, device=gpu))
    with pytest.raises(ValueError):  # an output may not alias the input
        xf = torch.zeros(1, 10, 96, device=gpu)
        fused_conv(xf, packed, xf)
    # a dilation whose halo exceeds the kernel's staging budget is refused by the library
    big = pack_conv1d(bf(rand(96, 96, 7, gen=gen)), None, dilation=27).to(gpu)
    with pytest.raises(N.OmniCodecError, match="status 2"):
        fused_conv(x, big, torch.empty(1, 10, 96, device=gpu))


def snake64(x: torch.Tensor, alpha: torch.Tensor) -> torch.Tensor:
    a = alpha.double().view(1, 1, -1)
    return x.double() + torch.sin(a * x.double()) ** 2 / (a + 1e-9)


@pytest.mark.parametrize("batch,length,c_in,c_out,k,d", [(3, 12, 192, 96, 7, 3), (2, 700, 96, 96, 7, 9),
                                                      (64, 12, 512, 256, 7, 1)])
def test_float32_input_with_the_snake_staged(gpu, batch, length, c_in, c_out, k, d):
    """x float32 -> Snake per input channel -> bf16 operand, as the decoder feeds every conv."""
    gen = torch.Generator().manual_seed(length + c_in)
    x = rand(batch, length, c_in, gen=gen)
    alpha = torch.rand(c_in, generator=gen) + 0.5
    w = bf(rand(c_out, c_in, k, gen=gen, scale=1 / math.sqrt(c_in * k)))
    b = rand(c_out, gen=gen, scale=0.1)
    packed = pack_conv1d(w, b, dilation=d).to(gpu)
    out = torch.empty(batch, length, c_out, dtype=torch.float32, device=gpu)
    a_d = alpha.to(gpu)
    fused_conv(x.to(gpu), packed, None, sum_out=out, in_activation=N.ACT_SNAKE, in_a=a_d,
               in_b=(a_d + 1e-9).reciprocal())
    u = bf(snake64(x, alpha).float())  # the staged operand: Snake in float32, rounded to bf16
    # the GPU's float32 Snake and this float64 one round to different bf16 neighbours for a few
    # operands (one bf16 ulp of the operand times a weight): a loose bound on every output, and a
    # float32-summation bound on almost all of them
    expected = conv_ref64(u, w, b, dilation=d)
    close(out, expected, rtol=0, atol=2e-3)
    err = (out.cpu().double() - expected).abs()
    assert (err > 1e-4).double().mean().item() < 0.01


@pytest.mark.parametrize("channels", [96, 192])
@pytest.mark.parametrize("batch,length,d", [(1, 500, 1), (3, 37, 9), (64, 12, 3)])
def test_fused_residual_unit_matches_float64(gpu, channels, batch, length, d):
    """x + conv1x1(Snake2(conv7_d(Snake1(x)))) in one launch: the k = 1 conv runs on the bf16
    tile the first conv leaves in LDS."""
    gen = torch.Generator().manual_seed(channels + length + d)
    c = channels
    x = rand(batch, length, c, gen=gen)
    a1 = torch.rand(c, generator=gen) + 0.5
    a2 = torch.rand(c, generator=gen) + 0.5
    w1 = bf(rand(c, c, 7, gen=gen, scale=1 / math.sqrt(c * 7)))
    b1 = rand(c, gen=gen, scale=0.1)
    w2 = bf(rand(c, c, 1, gen=gen, scale=1 / math.sqrt(c)))
    b2 = rand(c, gen=gen, scale=0.1)
    p1 = pack_conv1d(w1, b1, dilation=d).to(gpu)
    p2 = pack_conv1d(w2, b2).to(gpu)
    xd = x.to(gpu)
    out = torch.empty(batch, length, c, dtype=torch.float32, device=gpu)
    a1d, a2d = a1.to(gpu), a2.to(gpu)
    fused_conv(xd, p1, None, sum_out=out, residual=xd, second=p2, in_activation=N.ACT_SNAKE,
               in_a=a1d, in_b=(a1d + 1e-9).reciprocal(), mid_activation=N.ACT_SNAKE, mid_a=a2d,
               mid_b=(a2d + 1e-9).reciprocal())
    u = bf(snake64(x, a1).float())
    h = bf(snake64(conv_ref64(u, w1, b1, dilation=d).float(), a2).float())
    expected = x.double() + conv_ref64(h, w2, b2)
    # h is rounded to bf16 from a float32 sum on the GPU and a float64 one here: one bf16 ulp of h
    # may differ, which the k = 1 conv spreads over its channels
    close(out, expected, rtol=0, atol=3e-2)
    err = (out.cpu().double() - expected).abs()
    assert err.mean().item() < 2e-3
