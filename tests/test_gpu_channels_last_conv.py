"""The channels-last conv API on the GPU, the reference's tests restated (tests/unit_test/utils/
test_channels_last_conv.py:18-115) plus the cases its decoders run.

The reference's own cases (4 -> 6 channels, float32) take ``omni_conv1d_general``: float32
accumulation of float32 products, held to the float64 conv at float32 tolerance (assert_close's
defaults for float32, the reference's bound). bf16 cases whose shapes the MFMA kernel takes run
there, and are held to the float64 conv of the same bf16 operands at one bf16 rounding of the
output (rtol 2^-8)."""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from sglang_omni_amd.utils.channels_last_conv import (
    channels_last_conv1d,
    channels_last_conv_transpose1d,
    channels_last_folded_weight,
    channels_last_weight,
)

pytestmark = pytest.mark.gpu


def expected_causal(inputs, conv, left, *, stride=1):
    """F.conv1d in float64 on the CPU of the causally padded input (B, L, C) -> (B, L', C_out)."""
    x = F.pad(inputs.double().cpu().transpose(1, 2), (left, 0))
    y = F.conv1d(x, conv.weight.double().cpu(), None if conv.bias is None else conv.bias.double().cpu(),
                 stride=stride, dilation=conv.dilation, groups=conv.groups)
    return y.transpose(1, 2)


@pytest.mark.parametrize("length", [1, 5, 16])
@pytest.mark.parametrize("dilation,groups", [(1, 1), (3, 1), (9, 1), (1, 2), (3, 2)])
def test_conv1d_matches_the_causal_conv1d(gpu, length, dilation, groups):
    torch.manual_seed(length * 10 + dilation)
    conv = torch.nn.Conv1d(4, 6, 7, dilation=dilation, groups=groups).to(gpu)
    left = (7 - 1) * dilation
    inputs = torch.randn(2, length, 4, device=gpu)
    padded = F.pad(inputs, (0, 0, left, (-length) % dilation))
    actual = channels_last_conv1d(padded, conv, channels_last_weight(conv), conv.bias, length)
    torch.testing.assert_close(actual.double().cpu(), expected_causal(inputs, conv, left),
                               rtol=1.3e-6, atol=1e-5)


@pytest.mark.parametrize("length", [60, 61])
@pytest.mark.parametrize("stride,kernel_size", [(3, 6), (15, 30)])
def test_conv1d_matches_the_strided_causal_conv1d(gpu, length, stride, kernel_size):
    torch.manual_seed(stride)
    conv = torch.nn.Conv1d(4, 6, kernel_size, stride=stride).to(gpu)
    inputs = torch.randn(2, length, 4, device=gpu)
    outputs = (stride - 1 + length - kernel_size) // stride + 1
    padded = F.pad(inputs, (0, 0, stride - 1, (-(stride - 1 + length)) % stride))
    actual = channels_last_conv1d(padded, conv, channels_last_folded_weight(conv.weight.data, stride),
                                  conv.bias, outputs)
    assert actual.is_contiguous()
    torch.testing.assert_close(actual.double().cpu(),
                               expected_causal(inputs, conv, stride - 1, stride=stride),
                               rtol=1.3e-6, atol=1e-5)


@pytest.mark.parametrize("has_bias", [True, False])
@pytest.mark.parametrize("stride,padding,output_padding", [(2, 0, 0), (4, 1, 1)])
def test_conv_transpose1d_matches_the_conv_transpose1d(gpu, has_bias, stride, padding,
                                                      output_padding):
    torch.manual_seed(stride)
    conv = torch.nn.ConvTranspose1d(4, 6, 8, stride=stride, padding=padding,
                                    output_padding=output_padding).to(gpu)
    bias = conv.bias if has_bias else None
    inputs = torch.randn(2, 9, 4, device=gpu)
    expected = F.conv_transpose1d(inputs.double().cpu().transpose(1, 2), conv.weight.double().cpu(),
                                  None if bias is None else bias.double().cpu(), stride=stride,
                                  padding=padding, output_padding=output_padding).transpose(1, 2)
    actual = channels_last_conv_transpose1d(inputs, conv, channels_last_weight(conv), bias)
    torch.testing.assert_close(actual.double().cpu(), expected, rtol=1.3e-6, atol=1e-5)


# --------------------------------------------------------------------- the decoders' shapes


def bf(t):
    return t.to(torch.bfloat16)


@pytest.mark.parametrize("c_in,c_out,dilation,length", [(96, 96, 9, 300), (512, 1536, 1, 12),
                                                        (192, 192, 3, 64)])
def test_bf16_conv1d_on_the_mfma_kernel(gpu, c_in, c_out, dilation, length):
    torch.manual_seed(c_in + dilation)
    conv = torch.nn.Conv1d(c_in, c_out, 7, dilation=dilation).to(gpu).to(torch.bfloat16)
    left = 6 * dilation
    inputs = bf(torch.randn(3, length, c_in, device=gpu))
    padded = F.pad(inputs, (0, 0, left, 0))
    weight = channels_last_weight(conv)
    actual = channels_last_conv1d(padded, conv, weight, conv.bias, length)
    assert actual.dtype == torch.bfloat16 and actual.shape == (3, length, c_out)
    torch.testing.assert_close(actual.double().cpu(), expected_causal(inputs, conv, left),
                               rtol=2 ** -8, atol=1e-4)
    again = channels_last_conv1d(padded, conv, weight, conv.bias, length)  # packed weights reused
    assert torch.equal(again, actual)


@pytest.mark.parametrize("c_in,c_out,stride,padding,output_padding,dilation", [
    (1536, 768, 8, 0, 0, 1), (192, 96, 6, 3, 0, 1), (256, 128, 5, 3, 1, 1), (64, 32, 4, 2, 0, 2)])
def test_bf16_conv_transpose1d_on_the_mfma_kernel(gpu, c_in, c_out, stride, padding,
                                                  output_padding, dilation):
    torch.manual_seed(c_in + stride)
    conv = torch.nn.ConvTranspose1d(c_in, c_out, 2 * stride, stride=stride, padding=padding,
                                    output_padding=output_padding, dilation=dilation)
    conv = conv.to(gpu).to(torch.bfloat16)
    inputs = bf(torch.randn(2, 13, c_in, device=gpu))
    actual = channels_last_conv_transpose1d(inputs, conv, channels_last_weight(conv), conv.bias)
    expected = F.conv_transpose1d(inputs.double().cpu().transpose(1, 2), conv.weight.double().cpu(),
                                  conv.bias.double().cpu(), stride=stride, padding=padding,
                                  output_padding=output_padding, dilation=dilation).transpose(1, 2)
    assert actual.dtype == torch.bfloat16
    torch.testing.assert_close(actual.double().cpu(), expected, rtol=2 ** -8, atol=1e-4)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_depthwise_and_grouped_convs_in_every_dtype(gpu, dtype):
    """ConvNeXt's depthwise causal conv (groups = channels) and a grouped transposed conv, in
    the three activation dtypes: float32 accumulation rounded once to the dtype."""
    torch.manual_seed(3)
    tol = {torch.bfloat16: 2 ** -8, torch.float16: 2 ** -11, torch.float32: 1.3e-6}[dtype]
    dw = torch.nn.Conv1d(64, 64, 7, groups=64).to(gpu).to(dtype)
    inputs = torch.randn(2, 40, 64, device=gpu).to(dtype)
    padded = F.pad(inputs, (0, 0, 6, 0))
    actual = channels_last_conv1d(padded, dw, channels_last_weight(dw), dw.bias, 40)
    assert actual.dtype == dtype
    torch.testing.assert_close(actual.double().cpu(), expected_causal(inputs, dw, 6),
                               rtol=tol, atol=1e-4)
    up = torch.nn.ConvTranspose1d(32, 48, 6, stride=3, padding=1, groups=4).to(gpu).to(dtype)
    x = torch.randn(2, 11, 32, device=gpu).to(dtype)
    got = channels_last_conv_transpose1d(x, up, channels_last_weight(up), up.bias)
    want = F.conv_transpose1d(x.double().cpu().transpose(1, 2), up.weight.double().cpu(),
                              up.bias.double().cpu(), stride=3, padding=1, groups=4).transpose(1, 2)
    torch.testing.assert_close(got.double().cpu(), want, rtol=tol, atol=1e-4)
