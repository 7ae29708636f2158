"""Conv1d and ConvTranspose1d of (B, L, C) activations on the HIP MFMA conv, with the signatures
of sglang_omni/utils/channels_last_conv.py:45-120.

Weights are packed per call here (the reference passes a channels-last weight view); decoders
pack once at load time with ``sglang_omni_amd.kernels.conv.pack_*`` instead.
"""

from __future__ import annotations

import torch

from ..kernels.conv import fused_conv, pack_conv1d, pack_conv_transpose1d


def channels_last_conv1d(
    hidden_states: torch.Tensor,
    conv: torch.nn.Conv1d,
    weight: torch.Tensor,
    bias: torch.Tensor | None,
    length: int,
) -> torch.Tensor:
    """The stride-one conv of a (B, L, C) bf16 activation that carries its left context: the
    first ``length`` output rows, (B, length, C_out) float32."""
    if conv.stride[0] != 1 or conv.groups != 1:
        raise NotImplementedError("only stride-one, ungrouped convs run on the MFMA conv")
    dilation = conv.dilation[0]
    packed = pack_conv1d(weight.contiguous(), bias, dilation=dilation, causal=True)
    packed.left_pad = 0  # the input already carries its left context
    packed = packed.to(hidden_states.device)
    x = hidden_states.to(torch.bfloat16)
    out = torch.empty(x.shape[0], length, packed.n_cols, dtype=torch.float32, device=x.device)
    return fused_conv(x, packed, out, length=length, x_length=x.shape[1])


def channels_last_conv_transpose1d(
    hidden_states: torch.Tensor,
    conv: torch.nn.ConvTranspose1d,
    weight: torch.Tensor,
    bias: torch.Tensor | None,
) -> torch.Tensor:
    """The transposed conv (no padding, no output padding) of a (B, L, C) activation, returned as
    (B, (L-1)*s + k, C_out) float32."""
    if conv.padding[0] != 0 or conv.output_padding[0] != 0 or conv.groups != 1 or conv.dilation[0] != 1:
        raise NotImplementedError("only unpadded, ungrouped, undilated transposed convs")
    stride = conv.stride[0]
    k = weight.shape[-1]
    batch, length, _ = hidden_states.shape
    # every full output sample: extend by ceil(k/s) - 1 zero input positions on the right
    extra = (k + stride - 1) // stride - 1
    packed = pack_conv_transpose1d(weight.contiguous(), bias, stride=stride).to(hidden_states.device)
    x = hidden_states.to(torch.bfloat16)
    out = torch.empty(batch, length + extra, packed.n_cols, dtype=torch.float32, device=x.device)
    fused_conv(x, packed, out, length=length + extra, x_length=length)
    full = out.view(batch, (length + extra) * stride, packed.c_out)
    return full[:, : (length - 1) * stride + k]
