"""A stride-one, undilated conv from channels-last activations to one output channel, its bias
added and the result clamped to [-1, 1] (or tanh), accumulated in fp32 and rounded once —
``clamped_single_output_conv`` of sglang_omni/kernels/single_output_conv.py:62-102."""

from __future__ import annotations

import torch

from .. import _native as N


def clamped_single_output_conv(
    padded: torch.Tensor, conv: torch.nn.Conv1d, length: int, *, activation: str = "clamp"
) -> torch.Tensor:
    """The (B, 1, length) outputs of a stride-one, undilated, ungrouped conv to one output channel
    over a (B, length + kernel - 1, C) activation that carries its left context, its bias added
    and clamped to [-1, 1] (``activation="tanh"`` applies tanh instead)."""
    N.require_device(padded)
    batch_size, padded_length, channels = padded.shape
    taps = conv.kernel_size[0]
    if not (conv.out_channels == 1 and conv.stride == (1,) and conv.dilation == (1,)
            and conv.groups == 1):
        raise ValueError("a stride-one, undilated, ungrouped conv to one output channel")
    if padded_length != length + taps - 1:
        raise ValueError("the input carries the left context")
    if padded.stride(2) != 1 or padded.stride(1) != channels:
        raise ValueError("contiguous rows")
    if conv.in_channels != channels:
        raise ValueError(f"the conv takes {conv.in_channels} channels, the input has {channels}")
    weight = conv.weight.detach().float()[0].t().contiguous()  # [taps, C]
    bias = None if conv.bias is None else conv.bias.detach().float().contiguous()
    for t in (weight, bias):
        if t is not None and t.device != padded.device:
            raise ValueError(f"the conv's parameters are on {t.device}, the input on {padded.device}")
    output = padded.new_empty(batch_size, 1, length)
    act = {"clamp": N.ACT_CLAMP, "tanh": N.ACT_TANH, "none": N.ACT_NONE}[activation]
    context = padded[:, taps - 1 :]
    lib = N.load_library()
    N.check(
        lib.omni_single_output_conv(
            context.data_ptr(), N.omni_dtype(padded.dtype), padded.stride(0), padded.stride(1),
            batch_size, length, channels, 1, N.ACT_NONE, None, None, weight.data_ptr(),
            N.ptr(bias), taps, taps - 1,
            None, None, None, 0, 0, 0, act, output.data_ptr(), N.omni_dtype(output.dtype),
            output.stride(0), N.stream_handle(padded.device),
        ),
        "omni_single_output_conv",
    )
    return output


def single_output_conv(
    x: torch.Tensor,
    weight: torch.Tensor,
    bias: torch.Tensor | None,
    out: torch.Tensor,
    *,
    activation: int,
    left_pad: int,
    in_activation: int = N.ACT_NONE,
    in_a: torch.Tensor | None = None,
    in_b: torch.Tensor | None = None,
    history: torch.Tensor | None = None,
    slot_index: torch.Tensor | None = None,
    slot_parity: torch.Tensor | None = None,
    history_cold: bool = False,
) -> torch.Tensor:
    """Decoder form: x [B, L, C] (no context in the buffer; zeros or slot history left of 0,
    zeros right of L), activated per channel by ``in_activation`` (Snake with in_a / in_b),
    weight [taps, C] float32, out [B, 1, L]."""
    N.require_device(x, out, weight)
    dev = x.device
    batch, length, channels = x.shape
    taps = weight.shape[0]
    if (weight.dtype != torch.float32 or tuple(weight.shape) != (taps, channels)
            or not weight.is_contiguous() or weight.device != dev):
        raise ValueError(f"weight must be contiguous float32 [taps, {channels}] on {dev}")
    if out.device != dev or out.dim() != 3 or out.shape[0] != batch or out.shape[2] < length:
        raise ValueError(f"out must be [{batch}, 1, >= {length}] on {dev}")
    N.require_vector(bias, 1, "bias", dev)
    if in_activation == N.ACT_SNAKE:
        if in_a is None or in_b is None:
            raise ValueError("a Snake input activation needs in_a and in_b")
        N.require_vector(in_a, channels, "in_a", dev)
        N.require_vector(in_b, channels, "in_b", dev)
    N.require_slot_state(history, slot_index, slot_parity, rows=batch, samples=left_pad,
                         channels=channels, device=dev, what="single_output_conv")
    lib = N.load_library()
    N.check(
        lib.omni_single_output_conv(
            x.data_ptr(), N.omni_dtype(x.dtype), x.stride(0), x.stride(1), batch, length,
            channels, 0, in_activation, N.ptr(in_a), N.ptr(in_b), weight.data_ptr(), N.ptr(bias),
            taps, left_pad, N.ptr(history),
            N.ptr(slot_index), N.ptr(slot_parity), 0 if history is None else history.shape[0],
            0 if history is None else history.stride(0),
            int(history_cold), activation, out.data_ptr(), N.omni_dtype(out.dtype),
            out.stride(0), N.stream_handle(x.device),
        ),
        "omni_single_output_conv",
    )
    return out
