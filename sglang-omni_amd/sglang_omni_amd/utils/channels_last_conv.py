"""Conv1d and ConvTranspose1d of (B, L, C) activations, with the signatures and results of
sglang_omni/utils/channels_last_conv.py:17-120, on the HIP kernels.

* ``channels_last_conv1d(x, conv, weight, bias, length)``: x carries its left context; a
  stride-one undilated conv returns every output row, a dilated one the first ``length`` rows,
  and a strided one (given ``channels_last_folded_weight`` of its weight and an input whose
  length is a multiple of the stride) the first ``length`` rows of the stride-one conv over the
  input's stride phases laid along the channels.
* ``channels_last_conv_transpose1d(x, conv, weight, bias)``: the transposed conv with the
  module's stride, padding, output padding, groups and dilation, as (B, L_out, C_out).

Both return x's dtype. bf16 convs whose shapes the MFMA conv kernel takes (ungrouped, input
channels a multiple of 8, output columns a multiple of 16, dilated reach <= 64 samples) run
there, their weights packed once per weight tensor version; every other call (float32 / fp16,
grouped and depthwise convs, odd channel counts) runs ``omni_conv1d_general`` on the weight as
it is. Decoders pack their weights at load time with ``kernels.conv.pack_*`` instead.
"""

from __future__ import annotations

import weakref

import torch

from .. import _native as N
from ..kernels.conv import PackedConv, fused_conv, pack_conv1d, pack_conv_transpose1d

_DTYPES = (torch.float32, torch.bfloat16, torch.float16)


def channels_last_strides(weight: torch.Tensor) -> torch.Tensor:
    """A (C_out, C_in, k) weight's values with channels-last strides (its (C_out, k, C_in)
    transpose contiguous)."""
    return weight.transpose(1, 2).contiguous().transpose(1, 2)


def channels_last_weight(conv: torch.nn.Conv1d | torch.nn.ConvTranspose1d) -> torch.Tensor:
    """The module's weight with channels-last strides; the module keeps its own."""
    return channels_last_strides(conv.weight.data)


def channels_last_folded_weight(weight: torch.Tensor, stride: int) -> torch.Tensor:
    """The (C_out, C_in, k) weight of a stride-s conv as the (C_out, s * C_in, k / s) weight of
    the stride-one conv over the input's s phases laid along its channels: tap m of phase r is
    the original tap m * s + r, at input channel r * C_in + c."""
    c_out, c_in, k = weight.shape
    if k % stride:
        raise ValueError(f"a {k}-tap kernel does not fold into whole phases of stride {stride}")
    taps = k // stride
    folded = weight.reshape(c_out, c_in, taps, stride).permute(0, 3, 1, 2)
    return channels_last_strides(folded.reshape(c_out, stride * c_in, taps))


# ---------------------------------------------------------------------------- packed weights

# id(weight) -> (weak reference to the weight, key, packing); an entry leaves with its weight
_packed: dict[int, tuple[weakref.ref, tuple, PackedConv]] = {}


def _cached_pack(weight: torch.Tensor, key: tuple, make) -> PackedConv:
    """The MFMA packing of `weight` for `key`, made once per weight tensor and version."""
    full_key = (weight._version, weight.device) + key
    entry = _packed.get(id(weight))
    if entry is not None and entry[0]() is weight and entry[1] == full_key:
        return entry[2]
    packed = make().to(weight.device)
    if entry is None or entry[0]() is not weight:
        weakref.finalize(weight, _packed.pop, id(weight), None)
    _packed[id(weight)] = (weakref.ref(weight), full_key, packed)
    return packed


def _mfma_ok(x: torch.Tensor, c_in: int, n_cols: int, c_out: int, reach: int) -> bool:
    return (x.dtype == torch.bfloat16 and c_in % 8 == 0 and n_cols % 16 == 0 and c_out % 4 == 0
            and reach <= 64)


def _general(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None, *, c_out: int,
             groups: int, stride: int, dilation: int, pad_left: int, transposed: bool,
             length_out: int) -> torch.Tensor:
    batch, length_in, c_in = x.shape
    dt = x.dtype
    w = weight.detach()
    b = None if bias is None else bias.detach().to(dt).contiguous()
    if w.dtype != dt:
        w = w.to(dt)
    for t, name in ((w, "weight"), (b, "bias")):
        if t is not None and t.device != x.device:
            raise ValueError(f"the conv's {name} is on {t.device}, the input on {x.device}")
    y = torch.empty(batch, length_out, c_out, dtype=dt, device=x.device)
    lib = N.load_library()
    N.check(lib.omni_conv1d_general(
        x.data_ptr(), N.omni_dtype(dt), batch, length_in, c_in, *x.stride(), w.data_ptr(),
        w.shape[2], *w.stride(), N.ptr(b), c_out, groups, stride, dilation, pad_left,
        int(transposed), y.data_ptr(), length_out, *y.stride(), N.stream_handle(x.device)),
        "omni_conv1d_general")
    return y


def _check_input(x: torch.Tensor) -> None:
    N.require_device(x)
    if x.dim() != 3:
        raise ValueError(f"channels-last activations are (B, L, C); got {tuple(x.shape)}")
    if x.dtype not in _DTYPES:
        raise ValueError(f"the conv kernels take float32, bf16 or fp16 activations, not {x.dtype}")


# ---------------------------------------------------------------------------- the API


def channels_last_conv1d(hidden_states: torch.Tensor, conv: torch.nn.Conv1d,
                         weight: torch.Tensor, bias: torch.Tensor | None,
                         length: int) -> torch.Tensor:
    """The conv of a (B, L, C) activation that carries its left context (see the module
    docstring for which rows come back); (B, rows, C_out) in x's dtype, contiguous."""
    _check_input(hidden_states)
    dilation, stride, groups = conv.dilation[0], conv.stride[0], conv.groups
    if stride > 1 and (dilation != 1 or groups != 1):
        raise ValueError("a strided conv folds only when undilated and ungrouped")
    x = hidden_states
    if stride > 1:
        batch, padded, channels = x.shape
        if padded % stride:
            raise ValueError(f"{padded} input rows do not fold into whole phases of {stride}")
        x = x.reshape(batch, padded // stride, stride * channels)
    batch, length_in, c_in = x.shape
    c_out, _, taps = weight.shape
    if weight.shape[1] * groups != c_in:
        raise ValueError(f"the weight takes {weight.shape[1] * groups} input channels, the input "
                         f"has {c_in}")
    reach = (taps - 1) * dilation
    rows = length_in - reach if stride == 1 and dilation == 1 else length
    if rows < 0 or rows > length_in - reach:
        raise ValueError(f"{length_in} input rows give {length_in - reach} outputs, not {rows}")
    if groups == 1 and _mfma_ok(x, c_in, c_out, c_out, reach):
        if not x.is_contiguous() and (x.stride(2) != 1 or x.stride(1) % 8 or x.stride(0) % 8):
            x = x.contiguous()
        packed = _cached_pack(weight, ("conv", dilation), lambda: _with_left_pad(
            pack_conv1d(weight.detach(), None, dilation=dilation), 0))
        if bias is not None:
            packed = _with_bias(packed, bias, x.device)
        out = torch.empty(batch, rows, c_out, dtype=torch.bfloat16, device=x.device)
        fused_conv(x, packed, out, length=rows, x_length=length_in)
        return out
    return _general(x.contiguous() if x.stride(2) != 1 else x, weight, bias, c_out=c_out,
                    groups=groups, stride=1, dilation=dilation, pad_left=0, transposed=False,
                    length_out=rows)


def channels_last_conv_transpose1d(hidden_states: torch.Tensor, conv: torch.nn.ConvTranspose1d,
                                   weight: torch.Tensor,
                                   bias: torch.Tensor | None) -> torch.Tensor:
    """The transposed conv of a (B, L, C) activation with the module's stride, padding, output
    padding, groups and dilation: (B, (L-1)*s - 2p + d(k-1) + op + 1, C_out) in x's dtype."""
    _check_input(hidden_states)
    x = hidden_states
    stride, padding = conv.stride[0], conv.padding[0]
    output_padding, dilation, groups = conv.output_padding[0], conv.dilation[0], conv.groups
    batch, length_in, c_in = x.shape
    w_in, c_out_g, taps = weight.shape
    if w_in != c_in:
        raise ValueError(f"the weight takes {w_in} input channels, the input has {c_in}")
    c_out = c_out_g * groups
    length_out = (length_in - 1) * stride - 2 * padding + dilation * (taps - 1) + output_padding + 1
    if length_out < 0:
        raise ValueError("the transposed conv's padding removes more than it produces")
    reach = dilation * (taps - 1)
    if groups == 1 and _mfma_ok(x, c_in, stride * c_out, c_out, reach):
        if x.stride(2) != 1 or x.stride(1) % 8 or x.stride(0) % 8:
            x = x.contiguous()
        packed = _cached_pack(weight, ("transpose", stride, padding, dilation),
                              lambda: pack_conv_transpose1d(
                                  weight.detach(), None, stride=stride, padding=padding,
                                  dilation=dilation))
        if bias is not None:
            packed = _with_bias(packed, bias, x.device)
        if packed.taps <= 11:
            positions = -(-length_out // stride)
            out = torch.empty(batch, positions, stride * c_out, dtype=torch.bfloat16,
                              device=x.device)
            fused_conv(x, packed, out, length=positions, x_length=length_in)
            return out.view(batch, positions * stride, c_out)[:, :length_out]
    return _general(x if x.stride(2) == 1 else x.contiguous(), weight, bias, c_out=c_out,
                    groups=groups, stride=stride, dilation=dilation, pad_left=padding,
                    transposed=True, length_out=length_out)


def _with_left_pad(packed: PackedConv, left_pad: int) -> PackedConv:
    packed.left_pad = left_pad
    return packed


def _with_bias(packed: PackedConv, bias: torch.Tensor, device: torch.device) -> PackedConv:
    """The packing with the call's bias (float32 on the device): the bias is an argument of
    every call, not part of the cached packing."""
    b = bias.detach().to(device=device, dtype=torch.float32).contiguous()
    return PackedConv(packed.weight, packed.scale, b, packed.c_in, packed.c_out, packed.n_cols,
                      packed.taps, packed.dilation, packed.left_pad, packed.phases,
                      packed.macs_per_position)


__all__ = ["channels_last_conv1d", "channels_last_conv_transpose1d", "channels_last_folded_weight",
           "channels_last_strides", "channels_last_weight"]
