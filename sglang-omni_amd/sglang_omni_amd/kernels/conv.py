"""Fused polyphase convolution on bf16 MFMA: weight packing and the ``omni_conv1d_fused`` launch.

A stride-one Conv1d (any dilation, causal or 'same' padding) and a ConvTranspose1d (any stride
and padding) are both computed as

    out[b, i, n] = act(sum_j sum_ci Wp[n, j, ci] * x[b, i + j*d - left_pad, ci] + bias[n % C_out] ...)

with ``n`` running over ``phases * C_out`` columns. For the transposed conv, output sample
``s*i + r`` of channel ``co`` is column ``n = r*C_out + co`` of position ``i``, so the kernel's
``[B, L, s*C_out]`` output *is* the transposed conv's ``[B, L*s, C_out]`` output (channels-last).
This replaces ``channels_last_conv1d`` / ``channels_last_conv_transpose1d``
(sglang_omni/utils/channels_last_conv.py:45-120) and, with history, the exchange kernels around
them (sglang_omni/kernels/codec_state.py:150-210).
"""

from __future__ import annotations

import ctypes
from contextlib import contextmanager
from dataclasses import dataclass

import torch

from .. import _native as N

CHUNK = 32


@dataclass
class PackedConv:
    """A conv's weights in the kernel's layout plus its geometry.

    weight: [ceil(C_in/32), n_cols, taps, 32] bf16 (or float8_e4m3fn with ``scale[n_cols]``).
    """

    weight: torch.Tensor
    scale: torch.Tensor | None
    bias: torch.Tensor | None  # float32 [C_out]
    c_in: int
    c_out: int
    n_cols: int
    taps: int
    dilation: int
    left_pad: int
    phases: int
    macs_per_position: int = 0  # algorithmic multiply-adds per output (conv) / input (transposed) position

    @property
    def history(self) -> int:
        """Input samples a streaming (causal) decode keeps per slot."""
        return self.left_pad

    def to(self, device: torch.device) -> "PackedConv":
        return PackedConv(
            weight=self.weight.to(device),
            scale=None if self.scale is None else self.scale.to(device),
            bias=None if self.bias is None else self.bias.to(device),
            c_in=self.c_in, c_out=self.c_out, n_cols=self.n_cols, taps=self.taps,
            dilation=self.dilation, left_pad=self.left_pad, phases=self.phases,
            macs_per_position=self.macs_per_position,
        )


def _chunked(w: torch.Tensor) -> torch.Tensor:
    """[n_cols, taps, C_in] -> [ceil(C_in/32), n_cols, taps, 32], zero-padded channels."""
    n_cols, taps, c_in = w.shape
    chunks = (c_in + CHUNK - 1) // CHUNK
    padded = torch.zeros(n_cols, taps, chunks * CHUNK, dtype=w.dtype, device=w.device)
    padded[..., :c_in] = w
    return padded.view(n_cols, taps, chunks, CHUNK).permute(2, 0, 1, 3).contiguous()


def polyphase_taps(weight: torch.Tensor, stride: int, padding: int,
                   dilation: int = 1) -> tuple[torch.Tensor, int]:
    """A ConvTranspose1d weight [C_in, C_out, k] of stride s, padding p and dilation d as the
    stride-one weight [s*C_out, taps, C_in] over the input: output s*i + r is the transposed
    conv's sample s*i + r + p, which input q reaches through tap j when q*s + j*d = s*i + r + p,
    i.e. q = i + delta with delta = (r + p - j*d) / s for the taps j that make it whole.
    Returns (weight, left_pad) with tap index delta - min(delta)."""
    c_in, c_out, k = weight.shape
    s = stride
    entries = []  # (r, delta, j)
    for r in range(s):
        for j in range(k):
            num = r + padding - j * dilation
            if num % s == 0:
                entries.append((r, num // s, j))
    if not entries:
        raise ValueError("no tap reaches any output phase")
    d_min = min(e[1] for e in entries)
    d_max = max(e[1] for e in entries)
    taps = d_max - d_min + 1
    out = torch.zeros(s * c_out, taps, c_in, dtype=weight.dtype, device=weight.device)
    wt = weight.permute(1, 0, 2)  # [C_out, C_in, k]
    for r, delta, j in entries:
        out[r * c_out:(r + 1) * c_out, delta - d_min, :] += wt[:, :, j]
    return out, -d_min


def _finish(w_ntc: torch.Tensor, bias: torch.Tensor | None, *, c_in: int, c_out: int, taps: int,
            dilation: int, left_pad: int, phases: int, fp8: bool,
            scale: torch.Tensor | None = None) -> PackedConv:
    if fp8 and scale is not None:
        # an E4M3 weight with its per-output-channel scale (held exactly in float32 here)
        q = w_ntc.to(torch.float8_e4m3fn)
        scale_n = scale.float().reshape(c_out).repeat(phases).contiguous()
        return PackedConv(_chunked(q), scale_n, None if bias is None else bias.float(), c_in,
                          c_out, phases * c_out, taps, dilation, left_pad, phases)
    if fp8:
        # per-output-channel scales (shared by every phase of a transposed conv's channel)
        w = w_ntc.float().contiguous()
        amax = w.view(phases, c_out, -1).abs().amax(dim=(0, 2))
        scale_co = torch.where(amax > 0, amax / 448.0, torch.ones_like(amax))
        scale = scale_co.repeat(phases)
        q = (w / scale[:, None, None]).to(torch.float8_e4m3fn)
        return PackedConv(_chunked(q), scale.contiguous(), None if bias is None else bias.float(),
                          c_in, c_out, phases * c_out, taps, dilation, left_pad, phases)
    return PackedConv(_chunked(w_ntc.to(torch.bfloat16)), None,
                      None if bias is None else bias.float(), c_in, c_out, phases * c_out, taps,
                      dilation, left_pad, phases)


def pack_conv1d(weight: torch.Tensor, bias: torch.Tensor | None, *, dilation: int = 1,
                causal: bool = True, fp8: bool = False,
                scale: torch.Tensor | None = None) -> PackedConv:
    """Conv1d weight [C_out, C_in, k]: causal (left pad (k-1)*d, ``CausalConvNet``,
    modded_dac.py:541-572) or 'same' (pad (k*d-d)//2, hift_layers.py:67-92). An E4M3 weight
    comes with its float32 ``scale`` per output channel and is packed as it is."""
    c_out, c_in, k = weight.shape
    left = (k - 1) * dilation if causal else (k * dilation - dilation) // 2
    if weight.dtype == torch.float8_e4m3fn:
        if scale is None:
            raise ValueError("an E4M3 weight needs its per-output-channel scale")
        fp8, weight = True, weight.float()  # E4M3 values are exact in float32
    packed = _finish(weight.permute(0, 2, 1), bias, c_in=c_in, c_out=c_out, taps=k,
                     dilation=dilation, left_pad=left, phases=1, fp8=fp8, scale=scale)
    packed.macs_per_position = c_out * c_in * k
    return packed


def pack_conv_transpose1d(weight: torch.Tensor, bias: torch.Tensor | None, *, stride: int,
                          padding: int = 0, dilation: int = 1, fp8: bool = False,
                          scale: torch.Tensor | None = None) -> PackedConv:
    """ConvTranspose1d weight [C_in, C_out, k] in its polyphase form (output position i holds
    the transposed conv's samples s*i + p .. s*i + p + s - 1). ``padding = 0`` with a right trim
    of k - s is ``CausalTransConvNet`` (modded_dac.py:583-600); ``padding = (k-s)//2`` is the HiFT
    upsampler (hift.py:143-156)."""
    c_in, c_out, k = weight.shape
    if weight.dtype == torch.float8_e4m3fn:
        if scale is None:
            raise ValueError("an E4M3 weight needs its per-output-channel scale")
        fp8, weight = True, weight.float()  # E4M3 values are exact in float32
    w, left = polyphase_taps(weight, stride, padding, dilation)
    packed = _finish(w, bias, c_in=c_in, c_out=c_out, taps=w.shape[1], dilation=1,
                     left_pad=left, phases=stride, fp8=fp8, scale=scale)
    packed.macs_per_position = c_out * c_in * k  # every input sample meets all k taps
    return packed


def _conv_args(
    x: torch.Tensor,
    conv: PackedConv,
    out: torch.Tensor | None,
    *,
    length: int | None = None,
    x_length: int | None = None,
    in_activation: int = N.ACT_NONE,
    in_a: torch.Tensor | None = None,
    in_b: torch.Tensor | None = None,
    in_slope: float = 0.0,
    second: PackedConv | None = None,
    mid_activation: int = N.ACT_NONE,
    mid_a: torch.Tensor | None = None,
    mid_b: torch.Tensor | None = None,
    mid_slope: float = 0.0,
    activation: int = N.ACT_NONE,
    act_a: torch.Tensor | None = None,
    act_b: torch.Tensor | None = None,
    slope: float = 0.0,
    residual: torch.Tensor | None = None,
    sum_out: torch.Tensor | None = None,
    mix: tuple[torch.Tensor, torch.Tensor, float] | None = None,
    history: torch.Tensor | None = None,
    slot_index: torch.Tensor | None = None,
    slot_parity: torch.Tensor | None = None,
    history_cold: bool = False,
) -> N.ConvArgs:
    """Validate a ``fused_conv`` call and fill its ``omni_conv_args``: every pointer the kernels
    dereference is checked for device, dtype and extent here, before any launch."""
    N.require_device(x, out, sum_out, residual, conv.weight)
    dev = x.device
    if out is None and sum_out is None:
        raise ValueError("nothing to write: give out or sum_out")
    batch = x.shape[0]
    if length is None:
        length = x.shape[1]
    if x_length is None:
        x_length = x.shape[1] if history is None else length
    if x.dim() != 3 or x.dtype not in (torch.bfloat16, torch.float32) or x.stride(2) != 1:
        raise ValueError("x must be [B, L, C] bf16 or float32 with channel stride 1")
    if x.shape[2] != conv.c_in:
        raise ValueError(f"x has {x.shape[2]} channels, the conv takes {conv.c_in}")
    if x.shape[1] < x_length:
        raise ValueError(f"x holds {x.shape[1]} positions, fewer than x_length {x_length}")
    for t, name in ((conv.weight, "weight"), (conv.scale, "weight scale"), (conv.bias, "bias")):
        if t is not None and t.device != dev:
            raise ValueError(f"the conv's {name} is on {t.device}, x on {dev}")
    if second is not None and (second.c_in != conv.c_out or second.taps != 1
                               or conv.n_cols != conv.c_out or second.weight.dtype != conv.weight.dtype):
        raise ValueError("the fused second conv is a k = 1 conv over the first one's channels")
    if second is not None:
        N.require_device(second.weight)
        if second.weight.device != dev:
            raise ValueError(f"the second conv's weight is on {second.weight.device}, x on {dev}")
    n_cols = conv.n_cols if second is None else second.n_cols
    for t in (out, sum_out):
        if t is None:
            continue
        if t.device != dev:
            raise ValueError(f"an output is on {t.device}, x on {dev}")
        if t.dim() != 3 or t.shape[0] != batch or t.shape[2] != n_cols or t.stride(2) != 1:
            raise ValueError(f"outputs must be [B, {length}, {n_cols}] with channel stride 1")
        if t.shape[1] < length:
            raise ValueError("an output holds fewer positions than length")
        if t.data_ptr() == x.data_ptr():
            raise ValueError("an output may not alias x")
    aux = [t for t in (residual, sum_out) if t is not None]
    # the residual stream: float32, or float16 (a half-precision stream, added in float32)
    r_dtype = aux[0].dtype if aux else torch.float32
    if r_dtype not in (torch.float32, torch.float16):
        raise ValueError("residual / sum_out must be float32 or float16")
    if mix is not None:
        N.require_device(mix[0], mix[1])
        if not aux:
            r_dtype = mix[0].dtype
            if r_dtype not in (torch.float32, torch.float16):
                raise ValueError("mix streams must be float32 or float16")
        aux += [mix[0], mix[1]]
    for t in aux:
        if t.dtype != r_dtype or t.stride() != aux[0].stride():
            raise ValueError("residual / sum_out / mix must share one dtype and one stride")
        if (t.device != dev or t.dim() != 3 or t.shape[0] != batch or t.shape[1] < length
                or t.shape[2] != n_cols):
            raise ValueError(f"residual / sum_out / mix must be [B, {length}, {n_cols}] on {dev}")
    # per-channel coefficient arrays: the staging reads c_in entries, the epilogues one per
    # output channel (c_out; n = phase * c_out + co)
    c_out = conv.c_out if second is None else second.c_out
    for t, n, name in ((in_a, conv.c_in, "in_a"), (in_b, conv.c_in, "in_b"),
                       (mid_a, conv.c_out, "mid_a"), (mid_b, conv.c_out, "mid_b"),
                       (act_a, c_out, "act_a"), (act_b, c_out, "act_b")):
        N.require_vector(t, n, name, dev)
    N.require_slot_state(history, slot_index, slot_parity, rows=batch, samples=conv.left_pad,
                         channels=conv.c_in, device=dev, what="fused_conv")
    r_strides = aux[0].stride() if aux else (0, 0, 1)
    args = N.ConvArgs()
    args.x = x.data_ptr()
    args.x_dtype = N.omni_dtype(x.dtype)
    args.x_stride_b = x.stride(0)
    args.x_stride_t = x.stride(1)
    args.batch = batch
    args.length = length
    args.c_in = conv.c_in
    args.x_length = x_length
    args.in_activation = in_activation
    args.in_act_a = N.ptr(in_a)
    args.in_act_b = N.ptr(in_b)
    args.in_act_slope = in_slope
    args.weight = conv.weight.data_ptr()
    args.weight_dtype = N.omni_dtype(conv.weight.dtype)
    args.weight_scale = N.ptr(conv.scale)
    args.n_cols = conv.n_cols
    args.c_out = conv.c_out
    args.taps = conv.taps
    args.dilation = conv.dilation
    args.left_pad = conv.left_pad
    args.bias = N.ptr(conv.bias)
    if second is not None:
        args.weight2 = second.weight.data_ptr()
        args.weight2_scale = N.ptr(second.scale)
        args.bias2 = N.ptr(second.bias)
        args.mid_activation = mid_activation
        args.mid_act_a = N.ptr(mid_a)
        args.mid_act_b = N.ptr(mid_b)
        args.mid_act_slope = mid_slope
    if history is not None:
        args.hist_pool = history.data_ptr()
        args.slot_index = slot_index.data_ptr()
        args.slot_parity = slot_parity.data_ptr()
        args.hist_num_slots = history.shape[0]
        args.hist_slot_stride = history.stride(0)
        args.history_cold = int(history_cold)
    args.residual = N.ptr(residual)
    args.residual_stride_b = r_strides[0]
    args.residual_stride_t = r_strides[1]
    if mix is not None:
        args.mix_a = mix[0].data_ptr()
        args.mix_b = mix[1].data_ptr()
        args.mix_scale = float(mix[2])
    args.sum_out = N.ptr(sum_out)
    args.residual_dtype = N.omni_dtype(r_dtype)
    if out is not None:
        args.out = out.data_ptr()
        args.out_dtype = N.omni_dtype(out.dtype)
        args.out_stride_b = out.stride(0)
        args.out_stride_t = out.stride(1)
    else:
        args.out_dtype = N.DTYPE_BF16
    args.activation = activation
    args.act_a = N.ptr(act_a)
    args.act_b = N.ptr(act_b)
    args.act_slope = slope
    return args


def splitk_workspace_elements(x: torch.Tensor, conv: PackedConv, k_splits: int) -> int:
    """float32 elements of the workspace a ``k_splits`` launch of ``conv`` over x needs."""
    return k_splits * x.shape[0] * x.shape[1] * conv.n_cols


def splitk_conv(x: torch.Tensor, conv: PackedConv, out: torch.Tensor, *, k_splits: int,
                workspace: torch.Tensor, kernel: int = N.CONV_KERNEL_AUTO, config: int = 0,
                **kw) -> torch.Tensor:
    """``omni_conv1d_splitk``: the conv (k = 1, or k = 7 with its slot history) in ``k_splits``
    slices of the input channels, their float32 partials in ``workspace`` (at least
    ``splitk_workspace_elements`` contiguous float32 elements on x's GPU), summed in slice order,
    then the bias, the output activation (``activation`` / ``act_a`` / ``act_b`` as for
    ``fused_conv``) and the store. The summation order depends on the layer and k_splits only,
    so a row gives the same bits whatever batch or chunk of its stream it runs in."""
    need = splitk_workspace_elements(x, conv, k_splits)
    if (workspace is None or workspace.dtype != torch.float32 or not workspace.is_contiguous()
            or workspace.numel() < need or workspace.device != x.device):
        raise ValueError(f"split-K over {k_splits} slices needs a contiguous float32 workspace of "
                         f"{need} elements on {x.device}")
    args = _conv_args(x, conv, out, **kw)
    lib = N.load_library()
    N.check(lib.omni_conv1d_splitk(ctypes.byref(args), k_splits, workspace.data_ptr(),
                                   workspace.numel() * 4, kernel, config,
                                   N.stream_handle(x.device)), "omni_conv1d_splitk")
    return out


def gemm(x: torch.Tensor, conv: PackedConv, out: torch.Tensor, *, k_splits: int = 1,
         workspace: torch.Tensor | None = None, kernel: int = N.CONV_KERNEL_AUTO,
         config: int = 0) -> torch.Tensor:
    """out [B, L, n_cols] = x [B, L, C_in] (bf16) times a packed k = 1 conv (bias included), in
    ``k_splits`` slices of the input channels (``splitk_conv``) when k_splits > 1."""
    if k_splits == 1:
        return fused_conv(x, conv, out, kernel=kernel, config=config)
    if conv.taps != 1:
        raise ValueError("the split-K GEMM takes k = 1 convs")
    return splitk_conv(x, conv, out, k_splits=k_splits, workspace=workspace, kernel=kernel,
                       config=config)


def fused_conv(x: torch.Tensor, conv: PackedConv, out: torch.Tensor | None, *,
               kernel: int = N.CONV_KERNEL_AUTO, config: int = 0, **kw) -> torch.Tensor:
    """Launch ``omni_conv1d_fused`` on the current stream.

    x [B, >=x_length, C_in] bf16 or float32 (rows may sit in longer buffers; channel stride 1),
    activated per input channel by ``in_activation`` while it is staged; ``second`` is a k = 1
    conv (C_out -> C_out) fused behind this one with ``mid_activation`` between them;
    out [B, length, n_cols] bf16 or float32; residual / sum_out / mix (float32, or float16: a
    half-precision residual stream, widened exactly, added in float32 and rounded once when
    stored) tensors of one dtype with out's logical shape and one shared stride; history
    [slots, 2, left_pad, C_in] bf16 with int64
    slot_index [B] and slot_parity [slots]. ``kernel`` / ``config`` name a kernel family and the
    1-based entry of its tile list (``omni_conv1d_fused_with``) instead of the size-based choice.
    """
    args = _conv_args(x, conv, out, **kw)
    if _plan_log is not None:
        _plan_log.append(plan_args(args, kernel, config))
    lib = N.load_library()
    stream = N.stream_handle(x.device)
    if kernel == N.CONV_KERNEL_AUTO and config == 0:
        N.check(lib.omni_conv1d_fused(ctypes.byref(args), stream), "omni_conv1d_fused")
    else:
        N.check(lib.omni_conv1d_fused_with(ctypes.byref(args), kernel, config, stream),
                f"omni_conv1d_fused_with({N.CONV_KERNEL_NAMES.get(kernel, kernel)}, {config})")
    return out


_plan_log: list | None = None


def resblock_pair_supported(c1: PackedConv, c2: PackedConv) -> bool:
    """Whether ``resblock_pair`` takes this pair: 32 channels, bf16 weights, k = 3 / 7 / 11 with
    "same" padding, c1 dilation <= 5, c2 dilation 1."""
    k = c1.taps
    return (c1.c_in == c1.c_out == c1.n_cols == 32 and c2.c_in == c2.c_out == c2.n_cols == 32
            and c1.weight.dtype == c2.weight.dtype == torch.bfloat16 and k in (3, 7, 11)
            and c2.taps == k and c2.dilation == 1 and c1.dilation <= 5
            and c1.left_pad == (k - 1) * c1.dilation // 2 and c2.left_pad == (k - 1) // 2)


def resblock_pair(x: torch.Tensor, c1: PackedConv, c2: PackedConv, out: torch.Tensor | None, *,
                  slope1: float, **kw) -> torch.Tensor | None:
    """A ResBlock pair of a 32-channel stage in one launch (``omni_resblock_pair``): h =
    LeakyReLU(slope1)(c1(x)) stays on chip, then c2(h) with ``fused_conv``'s epilogue keywords
    (residual, sum_out, mix, activation, slope) into out. Equals ``fused_conv(x, c1, h,
    activation=LEAKY_RELU, slope=slope1)`` then ``fused_conv(h, c2, out, **kw)`` bit for bit."""
    if not resblock_pair_supported(c1, c2):
        raise ValueError("resblock_pair takes 32-channel bf16 pairs with k 3 / 7 / 11, same padding")
    if x.dtype != torch.bfloat16:
        raise ValueError("the pair's operand is bf16")
    # c2's arguments with x standing in for h (the same [B, L, 32] shape) for validation
    a2 = _conv_args(x, c2, out, **kw)
    a2.x = None
    a1 = N.ConvArgs()
    a1.x = x.data_ptr()
    a1.x_dtype = N.DTYPE_BF16
    a1.x_stride_b = x.stride(0)
    a1.x_stride_t = x.stride(1)
    a1.batch = x.shape[0]
    a1.length = x.shape[1]
    a1.c_in = c1.c_in
    a1.weight = c1.weight.data_ptr()
    a1.weight_dtype = N.DTYPE_BF16
    a1.n_cols = c1.n_cols
    a1.c_out = c1.c_out
    a1.taps = c1.taps
    a1.dilation = c1.dilation
    a1.left_pad = c1.left_pad
    a1.bias = N.ptr(c1.bias)
    a1.out_dtype = N.DTYPE_BF16
    a1.residual_dtype = N.DTYPE_F32
    a1.activation = N.ACT_LEAKY_RELU
    a1.act_slope = float(slope1)
    lib = N.load_library()
    N.check(lib.omni_resblock_pair(ctypes.byref(a1), ctypes.byref(a2), N.stream_handle(x.device)),
            "omni_resblock_pair")
    return out


@contextmanager
def recording_plans():
    """Collect the ``ConvPlan`` of every ``fused_conv`` call made inside the block (in call
    order), e.g. to see which tile configurations a workload's shapes take."""
    global _plan_log
    previous, _plan_log = _plan_log, []
    try:
        yield _plan_log
    finally:
        _plan_log = previous


@dataclass(frozen=True)
class ConvPlan:
    """The kernel family, 1-based tile entry, list length and workgroup count of a conv call."""

    kernel: int
    config: int
    configs: int
    workgroups: int

    @property
    def name(self) -> str:
        return f"{N.CONV_KERNEL_NAMES.get(self.kernel, 'none')}#{self.config}"


def plan_args(args: N.ConvArgs, kernel: int = N.CONV_KERNEL_AUTO, config: int = 0) -> ConvPlan:
    """What ``omni_conv1d_fused`` (or ``_with``) would launch for these arguments; nothing runs
    and no pointer is read, so this works without a GPU."""
    lib = N.load_library()
    k, c, n, w = ctypes.c_int(), ctypes.c_int(), ctypes.c_int(), ctypes.c_int64()
    N.check(lib.omni_conv1d_plan(ctypes.byref(args), kernel, config, ctypes.byref(k),
                                 ctypes.byref(c), ctypes.byref(n), ctypes.byref(w)),
            "omni_conv1d_plan")
    return ConvPlan(k.value, c.value, n.value, w.value)


def plan_shapes(*, batch: int, length: int, c_in: int, n_cols: int, c_out: int, taps: int,
                dilation: int = 1, left_pad: int | None = None, x_f32: bool = False,
                fp8: bool = False, in_activation: int = N.ACT_NONE, fused_unit: bool = False,
                history: bool = False, kernel: int = N.CONV_KERNEL_AUTO,
                config: int = 0) -> ConvPlan:
    """The plan of a conv call described by its shapes alone (placeholder aligned addresses)."""
    fake = 1 << 20
    args = N.ConvArgs()
    args.x = fake
    args.x_dtype = N.DTYPE_F32 if x_f32 else N.DTYPE_BF16
    args.x_stride_t = (c_in + 7) // 8 * 8
    args.x_stride_b = length * args.x_stride_t
    args.batch, args.length, args.c_in, args.x_length = batch, length, c_in, 0
    args.in_activation = in_activation
    if in_activation == N.ACT_SNAKE:
        args.in_act_a = args.in_act_b = fake
    args.weight = fake
    args.weight_dtype = N.DTYPE_FP8_E4M3 if fp8 else N.DTYPE_BF16
    args.weight_scale = fake if fp8 else None
    args.n_cols, args.c_out, args.taps, args.dilation = n_cols, c_out, taps, dilation
    args.left_pad = (taps - 1) * dilation if left_pad is None else left_pad
    if fused_unit:
        args.weight2 = fake
        args.weight2_scale = fake if fp8 else None
    if history:
        args.hist_pool = args.slot_index = args.slot_parity = fake
        args.hist_num_slots = batch
        args.hist_slot_stride = 2 * args.left_pad * c_in
    args.out = fake
    args.out_dtype = N.DTYPE_BF16
    args.out_stride_t = n_cols
    args.out_stride_b = length * n_cols
    return plan_args(args, kernel, config)


@dataclass
class FinalConv:
    """The decoder's conv to one channel when it runs inside the residual stack: weight
    [taps, C] float32 (tap-major), bias [1] or None, activation (ACT_TANH, ACT_CLAMP, ACT_NONE),
    out [B, 1, L] float32, and its streaming history pool [slots, 2, taps - 1, C] bf16 or None."""

    weight: torch.Tensor
    bias: torch.Tensor | None
    activation: int
    out: torch.Tensor
    history: torch.Tensor | None = None


@dataclass
class ResidualUnitWeights:
    """One residual unit of a decoder block: Snake(in) -> conv1 (k = 7, dilation) ->
    Snake(mid) -> conv2 (k = 1) -> + x, with the Snake coefficient pairs (a, b) as float32 [C]."""

    conv1: PackedConv
    conv2: PackedConv
    in_a: torch.Tensor
    in_b: torch.Tensor
    mid_a: torch.Tensor
    mid_b: torch.Tensor


def residual_stack(
    x: torch.Tensor,
    units: list[ResidualUnitWeights],
    out: torch.Tensor,
    out_a: torch.Tensor,
    out_b: torch.Tensor,
    *,
    x_out: torch.Tensor | None = None,
    histories: list[torch.Tensor | None] | None = None,
    slot_index: torch.Tensor | None = None,
    slot_parity: torch.Tensor | None = None,
    history_cold: bool = False,
    final: FinalConv | None = None,
    coef_table: torch.Tensor | None = None,
) -> torch.Tensor:
    """Launch ``omni_residual_stack``: every unit in turn over x [B, L, C] (float32, or a
    float16 residual stream, kept in float32 between the units), then out = Snake(out_a,
    out_b)(x_last) as bf16 [B, L, C] (and x_last into x_out, in x's dtype).
    histories[k] is unit k's conv1 history pool [slots, 2, 6 * dilation, C] bf16 (streaming).
    With ``final`` the decoder's conv to one channel runs over out inside the same launch and
    writes final.out [B, 1, L] float32 (out may then be None: the operand stays on chip); returns
    final.out, else out."""
    N.require_device(x, out, x_out)
    dev = x.device
    if not 1 <= len(units) <= N.MAX_RESIDUAL_UNITS:
        raise ValueError(f"1..{N.MAX_RESIDUAL_UNITS} residual units per launch")
    if x.dtype not in (torch.float32, torch.float16) or x.dim() != 3 or x.stride(2) != 1:
        raise ValueError("x must be float32 or float16 [B, L, C] with channel stride 1")
    batch, length, channels = x.shape
    if out is None and final is None:
        raise ValueError("the stack needs an output: out, or a final conv")
    for t, dt in ((out, torch.bfloat16), (x_out, x.dtype)):
        if t is None:
            continue
        if t.dtype != dt or t.dim() != 3 or tuple(t.shape) != (batch, length, channels) or t.stride(2) != 1:
            raise ValueError("out / x_out must be [B, L, C] (bf16 / x's dtype) with channel stride 1")
        if t.data_ptr() == x.data_ptr():
            raise ValueError("an output may not alias x")
    for t in (out, x_out):
        if t is not None and t.device != dev:
            raise ValueError(f"an output is on {t.device}, x on {dev}")
    N.require_vector(out_a, channels, "out_a", dev)
    N.require_vector(out_b, channels, "out_b", dev)
    if out_a is None or out_b is None:
        raise ValueError("the stack's output Snake needs out_a and out_b")
    if histories is not None and len(histories) != len(units):
        raise ValueError("one history pool (or None) per residual unit")
    for k, u in enumerate(units):
        for t, name in ((u.conv1.weight, "conv1 weight"), (u.conv2.weight, "conv2 weight"),
                        (u.conv1.scale, "conv1 scale"), (u.conv2.scale, "conv2 scale"),
                        (u.conv1.bias, "conv1 bias"), (u.conv2.bias, "conv2 bias")):
            if t is not None:
                N.require_device(t)
                if t.device != dev:
                    raise ValueError(f"unit {k}'s {name} is on {t.device}, x on {dev}")
        for t, name in ((u.in_a, "in_a"), (u.in_b, "in_b"), (u.mid_a, "mid_a"), (u.mid_b, "mid_b")):
            if t is None:
                raise ValueError(f"unit {k} needs its {name} Snake coefficients")
            N.require_vector(t, channels, f"unit {k} {name}", dev)
        if histories is not None:
            N.require_slot_state(histories[k], slot_index, slot_parity, rows=batch,
                                 samples=u.conv1.left_pad, channels=channels, device=dev,
                                 what=f"residual_stack unit {k}")
    if final is not None:
        N.require_device(final.weight, final.out)
        N.require_vector(final.bias, 1, "final.bias", dev)
        N.require_slot_state(final.history, slot_index, slot_parity, rows=batch,
                             samples=final.weight.shape[0] - 1, channels=channels, device=dev,
                             what="residual_stack final conv")
    wdtype = units[0].conv1.weight.dtype
    args = N.ResidualStackArgs()
    args.x = x.data_ptr()
    args.x_dtype = N.omni_dtype(x.dtype)
    args.x_stride_b, args.x_stride_t = x.stride(0), x.stride(1)
    args.batch, args.length, args.channels = batch, length, channels
    args.weight_dtype = N.omni_dtype(wdtype)
    args.num_units = len(units)
    for k, u in enumerate(units):
        c1, c2 = u.conv1, u.conv2
        if (c1.c_in != channels or c1.c_out != channels or c1.taps != 7 or c1.phases != 1
                or c1.left_pad != 6 * c1.dilation or c2.taps != 1 or c2.c_in != channels
                or c2.c_out != channels or c1.weight.dtype != wdtype or c2.weight.dtype != wdtype):
            raise ValueError("a residual unit is a causal k = 7 conv and a k = 1 conv over C channels")
        a = args.units[k]
        a.weight1 = c1.weight.data_ptr()
        a.weight1_scale = N.ptr(c1.scale)
        a.bias1 = N.ptr(c1.bias)
        a.dilation = c1.dilation
        a.in_act_a, a.in_act_b = u.in_a.data_ptr(), u.in_b.data_ptr()
        a.mid_act_a, a.mid_act_b = u.mid_a.data_ptr(), u.mid_b.data_ptr()
        a.weight2 = c2.weight.data_ptr()
        a.weight2_scale = N.ptr(c2.scale)
        a.bias2 = N.ptr(c2.bias)
        hist = histories[k] if histories is not None else None
        if hist is not None:
            if slot_index is None or slot_parity is None:
                raise ValueError("a history pool needs slot_index and slot_parity")
            a.hist_pool = hist.data_ptr()
            a.hist_slot_stride = hist.stride(0)
            args.hist_num_slots = hist.shape[0]
    if histories is not None and any(h is not None for h in histories):
        args.slot_index = slot_index.data_ptr()
        args.slot_parity = slot_parity.data_ptr()
        args.history_cold = int(history_cold)
    args.out_act_a, args.out_act_b = out_a.data_ptr(), out_b.data_ptr()
    if out is not None:
        args.out = out.data_ptr()
        args.out_stride_b, args.out_stride_t = out.stride(0), out.stride(1)
    if final is not None:
        f = final
        N.require_device(f.weight, f.out)
        taps = f.weight.shape[0]
        if (f.weight.dtype != torch.float32 or tuple(f.weight.shape) != (taps, channels)
                or not f.weight.is_contiguous()):
            raise ValueError("final.weight must be float32 [taps, C] contiguous")
        if (f.out.dtype != torch.float32 or tuple(f.out.shape) != (batch, 1, length)
                or f.out.stride(2) != 1):
            raise ValueError("final.out must be float32 [B, 1, L] with unit position stride")
        args.final_weight = f.weight.data_ptr()
        args.final_bias = N.ptr(f.bias)
        args.final_taps = taps
        args.final_activation = f.activation
        args.final_out = f.out.data_ptr()
        args.final_out_stride_b = f.out.stride(0)
        if f.history is not None:
            if slot_index is None or slot_parity is None:
                raise ValueError("a history pool needs slot_index and slot_parity")
            args.final_hist_pool = f.history.data_ptr()
            args.final_hist_slot_stride = f.history.stride(0)
            args.hist_num_slots = f.history.shape[0]
            args.slot_index = slot_index.data_ptr()
            args.slot_parity = slot_parity.data_ptr()
            args.history_cold = int(history_cold)
    if x_out is not None:
        args.x_out = x_out.data_ptr()
        args.x_out_stride_b, args.x_out_stride_t = x_out.stride(0), x_out.stride(1)
    if coef_table is not None:
        N.require_device(coef_table)
        if (coef_table.dtype != torch.float32 or coef_table.numel() != (8 * len(units) + 2) * channels
                or coef_table.device != dev or not coef_table.is_contiguous()):
            raise ValueError("coef_table must be stack_coefficients(...) of these units")
        args.coef_table = coef_table.data_ptr()
    lib = N.load_library()
    N.check(lib.omni_residual_stack(ctypes.byref(args), N.stream_handle(x.device)),
            "omni_residual_stack")
    return final.out if final is not None else out


def stack_coefficients(units: list[ResidualUnitWeights], out_a: torch.Tensor,
                       out_b: torch.Tensor) -> torch.Tensor:
    """The coefficient rows ``residual_stack`` launches over these units and output Snake read
    (``omni_residual_stack_coefficients``): computed once, passed as ``coef_table`` to every
    launch with the same weights."""
    channels = units[0].conv1.c_out
    N.require_device(out_a, out_b)
    args = N.ResidualStackArgs()
    args.channels = channels
    args.weight_dtype = N.omni_dtype(units[0].conv1.weight.dtype)
    args.num_units = len(units)
    for k, u in enumerate(units):
        a = args.units[k]
        a.weight1_scale = N.ptr(u.conv1.scale)
        a.bias1 = N.ptr(u.conv1.bias)
        a.in_act_a, a.in_act_b = u.in_a.data_ptr(), u.in_b.data_ptr()
        a.mid_act_a, a.mid_act_b = u.mid_a.data_ptr(), u.mid_b.data_ptr()
        a.weight2_scale = N.ptr(u.conv2.scale)
        a.bias2 = N.ptr(u.conv2.bias)
    args.out_act_a, args.out_act_b = out_a.data_ptr(), out_b.data_ptr()
    table = torch.empty((8 * len(units) + 2) * channels, dtype=torch.float32, device=out_a.device)
    lib = N.load_library()
    N.check(lib.omni_residual_stack_coefficients(ctypes.byref(args), table.data_ptr(),
                                                 table.numel(), N.stream_handle(out_a.device)),
            "omni_residual_stack_coefficients")
    return table
