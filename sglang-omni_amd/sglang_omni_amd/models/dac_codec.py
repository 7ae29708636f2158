"""The DAC-style causal codec decoder on HIP kernels: ``from_indices`` and streaming slot decodes.

Drop-in for the vocoder stage's codec (the ``AudioCodec`` protocol of
sglang_omni/scheduling/audio_stream.py:15-20: ``sample_rate``, ``frame_length``, ``delay``,
``from_indices``) and for the slot-decode API of
sglang_omni/models/qwen3_omni/components/code2wav.py:417-460 (``decode_slots(codes, pool,
slot_index, first_decode=...)``) with a ``CodecStatePool``-shaped state pool
(sglang_omni/models/qwen3_omni/components/codec_state_pool.py:63-145).

The decoder follows ``Decoder`` / ``DecoderBlock`` / ``ResidualUnit`` / ``CausalConvNet`` /
``CausalTransConvNet`` of sglang_omni/models/fishaudio_s2_pro/fish_speech/models/dac/
modded_dac.py:541-835 fed by the RVQ gather-sum (rvq.py:374-388). Every op runs in a HIP kernel,
on channels-last activations. The residual stream x stays in HBM between launches as float16
(``residual_dtype``; float32 on request), every residual add in float32; every producer also
writes the next conv's operand u = Snake(x) as bf16 in its epilogue, so each conv reads a ready
bf16 operand:

    rvq_gather_sum                       codes -> z (bf16)
    conv k7 (512 -> C0)                  z -> u = Snake(block 0)(x) (bf16)
    per block:
      polyphase ConvTranspose (k = 2s)   u -> x, u = Snake(unit 0 act1)(x)
      per residual unit (d = 1, 3, 9):
        96 channels (192 with fp8 weights): one launch
                                         conv k7 dilation d; bias + Snake(act2) -> bf16 tile in
                                         LDS; conv k1; bias + x -> x (in place),
                                         u' = Snake(next)(x) (bf16)
        otherwise:         two launches  conv k7; bias + Snake(act2) -> h (bf16)
                                         conv k1 of h; bias + x -> x (in place), u' = Snake(next)(x)
    conv to one channel k7               u = Snake(final)(x); tanh -> float32 waveform

Streaming keeps each causal conv's left context (its last (k-1)*d activated input samples) per
slot in HBM; the conv kernels read it in place of zeros and write the new context themselves,
double-buffered by a per-slot parity that ``omni_advance_slots`` flips at the end of the step. A
transposed conv with k = 2s needs one input sample of context, which is exactly the reference's
overlap-add.
"""

from __future__ import annotations

import weakref
from dataclasses import dataclass, field
from typing import Any

import torch

from .. import _native as N
from ..kernels.conv import (
    FinalConv,
    PackedConv,
    ResidualUnitWeights,
    fused_conv,
    pack_conv1d,
    pack_conv_transpose1d,
    residual_stack,
    splitk_conv,
    stack_coefficients,
)
from ..kernels.rvq import rvq_gather_sum
from ..kernels.single_output_conv import single_output_conv
from ..quantization import reference_weights
from ..utils.timing import NO_TIMER
from .configs import DacDecoderConfig


@dataclass
class _Layer:
    name: str
    conv: PackedConv
    out_a: torch.Tensor | None = None  # Snake a (alpha) of the operand the epilogue writes
    out_b: torch.Tensor | None = None  # Snake b (1 / (alpha + 1e-9))


@dataclass
class _Unit:
    conv1: _Layer  # k = 7, dilation d; its output gets Snake(act2)
    conv2: PackedConv  # k = 1; its output (the new x) gets Snake(next)
    mid_a: torch.Tensor  # Snake(act2) between the two convs
    mid_b: torch.Tensor
    next_a: torch.Tensor  # Snake of the next conv's input
    next_b: torch.Tensor
    fused: bool  # both convs in one launch


@dataclass
class _Block:
    up: _Layer  # out_a / out_b: Snake(act1) of the first unit
    units: list[_Unit]
    stride: int
    c_out: int
    stack: list[ResidualUnitWeights] | None = None  # the units as one residual-stack launch
    stack_coef: torch.Tensor | None = None  # their coefficient rows (computed once)
    up_kernel: int = 0  # the transposed conv's kernel size


# channel counts the fused residual-unit kernel handles (one column tile holds every channel)
FUSED_UNIT_CHANNELS = (96, 192)
# ... and those where it is the faster form with bf16 weights: with its 16-wave tiles (four waves
# per SIMD) the fused register-staged launch beats the two LDS-DMA conv launches of a
# 192-channel unit (h stays in LDS instead of a bf16 round trip through HBM): DAC step 0.97x
FUSED_UNIT_CHANNELS_BF16 = (96, 192)
# channel counts the residual-stack kernel (every unit of a block in one launch) handles
STACK_CHANNELS = (96,)
# K slices of the input conv with bf16 weights (kept when its input channels divide into them)
IN_CONV_SPLITS = 4


def _snake_coefficients(alpha: torch.Tensor | dict[str, torch.Tensor],
                        device: torch.device) -> tuple[torch.Tensor, torch.Tensor]:
    """The epilogues' (a, b) of v + b * sin(a * v)^2: Snake1d's alpha gives (alpha, 1 / (alpha +
    1e-9)); a SnakeBeta's {"alpha", "beta"} (log scale, modeling_qwen3_omni_moe.py:3566-3581)
    gives (exp(alpha), 1 / (exp(beta) + 1e-9))."""
    if isinstance(alpha, dict):
        a = torch.exp(alpha["alpha"].detach().float().reshape(-1))
        inv_b = (torch.exp(alpha["beta"].detach().float().reshape(-1)) + 1e-9).reciprocal()
        return a.to(device).contiguous(), inv_b.to(device).contiguous()
    a = alpha.detach().float().reshape(-1)
    return a.to(device).contiguous(), (a + 1e-9).reciprocal().to(device).contiguous()


# the attribute that marks an index tensor whose ids were checked distinct on the host, holding
# the tensor's version counter at the check (an in-place write to the tensor voids the mark)
_DISTINCT_MARK = "_omni_distinct_slots_version"


def mark_distinct_slots(index: torch.Tensor) -> torch.Tensor:
    """Mark ``index`` as holding distinct slot ids, checked by the caller on its host list, so
    a decode step takes it without reading it back from the device."""
    setattr(index, _DISTINCT_MARK, index._version)
    return index


def _marked_distinct(index: torch.Tensor) -> bool:
    return getattr(index, _DISTINCT_MARK, None) == index._version


class CodecStatePool:
    """Per-slot decoder state resident in HBM: for every causal conv with left context, a
    [slots, 2, context, C_in] bf16 pool (two copies, selected by the slot's parity), then
    ``capture_slots`` scratch slots past the streams' slots (for graph capture), mirroring
    ``CodecStatePool`` (sglang_omni/models/qwen3_omni/components/codec_state_pool.py:63-145)."""

    def __init__(self, layout: list[tuple[str, int, int]], *, num_slots: int, capture_slots: int = 0,
                 device: torch.device):
        total = num_slots + capture_slots
        self.device = device
        self.num_slots = num_slots
        self.free_slots = list(reversed(range(num_slots)))
        self.scratch_slots = tuple(range(num_slots, total))
        self.histories = {
            name: torch.zeros(total, 2, length, channels, dtype=torch.bfloat16, device=device)
            for name, channels, length in layout
            if length
        }
        self.parity = torch.zeros(total, dtype=torch.int64, device=device)
        self.bytes_per_slot = sum(2 * 2 * length * channels for _, channels, length in layout)

    def available_size(self) -> int:
        return len(self.free_slots)

    def acquire(self) -> int | None:
        """A free slot, or None when every slot is taken."""
        if not self.free_slots:
            return None
        return self.free_slots.pop()

    def release(self, slot: int) -> None:
        self.free_slots.append(slot)

    def stage_index(self, slots: list[int]) -> torch.Tensor:
        """The slots' ids on the device, copied from pinned memory so the host never waits.
        The rows of one decode step must name distinct slots of this pool."""
        slots = [int(s) for s in slots]
        if len(set(slots)) != len(slots):
            raise ValueError(f"the rows of a decode step name one slot twice: {slots}")
        total = self.parity.shape[0]
        if any(s < 0 or s >= total for s in slots):
            raise ValueError(f"slot ids must lie in [0, {total}): {slots}")
        if self.device.type != "cuda":
            index = torch.tensor(slots, dtype=torch.long, device=self.device)
        else:
            index = torch.tensor(slots, dtype=torch.long, pin_memory=True).to(self.device,
                                                                               non_blocking=True)
        mark_distinct_slots(index)
        return index

    def zero_slots(self, slots: torch.Tensor) -> None:
        """Clear the slots' state (both copies) and parity."""
        for pool in self.histories.values():
            pool.index_fill_(0, slots, 0)
        self.parity.index_fill_(0, slots, 0)


@dataclass
class _Workspace:
    z: torch.Tensor | None
    x: torch.Tensor  # the residual stream, float16 or float32 (updated in place by each unit)
    u: list[torch.Tensor]  # the bf16 operand of the next conv, two buffers (read while written)
    h: torch.Tensor  # bf16 activation between the two convs of an unfused residual unit
    # blocks whose residual units the fused kernel has no tile for at this shape (short rows with a
    # wide halo): they run as two launches
    unfused_blocks: set[int] = field(default_factory=set)
    front: dict[str, torch.Tensor] = field(default_factory=dict)  # a front's own buffers
    partials: torch.Tensor | None = None  # x's storage as float32: the split-K partials
    # False once the split-K input conv was refused at this shape (many rows of a few frames:
    # no split tile holds their history rows); the input conv then runs unsplit
    in_conv_split: bool = True


class DacCodecDecoder:
    """RVQ dequant + causal DAC decoder, every op on gfx950 HIP kernels.

    ``weights`` is the float32 master weight tree of ``configs.make_dac_weights``;
    ``weight_format`` "bf16" rounds every conv weight to bf16, "fp8" stores E4M3 weights with a
    float32 scale per output channel. Activations between convs are bf16, the residual stream
    float16 between launches (``residual_dtype``, or float32), accumulation float32.
    """

    def __init__(self, weights: dict[str, Any], config: DacDecoderConfig, *,
                 device: torch.device | str = "cuda", weight_format: str = "bf16",
                 residual_stacks: bool = True, residual_dtype: torch.dtype = torch.float16):
        if residual_dtype not in (torch.float16, torch.float32):
            raise ValueError(f"the residual stream is float16 or float32, not {residual_dtype}")
        # the residual stream between launches: float16 by default (as the reference's GPU
        # decoder keeps it, channels_last_decoder.py:114-122 with decode_dtype float16; every
        # residual add and the stack's units still run in float32), or float32
        self.residual_dtype = residual_dtype
        self.config = config
        self.device = torch.device(device)
        self.weight_format = weight_format
        fp8 = weight_format == "fp8"
        ref = reference_weights(weights, weight_format)
        self.sample_rate = config.sample_rate
        self.frame_length = config.hop_length
        self.delay = 0
        dev = self.device
        # "right": a transposed conv (k = 2s) emits s samples per input (modded_dac.py:583-600);
        # "both": the whole decode and a stream's first decode also drop its first s samples
        # (Qwen3OmniMoeCausalTransConvNet, modeling_qwen3_omni_moe.py:3216-3228)
        self.trim_first = getattr(config, "transconv_trim", "right") == "both"
        self.final_activation = (N.ACT_CLAMP if getattr(config, "final_activation", "tanh") == "clamp"
                                 else N.ACT_TANH)
        # conv-stack positions per code frame at the input conv
        self.front_upsample = 1
        self.codebooks = (ref["codebooks"].to(torch.bfloat16).to(dev).contiguous()
                          if "codebooks" in ref else None)
        self.num_codebooks = None if self.codebooks is None else self.codebooks.shape[0]

        # fp8: a float weight is quantized per output channel here; an E4M3 weight (a
        # checkpoint's, see quantization.fp8_conv_weight) is packed with its own scale
        def conv1d(src: dict, rsrc: dict, dilation: int = 1) -> PackedConv:
            w = src["weight"] if fp8 else rsrc["weight"]
            return pack_conv1d(w, rsrc["bias"], dilation=dilation, fp8=fp8,
                               scale=src.get("weight_scale") if fp8 else None).to(dev)

        def convt(src: dict, rsrc: dict, stride: int) -> PackedConv:
            w = src["weight"] if fp8 else rsrc["weight"]
            return pack_conv_transpose1d(w, rsrc["bias"], stride=stride, fp8=fp8,
                                         scale=src.get("weight_scale") if fp8 else None).to(dev)

        blocks_w, blocks_r = weights["blocks"], ref["blocks"]
        a0, b0 = _snake_coefficients(blocks_r[0]["alpha"], dev)
        self.in_conv = _Layer("in_conv", conv1d(weights["in_conv"], ref["in_conv"]), a0, b0)
        self.blocks: list[_Block] = []
        for i, (bw, br) in enumerate(zip(blocks_w, blocks_r)):
            units_r = br["units"]
            a, b = _snake_coefficients(units_r[0]["alpha1"], dev)
            up = _Layer(f"blocks.{i}.up", convt(bw["up"], br["up"], br["stride"]), a, b)
            units = []
            for u, (uw, ur) in enumerate(zip(bw["units"], units_r)):
                a2, b2 = _snake_coefficients(ur["alpha2"], dev)
                if u + 1 < len(units_r):
                    nxt = units_r[u + 1]["alpha1"]
                elif i + 1 < len(blocks_r):
                    nxt = blocks_r[i + 1]["alpha"]
                else:
                    nxt = ref["final"]["alpha"]
                an, bn = _snake_coefficients(nxt, dev)
                c1 = _Layer(f"blocks.{i}.units.{u}.conv1",
                            conv1d(uw["conv1"], ur["conv1"], ur["dilation"]), a2, b2)
                c2 = conv1d(uw["conv2"], ur["conv2"])
                units.append(_Unit(c1, c2, a2, b2, an, bn,
                                   c1.conv.c_out in (FUSED_UNIT_CHANNELS if fp8
                                                     else FUSED_UNIT_CHANNELS_BF16)))
            blk = _Block(up, units, br["stride"], up.conv.c_out,
                         up_kernel=int(br["up"]["weight"].shape[-1]))
            if (residual_stacks and blk.c_out in STACK_CHANNELS
                    and len(units) <= N.MAX_RESIDUAL_UNITS
                    and all(u.conv1.conv.taps == 7 and u.conv1.conv.dilation <= 10 for u in units)):
                ins = [(up.out_a, up.out_b)] + [(u.next_a, u.next_b) for u in units[:-1]]
                blk.stack = [ResidualUnitWeights(u.conv1.conv, u.conv2, a, b, u.mid_a, u.mid_b)
                             for u, (a, b) in zip(units, ins)]
                if self.device.type == "cuda":
                    blk.stack_coef = stack_coefficients(blk.stack, units[-1].next_a,
                                                        units[-1].next_b)
            self.blocks.append(blk)
        fw = ref["final"]["conv"]["weight"]  # [1, C, k]
        self.final_weight = fw[0].t().contiguous().float().to(dev)  # [k, C]
        self.final_bias = ref["final"]["conv"]["bias"].float().to(dev).contiguous()
        self.final_taps = fw.shape[-1]
        self.final_channels = fw.shape[1]
        # the final conv runs inside the last block's residual-stack launch (its operand never
        # leaves the chip) when that block has a stack over the final conv's channels
        self.final_in_stack = (bool(self.blocks) and self.blocks[-1].stack is not None
                               and self.blocks[-1].c_out == self.final_channels
                               and self.final_taps <= 8)
        # the input conv in K slices (omni_conv1d_splitk) with bf16 weights: at a streaming
        # step's few positions (64 streams x 12 frames) its unsplit tiles fill a quarter of the
        # GPU; the slice count is the layer's, never the batch's, so every decode of a stream
        # sums alike (streamed == whole, bit for bit) wherever a split tile holds the step; a
        # step of many rows of a few frames each, which none holds, runs the conv unsplit (the
        # same values to float32 summation order)
        ic_conv = self.in_conv.conv
        self.in_conv_splits = (IN_CONV_SPLITS if ic_conv.scale is None and ic_conv.taps in (1, 7)
                               and ic_conv.c_in % (32 * IN_CONV_SPLITS) == 0 else 1)
        self._workspaces: dict[tuple[int, int], _Workspace] = {}
        self._checked_index: tuple[weakref.ref, int] | None = None
        # a utils.timing.LaunchTimer installed here records every launch with its work
        self.timer = NO_TIMER

    # ---------------------------------------------------------------- state layout / pool

    def state_layout(self) -> list[tuple[str, int, int]]:
        """(name, channels, context samples) of every causal conv's per-slot left context, in
        decode order (k = 1 convs have none)."""
        layout = [("in_conv", self.in_conv.conv.c_in, self.in_conv.conv.left_pad)]
        for blk in self.blocks:
            layout.append((blk.up.name, blk.up.conv.c_in, blk.up.conv.left_pad))
            for unit in blk.units:
                layout.append((unit.conv1.name, unit.conv1.conv.c_in, unit.conv1.conv.left_pad))
        layout.append(("final", self.final_channels, self.final_taps - 1))
        return layout

    def new_state_pool(self, num_slots: int, capture_slots: int = 0) -> CodecStatePool:
        return CodecStatePool(self.state_layout(), num_slots=num_slots,
                              capture_slots=capture_slots, device=self.device)

    # ---------------------------------------------------------------- decode

    def _workspace(self, batch: int, frames: int) -> _Workspace:
        key = (batch, frames)
        ws = self._workspaces.get(key)
        if ws is None:
            dev = self.device
            length = frames * self.front_upsample
            largest = length * self.in_conv.conv.n_cols
            # x also holds the input conv's float32 split-K partials
            partials = largest * self.in_conv_splits if self.in_conv_splits > 1 else 0
            x_elems = 0
            for blk in self.blocks:
                length *= blk.stride
                largest = max(largest, length * blk.c_out)
                x_elems = max(x_elems, length * blk.c_out)
            size = self.residual_dtype.itemsize
            x_elems = max(x_elems, -(-partials * 4 // size))
            x_elems += x_elems % 2  # whole float32 words
            x = torch.empty(batch * x_elems, dtype=self.residual_dtype, device=dev)
            ws = _Workspace(
                z=None if self.codebooks is None else
                torch.empty(batch, frames, self.codebooks.shape[2], dtype=torch.bfloat16,
                            device=dev),
                x=x,
                u=[torch.empty(batch * largest, dtype=torch.bfloat16, device=dev) for _ in range(2)],
                h=torch.empty(batch * largest, dtype=torch.bfloat16, device=dev),
                partials=x.view(torch.float32),
            )
            self._workspaces[key] = ws
        return ws

    @staticmethod
    def _view(flat: torch.Tensor, batch: int, length: int, channels: int) -> torch.Tensor:
        return flat[: batch * length * channels].view(batch, length, channels)

    def _decode(self, codes: torch.Tensor, state: dict | None, *,
                latents: bool = False, window: int | None = None) -> torch.Tensor:
        if codes.dim() != 3:
            raise ValueError(f"codes must be [B, Q, T], got {tuple(codes.shape)}")
        batch, _, frames = codes.shape
        if batch == 0 or frames == 0:
            raise ValueError("codes must hold at least one row and one frame")
        if codes.device != self.device:
            raise ValueError(f"codes are on {codes.device}, the decoder on {self.device}")
        ws = self._workspace(batch, frames)

        def hist(name: str) -> dict:
            if state is None:
                return {}
            return {
                "history": state["pool"].histories.get(name),
                "slot_index": state["slot_index"],
                "slot_parity": state["pool"].parity,
                "history_cold": state["cold"],
            }

        timer = self.timer
        snake = N.ACT_SNAKE
        if latents:
            # layout / dtype plumbing of the caller's [B, D, T] latents: the input conv's
            # channels-last bf16 operand
            z, length = codes.transpose(1, 2).to(torch.bfloat16).contiguous(), frames
        else:
            z, length = self._front(codes, ws, state)
        if window is not None and window * self.front_upsample < length:
            # the conv stack over the last ``window`` frames only (a tail decode): their samples
            # and the state the stack leaves do not depend on what precedes the window
            keep = window * self.front_upsample
            z, length = z[:, length - keep:].contiguous(), keep
        # the whole decode and a stream's first decode drop each transposed conv's first s
        # samples when the decoder trims both sides
        trim = self.trim_first and (state is None or state["cold"])
        cur = 0
        u = self._view(ws.u[cur], batch, length, self.in_conv.conv.n_cols)
        ic = self.in_conv
        with timer.launch("conv", 2.0 * batch * length * ic.conv.macs_per_position, ic.name):
            split = self.in_conv_splits > 1 and ws.in_conv_split
            if split:
                # the partials go to the residual-stream buffer, unused until the first up conv
                try:
                    splitk_conv(z, ic.conv, u, k_splits=self.in_conv_splits, workspace=ws.partials,
                                activation=snake, act_a=ic.out_a, act_b=ic.out_b,
                                **hist(ic.name))
                except N.OmniCodecError as err:
                    # refused before any launch: nothing was written, so the unsplit conv
                    # below runs on the same inputs and history
                    if err.status != N.UNSUPPORTED:
                        raise
                    ws.in_conv_split = split = False
            if not split:
                fused_conv(z, ic.conv, u, activation=snake, act_a=ic.out_a, act_b=ic.out_b,
                           **hist(ic.name))
        for bi, blk in enumerate(self.blocks):
            up = blk.up
            out_len = length * blk.stride
            c = blk.c_out
            # the polyphase output [B, L, s*C] is the transposed conv's [B, L*s, C]
            x = self._view(ws.x, batch, out_len, c)
            u_next = self._view(ws.u[1 - cur], batch, out_len, c)
            # with a residual stack the up conv writes only x: the stack takes its own operand
            with timer.launch("conv", 2.0 * batch * length * up.conv.macs_per_position, up.name):
                fused_conv(u, up.conv,
                           None if blk.stack else u_next.view(batch, length, up.conv.n_cols),
                           sum_out=x.view(batch, length, up.conv.n_cols), activation=snake,
                           act_a=up.out_a, act_b=up.out_b, **hist(up.name))
            if trim:
                # the first input sample's s outputs leave the stream: every later op reads the
                # views that start after them
                x = x[:, blk.stride:]
                u_next = u_next[:, blk.stride:]
                out_len -= blk.stride
            cur = 1 - cur
            u = u_next
            length = out_len
            if blk.stack:
                flops = 2.0 * batch * length * sum(
                    u.conv1.macs_per_position + u.conv2.macs_per_position for u in blk.stack)
                u_next = self._view(ws.u[1 - cur], batch, length, c)
                h = {}
                if state is not None:
                    h = {"histories": [state["pool"].histories.get(un.conv1.name)
                                       for un in blk.units],
                         "slot_index": state["slot_index"],
                         "slot_parity": state["pool"].parity,
                         "history_cold": state["cold"]}
                last = blk.units[-1]
                if bi + 1 == len(self.blocks) and self.final_in_stack:
                    # the last block: the final conv runs inside the stack launch
                    final = FinalConv(self.final_weight, self.final_bias, self.final_activation,
                                      torch.empty(batch, 1, length, dtype=torch.float32,
                                                  device=self.device),
                                      hist("final").get("history"))
                    flops += 2.0 * batch * length * self.final_taps * self.final_channels
                    with timer.launch(f"stack{c}", flops, f"blocks.{bi}.units+final"):
                        wave = residual_stack(x, blk.stack, None, last.next_a, last.next_b,
                                              final=final, coef_table=blk.stack_coef, **h)
                    return self._finish_step(wave, state, batch)
                with timer.launch(f"stack{c}", flops, f"blocks.{bi}.units"):
                    residual_stack(x, blk.stack, u_next, last.next_a, last.next_b,
                                   coef_table=blk.stack_coef, **h)
                cur = 1 - cur
                u = u_next
                continue
            for unit in blk.units:
                c1 = unit.conv1
                # the block's last unit: only its Snake output is read again (by the next
                # block's up conv), so the residual stream is not written back
                x_out = None if unit is blk.units[-1] else x
                flops = 2.0 * batch * length * (c1.conv.macs_per_position +
                                                unit.conv2.macs_per_position)
                u_next = self._view(ws.u[1 - cur], batch, length, c)
                fused = False
                if unit.fused and bi not in ws.unfused_blocks:
                    try:
                        with timer.launch(f"unit{c}", flops, c1.name):
                            fused_conv(u, c1.conv, u_next, second=unit.conv2,
                                       mid_activation=snake, mid_a=unit.mid_a, mid_b=unit.mid_b,
                                       residual=x, sum_out=x_out, activation=snake,
                                       act_a=unit.next_a, act_b=unit.next_b, **hist(c1.name))
                        fused = True
                    except N.OmniCodecError as err:
                        if err.status != N.UNSUPPORTED:
                            raise
                        ws.unfused_blocks.add(bi)
                if not fused:
                    h = self._view(ws.h, batch, length, c)
                    with timer.launch("conv", 2.0 * batch * length * c1.conv.macs_per_position,
                                      c1.name):
                        fused_conv(u, c1.conv, h, activation=snake, act_a=unit.mid_a,
                                   act_b=unit.mid_b, **hist(c1.name))
                    with timer.launch("conv", 2.0 * batch * length * unit.conv2.macs_per_position,
                                      c1.name.replace("conv1", "conv2")):
                        fused_conv(h, unit.conv2, u_next, residual=x, sum_out=x_out,
                                   activation=snake, act_a=unit.next_a, act_b=unit.next_b)
                cur = 1 - cur
                u = u_next
        wave = torch.empty(batch, 1, length, dtype=torch.float32, device=self.device)
        with timer.launch("final", 2.0 * batch * length * self.final_taps * self.final_channels):
            single_output_conv(u, self.final_weight, self.final_bias, wave,
                               activation=self.final_activation, left_pad=self.final_taps - 1,
                               **hist("final"))
        return self._finish_step(wave, state, batch)

    def _front(self, codes: torch.Tensor, ws: _Workspace,
               state: dict | None) -> tuple[torch.Tensor, int]:
        """The input conv's operand [B, L, C] bf16 and L: the RVQ gather-sum of the codes."""
        batch, _, frames = codes.shape
        if self.codebooks is None:
            raise ValueError("this decoder has no codebooks (its quantizer does more than a "
                             "gather-sum): decode its latents with decode(z)")
        if ws.z is None:
            ws.z = torch.empty(batch, frames, self.codebooks.shape[2], dtype=torch.bfloat16,
                               device=self.device)
        k_books, _, dim = self.codebooks.shape
        rvq_bytes = batch * frames * (k_books * dim * 2 + dim * 2 + k_books * codes.element_size())
        with self.timer.launch("rvq", rvq_bytes):
            rvq_gather_sum(codes, self.codebooks, out=ws.z, clamp=True)
        return ws.z, frames

    def _finish_step(self, wave: torch.Tensor, state: dict | None, batch: int) -> torch.Tensor:
        """End of a decode step: flip the slot parity of the step's rows (streaming)."""
        if state is not None:
            lib = N.load_library()
            parity = state["pool"].parity
            N.check(lib.omni_advance_slots(parity.data_ptr(), parity.shape[0],
                                           state["slot_index"].data_ptr(), batch,
                                           N.stream_handle(self.device)), "omni_advance_slots")
        return wave

    # the largest activation buffer of one call stays below this many bytes (the kernels address
    # each buffer with 32-bit byte offsets)
    MAX_BUFFER_BYTES = 1 << 30

    def frames_per_call(self, batch: int) -> int:
        """Frames one decode call takes for ``batch`` rows: longer inputs are decoded in chunks of
        this many frames through per-row slot state, which gives the same bits."""
        per_frame, samples = 0, self.front_upsample
        for blk in self.blocks:
            samples *= blk.stride
            per_frame = max(per_frame, samples * blk.c_out * 4)
        return max(1, self.MAX_BUFFER_BYTES // (max(batch, 1) * per_frame))

    @torch.no_grad()
    def from_indices(self, indices: torch.Tensor) -> torch.Tensor:
        """[B, Q, T] codes -> [B, 1, T * frame_length] float32 waveform (``DAC.from_indices``,
        modded_dac.py:990-992). Codes above the codebook size read its last entry."""
        if indices.dim() != 3:
            raise ValueError(f"codes must be [B, Q, T], got {tuple(indices.shape)}")
        batch, _, frames = indices.shape
        step = self.frames_per_call(batch)
        if frames <= step:
            return self._decode(indices, None)
        pool = self.new_state_pool(num_slots=batch)
        rows = torch.arange(batch, device=self.device)
        parts = [self._decode(indices[..., s:s + step],
                              {"pool": pool, "slot_index": rows, "cold": s == 0})
                 for s in range(0, frames, step)]
        return torch.cat(parts, dim=-1)

    __call__ = from_indices

    @torch.no_grad()
    def decode(self, z: torch.Tensor) -> torch.Tensor:
        """[B, D, T] latents -> [B, 1, T * frame_length] float32 waveform: the decoder without
        the quantizer (``DAC.decode``, modded_dac.py:1004-1020). Long inputs decode in chunks
        through slot state, which gives the same bits."""
        if z.dim() != 3 or z.shape[1] != self.in_conv.conv.c_in:
            raise ValueError(f"latents must be [B, {self.in_conv.conv.c_in}, T], got "
                             f"{tuple(z.shape)}")
        if not z.is_floating_point():
            raise ValueError(f"latents must be floating point, got {z.dtype}")
        batch, _, frames = z.shape
        step = self.frames_per_call(batch)
        if frames <= step:
            return self._decode(z, None, latents=True)
        pool = self.new_state_pool(num_slots=batch)
        rows = torch.arange(batch, device=self.device)
        parts = [self._decode(z[..., s:s + step], {"pool": pool, "slot_index": rows,
                                                   "cold": s == 0}, latents=True)
                 for s in range(0, frames, step)]
        return torch.cat(parts, dim=-1)

    def _check_distinct_slots(self, slot_index: torch.Tensor) -> None:
        """Rows naming one slot twice would race on its history and parity: refuse them. An
        index from ``CodecStatePool.stage_index`` (or marked by ``mark_distinct_slots``) was
        checked on its host list and is taken as it is, so a serving step never waits for the
        GPU; any other index is read back once per tensor (and again after an in-place change
        to it). Under graph capture the check is the caller's (the graph runner checks its host
        lists)."""
        if _marked_distinct(slot_index) or torch.cuda.is_current_stream_capturing():
            return
        ref = self._checked_index
        if ref is not None and ref[0]() is slot_index and ref[1] == slot_index._version:
            return
        ids = slot_index.tolist()
        if len(set(ids)) != len(ids):
            raise ValueError(f"the rows of a decode step name one slot twice: {ids}")
        self._checked_index = (weakref.ref(slot_index), slot_index._version)

    @torch.no_grad()
    def decode_slots(self, codes: torch.Tensor, pool: CodecStatePool, slot_index: torch.Tensor,
                     *, first_decode: bool) -> torch.Tensor:
        """The (B, 1, T * frame_length) waveform of the (B, Q, T) codes after the frames the rows'
        slots hold, their state advanced in place; decoding a stream in any split of chunks gives
        the waveform ``from_indices`` gives on all of it. A first decode starts every row's
        stream and reads no slot. Rows must name distinct slots. Capturable in a graph with a
        static ``slot_index``."""
        if slot_index.dtype != torch.int64 or slot_index.shape != (codes.shape[0],):
            raise ValueError("slot_index must be int64 [B]")
        if slot_index.device != self.device or pool.device != self.device:
            raise ValueError(f"slot_index ({slot_index.device}) and the pool ({pool.device}) must "
                             f"be on the decoder's device {self.device}")
        if not slot_index.is_contiguous():
            raise ValueError("slot_index must be contiguous")
        self._check_distinct_slots(slot_index)
        return self._decode(codes, {"pool": pool, "slot_index": slot_index, "cold": first_decode})
