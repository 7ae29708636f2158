"""The code2wav front's linear layers on ``omni_gemm``: out = epilogue(x @ W^T) with the
elementwise pass that follows each GEMM in the reference run on the float32 accumulators
(sglang_omni/models/qwen3_omni/components/code2wav.py:253-326: the qkv GEMM, the layer-scaled
addcmul after o_proj and down_proj, silu_and_mul after gate_up; incremental_codec.py:174-180:
GELU after pwconv1, residual + gamma * pwconv2). Every row's result is independent of the rows
batched with it."""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from .. import _native as N
from .code2wav_front import _check_rings, _num_slots

STORE, SILU_MUL, GELU, SCALED_RESIDUAL = (N.GEMM_STORE, N.GEMM_SILU_MUL, N.GEMM_GELU,
                                          N.GEMM_SCALED_RESIDUAL)


@dataclass
class LinearWeight:
    """A linear layer's weight [out, in] as bf16 rows for ``omni_gemm`` (``gated``: a merged
    gate / up weight [2 I, in], rows interleaved in blocks of 16 so that each gate block sits
    beside its up block), with an optional float32 bias in the same row order."""

    weight: torch.Tensor
    bias: torch.Tensor | None
    in_features: int
    out_features: int  # columns of the GEMM's output (I for a gated weight)
    gated: bool = False

    def to(self, device) -> "LinearWeight":
        return LinearWeight(self.weight.to(device), None if self.bias is None else self.bias.to(device),
                            self.in_features, self.out_features, self.gated)


def _interleave16(t: torch.Tensor) -> torch.Tensor:
    """[2 I, ...] (gate rows, then up rows) -> blocks of 16: gate 0-15, up 0-15, gate 16-31, ..."""
    inter = t.shape[0] // 2
    gate, up = t[:inter], t[inter:]
    blocks = torch.stack([gate.reshape(inter // 16, 16, *t.shape[1:]),
                          up.reshape(inter // 16, 16, *t.shape[1:])], dim=1)
    return blocks.reshape(t.shape)


def pack_linear(weight: torch.Tensor, bias: torch.Tensor | None = None, *,
                gated: bool = False) -> LinearWeight:
    """weight [out, in] (any float dtype) -> bf16 [out, in]; ``gated`` marks a merged [gate; up]
    weight whose GEMM applies silu(gate) * up."""
    if weight.dim() != 2:
        raise ValueError("a linear weight is [out_features, in_features]")
    n, k = weight.shape
    if k % 64 or n % 64:
        raise ValueError(f"omni_gemm takes in_features and out_features in multiples of 64, got "
                         f"[{n}, {k}]")
    w = weight.detach().to(torch.bfloat16)
    b = None if bias is None else bias.detach().float()
    if gated:
        if n % 32:
            raise ValueError("a gated weight holds 2 * I rows, I a multiple of 16")
        w = _interleave16(w)
        b = None if b is None else _interleave16(b)
    return LinearWeight(w.contiguous(), None if b is None else b.contiguous(), k,
                        n // 2 if gated else n, gated)


def linear(x: torch.Tensor, weight: LinearWeight, out: torch.Tensor, *,
           epilogue: int | None = None, scale: torch.Tensor | None = None,
           residual: torch.Tensor | None = None, config: int = 0) -> torch.Tensor:
    """out = epilogue(x [rows, in] bf16 @ W^T + bias) on the current stream.

    STORE (default; SILU_MUL for a gated weight): out bf16 [rows, out_features]. GELU: out bf16
    = GELU(acc + bias). SCALED_RESIDUAL: out (float32, or bf16) = residual (float32 [rows,
    out_features], may be out) + scale * (acc + bias). Rows of x, out and residual contiguous
    along the features; ``config`` forces one of ``omni_gemm``'s tiles (1 - 6), each giving the
    same bits."""
    N.require_device(x, weight.weight, weight.bias, out, scale, residual)
    if epilogue is None:
        epilogue = SILU_MUL if weight.gated else STORE
    if (epilogue == SILU_MUL) != weight.gated:
        raise ValueError("silu_mul takes a gated weight, and a gated weight only silu_mul")
    if x.dtype != torch.bfloat16 or x.dim() != 2 or x.stride(1) != 1:
        raise ValueError("x must be bf16 [rows, in_features] with contiguous rows")
    rows = x.shape[0]
    if x.shape[1] != weight.in_features:
        raise ValueError(f"x has {x.shape[1]} features, the weight takes {weight.in_features}")
    if out.dim() != 2 or out.shape != (rows, weight.out_features) or out.stride(1) != 1:
        raise ValueError(f"out must be [{rows}, {weight.out_features}] with contiguous rows")
    want = (torch.float32, torch.bfloat16) if epilogue == SCALED_RESIDUAL else (torch.bfloat16,)
    if out.dtype not in want:
        raise ValueError(f"out must be {' or '.join(str(d) for d in want)}")
    if epilogue == SCALED_RESIDUAL:
        if scale is None or residual is None:
            raise ValueError("the scaled residual takes scale and residual")
        if residual.dtype != torch.float32 or residual.shape != out.shape or residual.stride(1) != 1:
            raise ValueError("residual must be float32 like out, with contiguous rows")
        if scale.dtype != torch.float32 or scale.shape != (weight.out_features,):
            raise ValueError("scale must be float32 [out_features]")
    args = _gemm_args(x, weight, out, epilogue, scale, residual, config)
    lib = N.load_library()
    N.check(lib.omni_gemm(ctypes.byref(args), N.stream_handle(x.device)), "omni_gemm")
    return out


def _gemm_args(x, weight, out, epilogue, scale, residual, config):
    args = N.GemmArgs()
    args.a = x.data_ptr()
    args.a_stride = x.stride(0)
    args.w = weight.weight.data_ptr()
    args.rows = x.shape[0]
    args.k = weight.in_features
    args.n = weight.weight.shape[0]
    args.bias = N.ptr(weight.bias)
    args.epilogue = epilogue
    args.out_dtype = N.DTYPE_F32 if out.dtype == torch.float32 else N.DTYPE_BF16
    args.config = config
    args.scale = N.ptr(scale)
    args.residual = N.ptr(residual)
    args.residual_stride = 0 if residual is None else residual.stride(0)
    args.out = out.data_ptr()
    args.out_stride = out.stride(0)
    return args


def linear_rope_kv(x: torch.Tensor, weight: LinearWeight, qkv: torch.Tensor, batch: int,
                   heads: int, kv_heads: int, head_dim: int, inv_freq: torch.Tensor, *,
                   slot_index: torch.Tensor | None = None, positions: torch.Tensor | None = None,
                   cold: bool = True, key_ring: torch.Tensor | None = None,
                   value_ring: torch.Tensor | None = None, ring_frames: int = 0,
                   config: int = 0) -> torch.Tensor:
    """qkv = x @ W^T (+ bias) with the rotary embedding of its q and k heads and the new K / V
    rows into the rings in the GEMM's epilogue: the bits of ``linear(x, weight, qkv)`` followed
    by ``code2wav_front.rope_kv_write(qkv, batch, ...)``, in one launch (qkv_proj then
    apply_rope_inplace_with_kvcache, code2wav.py:267, :205-215). Returns qkv."""
    N.require_device(x, weight.weight, weight.bias, qkv, inv_freq, slot_index, positions,
                     key_ring, value_ring)
    if weight.gated:
        raise ValueError("the qkv weight is not gated")
    if qkv.dtype != torch.bfloat16:
        raise ValueError("qkv must be bf16")
    if x.dtype != torch.bfloat16 or x.dim() != 2 or x.stride(1) != 1:
        raise ValueError("x must be bf16 [rows, in_features] with contiguous rows")
    rows = x.shape[0]
    if x.shape[1] != weight.in_features:
        raise ValueError(f"x has {x.shape[1]} features, the weight takes {weight.in_features}")
    if qkv.dim() != 2 or qkv.shape != (rows, weight.out_features) or qkv.stride(1) != 1:
        raise ValueError(f"qkv must be [{rows}, {weight.out_features}] with contiguous rows")
    if batch < 1 or rows % batch:
        raise ValueError("x rows must be batch * frames")
    if slot_index is not None and (slot_index.dtype != torch.int64 or slot_index.numel() < batch):
        raise ValueError("slot_index must be int64 with one entry per batch row")
    _check_rings(key_ring, value_ring, kv_heads * head_dim)
    num_slots = _num_slots(positions, key_ring, ring_frames)
    args = _gemm_args(x, weight, qkv, STORE, None, None, config)
    lib = N.load_library()
    N.check(lib.omni_gemm_rope_kv(ctypes.byref(args), rows // batch, heads, kv_heads, head_dim,
                                  inv_freq.data_ptr(), N.ptr(slot_index), N.ptr(positions),
                                  int(cold), num_slots, N.ptr(key_ring), N.ptr(value_ring),
                                  ring_frames, N.stream_handle(x.device)),
            "omni_gemm_rope_kv")
    return qkv
