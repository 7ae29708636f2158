"""The Qwen3-Omni code2wav front's HIP kernels: the ops around the pre-transformer's and the
ConvNeXt upsamplers' GEMMs (sglang_omni/models/qwen3_omni/components/code2wav.py:107-324 runs
them as rmsnorm / rope / attention / silu_and_mul / addcmul kernels; incremental_codec.py:137-175
the ConvNeXt blocks). Every wrapper launches on the current stream and validates before launch.
"""

from __future__ import annotations

import torch

from .. import _native as N


def _bf16_rows(t: torch.Tensor, name: str) -> None:
    if t.dtype != torch.bfloat16 or t.dim() != 2 or t.stride(1) != 1:
        raise ValueError(f"{name} must be bf16 [rows, width] with contiguous rows")


def _num_slots(positions: torch.Tensor | None, key_ring: torch.Tensor | None,
               ring_frames: int) -> int:
    """The slot count the positions and the rings agree on (0 without either)."""
    counts = set()
    if positions is not None:
        counts.add(positions.shape[0])
    if key_ring is not None:
        if ring_frames < 1 or key_ring.shape[0] % ring_frames:
            raise ValueError("a ring holds ring_frames rows per slot")
        counts.add(key_ring.shape[0] // ring_frames)
    if len(counts) > 1:
        raise ValueError(f"positions and rings disagree on the slot count: {sorted(counts)}")
    return counts.pop() if counts else 0


def _check_rings(key_ring: torch.Tensor | None, value_ring: torch.Tensor | None,
                 kv_width: int) -> None:
    """The K / V rings: both or neither, contiguous bf16 [slots * ring_frames, kv_width]."""
    if (key_ring is None) != (value_ring is None):
        raise ValueError("key_ring and value_ring come together")
    for ring in (key_ring, value_ring):
        if ring is not None and (ring.dtype != torch.bfloat16 or ring.dim() != 2
                                 or not ring.is_contiguous() or ring.shape[1] != kv_width
                                 or ring.shape != key_ring.shape):
            raise ValueError(f"the rings must be contiguous bf16 [slots * ring_frames, {kv_width}]")


def rms_norm_residual(h: torch.Tensor, weight: torch.Tensor, eps: float, normed: torch.Tensor, *,
                      delta: torch.Tensor | None = None,
                      scale: torch.Tensor | None = None) -> torch.Tensor:
    """h [rows, C] float32 (contiguous) += scale * delta (bf16 [rows, C]) when delta is given;
    normed (bf16 [rows, C]) = RMSNorm(h) * weight. Returns normed."""
    N.require_device(h, weight, normed, delta, scale)
    if h.dtype != torch.float32 or h.dim() != 2 or not h.is_contiguous():
        raise ValueError("h must be contiguous float32 [rows, C]")
    rows, channels = h.shape
    _bf16_rows(normed, "normed")
    if normed.shape != h.shape:
        raise ValueError("normed must match h")
    if delta is not None:
        _bf16_rows(delta, "delta")
        if delta.shape != h.shape or scale is None:
            raise ValueError("delta must match h and come with a scale")
    lib = N.load_library()
    N.check(lib.omni_rms_norm_residual(h.data_ptr(), rows, channels, N.ptr(delta),
                                       0 if delta is None else delta.stride(0), N.ptr(scale),
                                       weight.data_ptr(), float(eps), normed.data_ptr(),
                                       normed.stride(0), N.stream_handle(h.device)),
            "omni_rms_norm_residual")
    return normed


def rope_kv_write(qkv: torch.Tensor, batch: int, heads: int, kv_heads: int, head_dim: int,
                  inv_freq: torch.Tensor, *, slot_index: torch.Tensor | None = None,
                  positions: torch.Tensor | None = None, cold: bool = True,
                  key_ring: torch.Tensor | None = None, value_ring: torch.Tensor | None = None,
                  ring_frames: int = 0) -> None:
    """Rotary embedding of q and k in qkv [batch * frames, >= (heads + 2 kv_heads) * head_dim]
    (bf16) in place, at each row's stream positions, and the new K / V into the rings."""
    N.require_device(qkv, inv_freq, slot_index, positions, key_ring, value_ring)
    _bf16_rows(qkv, "qkv")
    if qkv.shape[0] % max(batch, 1):
        raise ValueError("qkv rows must be batch * frames")
    frames = qkv.shape[0] // max(batch, 1)
    _check_rings(key_ring, value_ring, kv_heads * head_dim)
    num_slots = _num_slots(positions, key_ring, ring_frames)
    lib = N.load_library()
    N.check(lib.omni_rope_kv_write(qkv.data_ptr(), batch, frames, qkv.stride(0), heads, kv_heads,
                                   head_dim, inv_freq.data_ptr(), N.ptr(slot_index),
                                   N.ptr(positions), int(cold), num_slots, N.ptr(key_ring),
                                   N.ptr(value_ring), ring_frames, N.stream_handle(qkv.device)),
            "omni_rope_kv_write")


def window_attention(qkv: torch.Tensor, batch: int, heads: int, kv_heads: int, head_dim: int,
                     window: int, scale: float, out: torch.Tensor, *,
                     slot_index: torch.Tensor | None = None, positions: torch.Tensor | None = None,
                     cold: bool = True, key_ring: torch.Tensor | None = None,
                     value_ring: torch.Tensor | None = None, ring_frames: int = 0) -> torch.Tensor:
    """Sliding-window causal attention of the (rotated) queries in qkv over the rings' window or,
    for a first decode without rings, over qkv's own keys; out [batch * frames, heads * head_dim]
    bf16. Returns out."""
    N.require_device(qkv, out, slot_index, positions, key_ring, value_ring)
    _bf16_rows(qkv, "qkv")
    _bf16_rows(out, "out")
    frames = qkv.shape[0] // max(batch, 1)
    if out.shape[0] != qkv.shape[0]:
        raise ValueError("out must have one row per qkv row")
    num_slots = _num_slots(positions, key_ring, ring_frames)
    lib = N.load_library()
    N.check(lib.omni_window_attention(qkv.data_ptr(), batch, frames, qkv.stride(0), heads,
                                      kv_heads, head_dim, window, float(scale), N.ptr(key_ring),
                                      N.ptr(value_ring), ring_frames, N.ptr(slot_index),
                                      N.ptr(positions), int(cold), num_slots, out.data_ptr(),
                                      out.stride(0), N.stream_handle(qkv.device)),
            "omni_window_attention")
    return out


def silu_mul(gate_up: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
    """out [rows, I] = silu(gate_up[:, :I]) * gate_up[:, I:], bf16."""
    N.require_device(gate_up, out)
    _bf16_rows(gate_up, "gate_up")
    _bf16_rows(out, "out")
    rows, inter = out.shape
    if gate_up.shape != (rows, 2 * inter):
        raise ValueError("gate_up must be [rows, 2 * I]")
    lib = N.load_library()
    N.check(lib.omni_silu_mul(gate_up.data_ptr(), rows, inter, gate_up.stride(0), out.data_ptr(),
                              out.stride(0), N.stream_handle(out.device)), "omni_silu_mul")
    return out


def dwconv_layernorm(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor,
                     ln_weight: torch.Tensor, ln_bias: torch.Tensor, eps: float,
                     out: torch.Tensor, *, history: torch.Tensor | None = None,
                     slot_index: torch.Tensor | None = None,
                     slot_parity: torch.Tensor | None = None,
                     history_cold: bool = False) -> torch.Tensor:
    """ConvNeXt's depthwise causal conv (weight [7, C] float32) of x [B, L, C] float32 (rows of C
    contiguous), + bias, then LayerNorm into out [B, L, C] bf16; history [slots, 2, 6, C] float32
    streams the conv's left context (copy slot_parity & 1 read, the other written)."""
    N.require_device(x, weight, out, history, slot_index, slot_parity)
    if x.dtype != torch.float32 or x.dim() != 3 or x.stride(2) != 1 or x.stride(1) != x.shape[2]:
        raise ValueError("x must be float32 [B, L, C] with contiguous rows")
    batch, length, channels = x.shape
    if weight.shape != (7, channels) or weight.dtype != torch.float32:
        raise ValueError("weight must be float32 [7, C]")
    if out.dtype != torch.bfloat16 or out.shape != x.shape or out.stride(1) != channels \
            or out.stride(2) != 1:
        raise ValueError("out must be bf16 [B, L, C] with contiguous rows")
    if history is not None and (history.dtype != torch.float32 or history.shape[1:] != (2, 6, channels)):
        raise ValueError("history must be float32 [slots, 2, 6, C]")
    lib = N.load_library()
    N.check(lib.omni_dwconv_layernorm(
        x.data_ptr(), batch, length, channels, x.stride(0), weight.data_ptr(), bias.data_ptr(),
        ln_weight.data_ptr(), ln_bias.data_ptr(), float(eps), N.ptr(history),
        0 if history is None else history.stride(0), N.ptr(slot_index), N.ptr(slot_parity),
        0 if history is None else history.shape[0], int(history_cold), out.data_ptr(),
        out.stride(0), N.stream_handle(x.device)), "omni_dwconv_layernorm")
    return out


def bias_gelu(y: torch.Tensor, bias: torch.Tensor) -> torch.Tensor:
    """y = GELU(y + bias) in place (bf16 [rows, N], erf form)."""
    N.require_device(y, bias)
    _bf16_rows(y, "y")
    lib = N.load_library()
    N.check(lib.omni_bias_gelu(y.data_ptr(), y.shape[0], y.shape[1], y.stride(0), bias.data_ptr(),
                               N.stream_handle(y.device)), "omni_bias_gelu")
    return y


def bias_scale_residual(r: torch.Tensor, y: torch.Tensor, bias: torch.Tensor, gamma: torch.Tensor,
                        out: torch.Tensor | None = None) -> torch.Tensor:
    """r [rows, C] float32 += gamma * (y + bias), y bf16 [rows, C]; out (bf16 [rows, C]) gets
    the new r rounded. Returns r."""
    N.require_device(r, y, bias, gamma, out)
    if r.dtype != torch.float32 or r.dim() != 2 or not r.is_contiguous():
        raise ValueError("r must be contiguous float32 [rows, C]")
    _bf16_rows(y, "y")
    if y.shape != r.shape or (out is not None and out.shape != r.shape):
        raise ValueError("y / out must match r")
    if out is not None:
        _bf16_rows(out, "out")
    lib = N.load_library()
    N.check(lib.omni_bias_scale_residual(r.data_ptr(), r.shape[0], r.shape[1], y.data_ptr(),
                                         y.stride(0), bias.data_ptr(), gamma.data_ptr(),
                                         N.ptr(out), 0 if out is None else out.stride(0),
                                         N.stream_handle(r.device)), "omni_bias_scale_residual")
    return r


def advance_positions(positions: torch.Tensor, slot_index: torch.Tensor, new_frames: int,
                      cold: bool) -> None:
    """positions[slot] = (0 if cold else positions[slot]) + new_frames for the rows' slots."""
    N.require_device(positions, slot_index)
    lib = N.load_library()
    N.check(lib.omni_advance_positions(positions.data_ptr(), positions.shape[0],
                                       slot_index.data_ptr(), slot_index.shape[0], new_frames,
                                       int(cold), N.stream_handle(positions.device)),
            "omni_advance_positions")
