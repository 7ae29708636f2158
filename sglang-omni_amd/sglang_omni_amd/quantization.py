"""Weight formats for the codec decoders: bf16 rounding and the fp8-weight conv path.

The reference's quantization glue (sglang_omni/quantization.py:137-187) has no conv / vocoder
path; this module adds one. Conv weights are stored as OCP E4M3 (``torch.float8_e4m3fn``) with a
float32 scale per output channel, ``s[co] = max|W[co]| / 448`` and ``q = e4m3(W / s)``; the conv
kernel dequantizes them to bf16 in LDS and applies ``s`` in its epilogue (W8A16 on bf16 MFMA).

``reference_weights`` returns the float32 weights a decoder with a given weight format actually
multiplies by (bf16-rounded, or fp8-dequantized), which is what a float32 reference of that
decoder must use.

Checkpoints that already hold E4M3 weights carry a dequantization multiplier named
``weight_scale_inv`` (per tensor, per output channel, or per [rows x cols] block of the weight
flattened to [C_out, C_in * k]); ``fp8_conv_weight`` maps one onto this module's format, with the
reference's checks and its optional reciprocal (sglang_omni/quantization.py:137-166,
``convert_fp8_weight_scale_inv``). A conv dict of a weight tree may then hold the E4M3 ``weight``
with its ``weight_scale`` [C_out], which the decoders pack as they are.
"""

from __future__ import annotations

from typing import Any

import torch

FP8_E4M3_MAX = 448.0


def quantize_fp8(weight: torch.Tensor, channel_dim: int) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-output-channel E4M3 quantization along ``channel_dim``; returns (q, scale float32)."""
    w = weight.float().movedim(channel_dim, 0)
    amax = w.reshape(w.shape[0], -1).abs().amax(dim=1)
    scale = torch.where(amax > 0, amax / FP8_E4M3_MAX, torch.ones_like(amax))
    q = (w / scale.view(-1, *([1] * (w.dim() - 1)))).to(torch.float8_e4m3fn)
    return q.movedim(0, channel_dim).contiguous(), scale


def dequantize_fp8(q: torch.Tensor, scale: torch.Tensor, channel_dim: int) -> torch.Tensor:
    shape = [1] * q.dim()
    shape[channel_dim] = -1
    return q.float() * scale.view(shape)


def checkpoint_fp8_multiplier(name: str, scale: torch.Tensor, *, inverted: bool) -> torch.Tensor:
    """A checkpoint's ``weight_scale_inv`` as the float32 multiplier that dequantizes its E4M3
    weight, refusing what the reference's loader refuses: a non-floating-point, empty,
    non-finite or zero scale. ``inverted`` checkpoints store the multiplier's reciprocal."""
    if not torch.is_floating_point(scale):
        raise TypeError(f"FP8 scale tensor for {name} must be floating point")
    if scale.numel() == 0:
        raise ValueError(f"FP8 scale tensor for {name} is empty")
    if not bool(torch.isfinite(scale).all()):
        raise ValueError(f"FP8 scale tensor for {name} holds non-finite values")
    if bool((scale == 0).any()):
        raise ValueError(f"FP8 scale tensor for {name} holds zeros")
    scale = scale.detach().float()
    return scale.reciprocal() if inverted else scale


def fp8_conv_weight(name: str, weight: torch.Tensor, scale_inv: torch.Tensor, *,
                    inverted: bool = False, block_size: tuple[int, int] | None = None,
                    transposed: bool = False) -> tuple[torch.Tensor, torch.Tensor]:
    """(E4M3 weight, float32 scale per output channel) for the conv kernels from a checkpoint's
    E4M3 conv weight ([C_out, C_in, k], or [C_in, C_out, k] when ``transposed``) and its
    ``weight_scale_inv``: a scalar, one value per output channel, or (Conv1d only, with
    ``block_size`` = (rows, cols)) one per block of the weight viewed as [C_out, C_in * k].
    Per-tensor and per-channel multipliers, and blocks whose multipliers are constant along each
    row of blocks, map exactly; other block layouts are dequantized and requantized per output
    channel (one E4M3 rounding)."""
    if weight.dtype != torch.float8_e4m3fn or weight.dim() != 3:
        raise ValueError(f"{name}: expected a 3-dimensional float8_e4m3fn conv weight")
    m = checkpoint_fp8_multiplier(name, scale_inv, inverted=inverted)
    ch_dim = 1 if transposed else 0
    c_out = weight.shape[ch_dim]
    if m.numel() == 1:
        return weight, m.reshape(1).expand(c_out).contiguous()
    if block_size is None:
        if m.numel() != c_out:
            raise ValueError(f"{name}: {m.numel()} scales for {c_out} output channels")
        return weight, m.reshape(c_out).contiguous()
    if transposed:
        raise ValueError(f"{name}: block scales are read for Conv1d weights only")
    rows, cols = block_size
    flat = weight.reshape(c_out, -1)
    blocks = (-(-c_out // rows), -(-flat.shape[1] // cols))
    if tuple(m.shape) != blocks:
        raise ValueError(f"{name}: block scales of shape {tuple(m.shape)}, expected {blocks}")
    if bool((m == m[:, :1]).all()):
        return weight, m[:, 0].repeat_interleave(rows)[:c_out].contiguous()
    full = m.repeat_interleave(rows, 0)[:c_out].repeat_interleave(cols, 1)[:, :flat.shape[1]]
    dense = (flat.float() * full).reshape(weight.shape)
    return quantize_fp8(dense, 0)


def _map_convs(weights: dict[str, Any], fn) -> dict[str, Any]:
    """Apply fn(conv_dict, kind) to every conv of a DAC or HiFiGAN weight tree; copies the rest."""

    def walk(node: Any, key: str | None) -> Any:
        if isinstance(node, dict):
            if "weight" in node and isinstance(node["weight"], torch.Tensor):
                kind = "transpose" if key == "up" else "conv"
                return fn(node, kind)
            return {k: walk(v, k) for k, v in node.items()}
        if isinstance(node, list):
            return [walk(v, key) for v in node]
        return node

    return walk(weights, None)


def _float_weight(node: dict[str, Any], kind: str) -> torch.Tensor:
    """A conv dict's weight as float32 values: an E4M3 weight dequantized by its
    ``weight_scale`` (per output channel)."""
    w = node["weight"]
    if w.dtype == torch.float8_e4m3fn:
        return dequantize_fp8(w, node["weight_scale"], 1 if kind == "transpose" else 0)
    return w


def round_bf16(weights: dict[str, Any]) -> dict[str, Any]:
    """The weight tree with every conv weight and bias, and the codebooks, rounded to bf16
    (kept as float32 values). Snake alphas stay float32."""

    def conv(node: dict[str, Any], kind: str) -> dict[str, Any]:
        out = {k: v for k, v in node.items() if k != "weight_scale"}
        out["weight"] = _float_weight(node, kind).to(torch.bfloat16).float()
        if node.get("bias") is not None:
            out["bias"] = node["bias"].to(torch.bfloat16).float()
        return out

    out = _map_convs(weights, conv)
    if "codebooks" in weights:
        out["codebooks"] = weights["codebooks"].to(torch.bfloat16).float()
    return out


def fp8_dequantized(weights: dict[str, Any]) -> dict[str, Any]:
    """The weight tree with every conv weight replaced by the values its fp8 form holds: the
    per-output-channel quantize -> dequantize round trip of a float weight, or an E4M3 weight
    dequantized by its own scale (biases bf16-rounded; codebooks bf16-rounded)."""

    def conv(node: dict[str, Any], kind: str) -> dict[str, Any]:
        out = {k: v for k, v in node.items() if k != "weight_scale"}
        dim = 1 if kind == "transpose" else 0
        if node["weight"].dtype == torch.float8_e4m3fn:
            out["weight"] = _float_weight(node, kind)
        else:
            q, s = quantize_fp8(node["weight"], dim)
            out["weight"] = dequantize_fp8(q, s, dim)
        if node.get("bias") is not None:
            out["bias"] = node["bias"].to(torch.bfloat16).float()
        return out

    out = _map_convs(weights, conv)
    if "codebooks" in weights:
        out["codebooks"] = weights["codebooks"].to(torch.bfloat16).float()
    return out


def reference_weights(weights: dict[str, Any], weight_format: str) -> dict[str, Any]:
    """The float32 weights a decoder in ``weight_format`` ("bf16" or "fp8") computes with."""
    if weight_format == "bf16":
        return round_bf16(weights)
    if weight_format == "fp8":
        return fp8_dequantized(weights)
    raise ValueError(f"unknown weight format {weight_format!r}")
