"""Weight formats for the codec decoders: bf16 rounding and the fp8-weight conv path.

The reference's quantization glue (sglang_omni/quantization.py:137-187) has no conv / vocoder
path; this module adds one. Conv weights are stored as OCP E4M3 (``torch.float8_e4m3fn``) with a
float32 scale per output channel, ``s[co] = max|W[co]| / 448`` and ``q = e4m3(W / s)``; the conv
kernel dequantizes them to bf16 in LDS and applies ``s`` in its epilogue (W8A16 on bf16 MFMA).

``reference_weights`` returns the float32 weights a decoder with a given weight format actually
multiplies by (bf16-rounded, or fp8-dequantized), which is what a float32 reference of that
decoder must use.
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


def round_bf16(weights: dict[str, Any]) -> dict[str, Any]:
    """The weight tree with every conv weight and bias, and the codebooks, rounded to bf16
    (kept as float32 values). Snake alphas stay float32."""

    def conv(node: dict[str, Any], kind: str) -> dict[str, Any]:
        out = dict(node)
        out["weight"] = node["weight"].to(torch.bfloat16).float()
        if node.get("bias") is not None:
            out["bias"] = node["bias"].to(torch.bfloat16).float()
        return out

    out = _map_convs(weights, conv)
    if "codebooks" in weights:
        out["codebooks"] = weights["codebooks"].to(torch.bfloat16).float()
    return out


def fp8_dequantized(weights: dict[str, Any]) -> dict[str, Any]:
    """The weight tree with every conv weight replaced by its fp8 per-output-channel
    quantize -> dequantize round trip (biases bf16-rounded; codebooks bf16-rounded)."""

    def conv(node: dict[str, Any], kind: str) -> dict[str, Any]:
        out = dict(node)
        dim = 1 if kind == "transpose" else 0
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
