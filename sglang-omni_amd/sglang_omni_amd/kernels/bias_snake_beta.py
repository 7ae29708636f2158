"""``fused_bias_snake_beta`` (sglang_omni/kernels/bias_snake_beta.py:102-151) on the HIP kernel.

out = SnakeBeta(conv_output + bias [+ residual]) for bf16 / fp16 channels-last activations, with
the sum optionally kept in sum_out. Each step rounds to the activations' dtype exactly where the
unfused eager chain (add bias, add residual, then SnakeBeta's mul / sin / square / mul / add)
materializes a tensor, so the result has the eager chain's bits.

``SnakeBetaParameters`` and ``SnakeBetaCoefficients`` keep the reference's names and fields, the
interface its callers build the per-channel coefficients with (bias_snake_beta.py:19-42)."""

from __future__ import annotations

from dataclasses import dataclass
from typing import Protocol

import torch

from .. import _native as N


class SnakeBetaParameters(Protocol):
    """Anything holding a SnakeBeta module's parameters: log-scale ``alpha`` and ``beta`` per
    channel and the ``no_div_by_zero`` epsilon."""

    alpha: torch.Tensor
    beta: torch.Tensor
    no_div_by_zero: float


@dataclass(frozen=True, kw_only=True)
class SnakeBetaCoefficients:
    """Per-channel ``alpha_scale`` = exp(alpha) and ``inverse_beta`` = 1 / (exp(beta) + eps),
    evaluated once with the same torch ops (and dtype) as SnakeBeta's forward, so the kernel
    multiplies by the values the eager module would."""

    alpha_scale: torch.Tensor
    inverse_beta: torch.Tensor

    @classmethod
    @torch.no_grad()
    def from_activation(cls, activation: SnakeBetaParameters) -> "SnakeBetaCoefficients":
        return cls(
            alpha_scale=torch.exp(activation.alpha),
            inverse_beta=1.0 / (torch.exp(activation.beta) + activation.no_div_by_zero),
        )


def fused_bias_snake_beta(
    conv_output: torch.Tensor,
    bias: torch.Tensor | None,
    coefficients: SnakeBetaCoefficients,
    out: torch.Tensor,
    *,
    residual: torch.Tensor | None = None,
    sum_out: torch.Tensor | None = None,
) -> None:
    """Write SnakeBeta(conv_output + bias (+ residual)) into ``out`` and the pre-activation sum
    into ``sum_out`` when one is given. Tensors are [B, L, C] in bf16 or fp16: each batch row of
    conv_output and out is one contiguous [L, C] span (rows may be spaced further apart), while
    residual and sum_out are fully contiguous."""
    N.require_device(conv_output, out)
    batch, length, channels = conv_output.shape
    row = (channels, 1)
    if conv_output.stride()[1:] != row or out.stride()[1:] != row:
        raise ValueError("each row of conv_output and out is one contiguous span")
    if not all(t is None or t.is_contiguous() for t in (residual, sum_out)):
        raise ValueError("residual and sum_out are contiguous")
    dtype = out.dtype
    if conv_output.dtype != dtype:
        raise ValueError("conv_output and out share a dtype")
    pdt = coefficients.alpha_scale.dtype
    params = [t.to(pdt).contiguous() if t is not None else None
              for t in (bias, coefficients.alpha_scale, coefficients.inverse_beta)]
    lib = N.load_library()
    N.check(
        lib.omni_bias_snake_beta(
            conv_output.data_ptr(), conv_output.stride(0), batch, length, channels,
            N.ptr(params[0]), params[1].data_ptr(), params[2].data_ptr(), N.omni_dtype(pdt),
            N.ptr(residual), N.ptr(sum_out), out.data_ptr(), out.stride(0), N.omni_dtype(dtype),
            N.stream_handle(out.device),
        ),
        "omni_bias_snake_beta",
    )
