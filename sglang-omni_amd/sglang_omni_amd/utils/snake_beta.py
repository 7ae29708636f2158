"""Snake-family activations on the GPU with the reference's module-level API.

``fused_snake_beta`` mirrors sglang_omni/utils/snake_beta.py:200-234 (SnakeBeta with log-scale
alpha/beta, rounded like the eager bf16 op chain); ``snake1d`` mirrors the DAC ``Snake1d``
channels-last kernel (sglang_omni/models/fishaudio_drama3/channels_last_decoder.py:35-67), which
computes in float32 and rounds once.
"""

from __future__ import annotations

import torch

from .. import _native as N


def _run(x: torch.Tensor, a: torch.Tensor, b: torch.Tensor, channels_last: bool,
         round_intermediates: bool) -> torch.Tensor:
    N.require_device(x)
    if not x.is_contiguous():
        raise ValueError("x must be contiguous")
    if channels_last:
        batch, frames, channels = x.shape
    else:
        batch, channels, frames = x.shape
    y = torch.empty_like(x)
    a = a.detach().float().reshape(-1).contiguous()
    b = b.detach().float().reshape(-1).contiguous()
    N.require_vector(a, channels, "alpha", x.device)
    N.require_vector(b, channels, "beta", x.device)
    lib = N.load_library()
    N.check(
        lib.omni_snake(x.data_ptr(), y.data_ptr(), N.omni_dtype(x.dtype), batch, frames, channels,
                       int(channels_last), a.data_ptr(), b.data_ptr(), int(round_intermediates),
                       N.stream_handle(x.device)),
        "omni_snake",
    )
    return y


def fused_snake_beta(
    x: torch.Tensor, alpha: torch.Tensor, beta: torch.Tensor, eps: float = 1e-9,
    *, channels_last: bool = False
) -> torch.Tensor:
    """SnakeBeta x + 1/(exp(beta) + eps) * sin(x * exp(alpha))^2 of a [B, C, T] (or channels-last
    [B, T, C]) tensor, rounded after each op as the eager chain in x's dtype does."""
    a = torch.exp(alpha.detach().float())
    b = 1.0 / (torch.exp(beta.detach().float()) + eps)
    if x.dtype in (torch.bfloat16, torch.float16):
        # the eager chain computes exp(alpha) and 1/(exp(beta)+eps) in the parameters' dtype
        a = a.to(x.dtype).float()
        b = b.to(x.dtype).float()
    return _run(x, a, b, channels_last, round_intermediates=x.dtype != torch.float32)


def snake1d(x: torch.Tensor, alpha: torch.Tensor, *, channels_last: bool = True) -> torch.Tensor:
    """DAC Snake1d: x + (alpha + 1e-9)^-1 sin(alpha x)^2 in float32, rounded once to x's dtype."""
    a = alpha.detach().float().reshape(-1)
    return _run(x, a, (a + 1e-9).reciprocal(), channels_last, round_intermediates=False)


class FusedSnakeBeta(torch.nn.Module):
    """Drop-in SnakeBeta module (log-scale alpha/beta, [B, C, T]) running the HIP kernel."""

    def __init__(self, alpha: torch.Tensor, beta: torch.Tensor, no_div_by_zero: float = 1e-9):
        super().__init__()
        self.alpha = torch.nn.Parameter(alpha.detach().clone(), requires_grad=False)
        self.beta = torch.nn.Parameter(beta.detach().clone(), requires_grad=False)
        self.no_div_by_zero = no_div_by_zero

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return fused_snake_beta(x.contiguous(), self.alpha, self.beta, self.no_div_by_zero)
