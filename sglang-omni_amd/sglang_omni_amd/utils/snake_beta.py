"""SnakeBeta for the Qwen3-TTS / Qwen3-Omni vocoders on the HIP kernel, with the interface of
sglang_omni/utils/snake_beta.py:200-328: ``fused_snake_beta``, the drop-in module
``FusedSnakeBeta``, ``prewarm`` and ``fuse_vocoder_decoder``.

The eager SnakeBeta forward on a bf16 tensor runs ``exp``, ``exp``, ``+ eps``, ``1 /``, ``*``,
``sin``, ``pow 2``, ``*``, ``+`` as separate ops, each computing in float32 and rounding to bf16.
``omni_snake_beta`` evaluates that chain per element with a round to bf16 after every step,
reading the module's raw log-scale parameters at every launch (a captured graph sees their
current values), so inside its envelope the result has the eager forward's bits:

    x [B, C, T] bf16, contiguous or the [B, C, T] view of a contiguous [B, T, C];
    alpha, beta bf16 [C] on x's GPU; 1 <= T <= MAX_T.

Outside the envelope ``fused_snake_beta`` returns None and ``FusedSnakeBeta`` runs the eager ops,
as the reference does. On a GPU the library must load: a missing library raises instead of
falling back.

``snake1d`` is the DAC Snake1d (x + (alpha + 1e-9)^-1 sin(alpha x)^2 in float32, rounded once) of
the channels-last decoder (sglang_omni/models/fishaudio_drama3/channels_last_decoder.py:35-67).
"""

from __future__ import annotations

import logging

import torch

from .. import _native as N

# the reference's envelope bound on T (sglang_omni/utils/snake_beta.py:58), kept so calls fall
# back exactly where the reference's do
MAX_T = 65535 * 1024

logger = logging.getLogger(__name__)


def _layout(x: torch.Tensor) -> int | None:
    """0 for a contiguous [B, C, T], 1 for the [B, C, T] view of a contiguous [B, T, C], None
    for any other layout."""
    if x.is_contiguous():
        return 0
    if x.transpose(1, 2).is_contiguous():
        return 1
    return None


@torch.library.custom_op("sglang_omni_amd::snake_beta", mutates_args=())
def launch(x: torch.Tensor, alpha: torch.Tensor, beta: torch.Tensor, eps: float) -> torch.Tensor:
    """One ``omni_snake_beta`` launch on the current stream (an opaque op to torch.compile)."""
    batch, channels, frames = x.shape
    y = torch.empty_like(x)  # keeps x's strides in both layouts
    lib = N.load_library()
    N.check(lib.omni_snake_beta(x.data_ptr(), y.data_ptr(), N.omni_dtype(x.dtype), batch,
                                channels, frames, _layout(x), alpha.data_ptr(), beta.data_ptr(),
                                N.omni_dtype(alpha.dtype), float(eps), N.stream_handle(x.device)),
            "omni_snake_beta")
    return y


@launch.register_fake
def _(x: torch.Tensor, alpha: torch.Tensor, beta: torch.Tensor, eps: float) -> torch.Tensor:
    return torch.empty_like(x)


def fused_snake_beta(x: torch.Tensor, alpha: torch.Tensor, beta: torch.Tensor,
                     eps: float) -> torch.Tensor | None:
    """SnakeBeta of x with the module's log-scale parameters and epsilon, bitwise equal to the
    eager forward, in x's layout; None outside the envelope (see the module docstring)."""
    if x.device.type != "cuda" or alpha.device != x.device or beta.device != x.device:
        return None
    if x.dtype != torch.bfloat16 or alpha.dtype != torch.bfloat16 or beta.dtype != torch.bfloat16:
        return None
    if x.dim() != 3 or x.numel() == 0 or x.shape[2] > MAX_T or _layout(x) is None:
        return None
    if tuple(alpha.shape) != (x.shape[1],) or tuple(beta.shape) != (x.shape[1],):
        return None
    return launch(x, alpha.contiguous(), beta.contiguous(), float(eps))


def _eager_snake_beta(x: torch.Tensor, alpha: torch.Tensor, beta: torch.Tensor,
                      eps: float) -> torch.Tensor:
    """SnakeBeta's own ops in its own order: the result outside the fused envelope."""
    a = torch.exp(alpha[None, :, None])
    b = torch.exp(beta[None, :, None])
    return x + (1.0 / (b + eps)) * torch.pow(torch.sin(x * a), 2)


class FusedSnakeBeta(torch.nn.Module):
    """Drop-in replacement for a SnakeBeta module that shares its parameters: the fused kernel
    inside the envelope, SnakeBeta's own ops outside it."""

    def __init__(self, original: torch.nn.Module) -> None:
        super().__init__()
        self.alpha = original.alpha
        self.beta = original.beta
        self.no_div_by_zero = original.no_div_by_zero
        self.train(original.training)

    def forward(self, hidden_states: torch.Tensor) -> torch.Tensor:
        out = fused_snake_beta(hidden_states, self.alpha, self.beta, self.no_div_by_zero)
        if out is None:
            out = _eager_snake_beta(hidden_states, self.alpha, self.beta, self.no_div_by_zero)
        return out


def prewarm(device: torch.device) -> None:
    """Load the library and run the kernel once per layout on `device`, so that nothing is
    loaded for the first time while a graph is being captured."""
    device = torch.device(device)
    if device.type != "cuda":
        return
    N.load_library()
    with torch.cuda.device(device):
        params = torch.zeros(8, dtype=torch.bfloat16, device=device)
        launch(torch.zeros(1, 8, 4, dtype=torch.bfloat16, device=device), params, params, 0.0)
        launch(torch.zeros(1, 4, 8, dtype=torch.bfloat16, device=device).transpose(1, 2),
               params, params, 0.0)


def prewarm_replacements(replacements: list[tuple[torch.nn.Module, str]]) -> None:
    """Prewarm every GPU the replaced modules' parameters live on."""
    for device in {getattr(parent, name).alpha.device for parent, name in replacements}:
        prewarm(device)


def fuse_vocoder_decoder(decoder: torch.nn.Module) -> int:
    """Replace every SnakeBeta (``SnakeBeta`` / ``Qwen3OmniMoeSnakeBeta``) child in `decoder`
    with a ``FusedSnakeBeta`` sharing its parameters; returns how many were replaced (0 on a
    second call). The kernel is prewarmed first: if that fails the decoder keeps its eager
    modules and 0 is returned. A GPU decoder with no library raises."""
    targets = [(parent, name) for parent in decoder.modules()
               for name, child in parent.named_children()
               if type(child).__name__ in ("SnakeBeta", "Qwen3OmniMoeSnakeBeta")]
    if not targets:
        return 0
    if any(getattr(p, n).alpha.device.type == "cuda" for p, n in targets):
        N.load_library()
    try:
        prewarm_replacements(targets)
    except Exception:
        logger.warning("SnakeBeta prewarm failed; the decoder keeps its eager modules",
                       exc_info=True)
        return 0
    for parent, name in targets:
        setattr(parent, name, FusedSnakeBeta(getattr(parent, name)))
    return len(targets)


def _snake(x: torch.Tensor, a: torch.Tensor, b: torch.Tensor, channels_last: bool,
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
    N.check(lib.omni_snake(x.data_ptr(), y.data_ptr(), N.omni_dtype(x.dtype), batch, frames,
                           channels, int(channels_last), a.data_ptr(), b.data_ptr(),
                           int(round_intermediates), N.stream_handle(x.device)), "omni_snake")
    return y


def snake1d(x: torch.Tensor, alpha: torch.Tensor, *, channels_last: bool = True) -> torch.Tensor:
    """DAC Snake1d: x + (alpha + 1e-9)^-1 sin(alpha x)^2 in float32, rounded once to x's dtype."""
    a = alpha.detach().float().reshape(-1)
    return _snake(x, a, (a + 1e-9).reciprocal(), channels_last, round_intermediates=False)


__all__ = ["FusedSnakeBeta", "MAX_T", "fuse_vocoder_decoder", "fused_snake_beta", "prewarm",
           "prewarm_replacements", "snake1d"]
