"""HiFT's short-time Fourier transform and its inverse on the HIP kernels.

``short_time_spectrum`` and ``overlap_add_inverse`` keep the names, argument order and layouts of
the reference's kernels (sglang_omni/models/fun_cosyvoice3/hift_kernels.py:304-360);
``HiftStft`` holds the bases the reference's channels-last HiFT builds
(sglang_omni/models/fun_cosyvoice3/hift_channels_last.py:88-125) and adds ``tail``, the
magnitude / phase / inverse / clamp of the vocoder's last conv output in one launch.
"""

from __future__ import annotations

import math

import torch

from .. import _native as N


def _check_f32(*tensors: torch.Tensor) -> None:
    for t in tensors:
        if t.dtype != torch.float32:
            raise ValueError("the transforms take float32 tensors")
        if not t.is_contiguous():
            raise ValueError("the transforms take contiguous tensors")


def _geometry(basis: torch.Tensor, hop_length: int) -> tuple[int, int]:
    components, n_fft = basis.shape
    bins = components // 2
    if components != 2 * bins or bins != n_fft // 2 + 1 or n_fft % hop_length:
        raise ValueError(f"basis {tuple(basis.shape)} and hop {hop_length}: need [2 * (n_fft // 2 "
                         f"+ 1), n_fft] with hop dividing n_fft")
    return n_fft, bins


def short_time_spectrum(padded_signal: torch.Tensor, basis: torch.Tensor,
                        hop_length: int) -> torch.Tensor:
    """padded_signal: (rows, samples) float32, already (reflect) padded; basis: (2 * bins, n_fft),
    the windowed cosines then the windowed negative sines. Returns (rows, 2 * bins, frames), the
    real parts then the imaginary parts."""
    return _spectrum(padded_signal, basis, hop_length, center=False)


def _spectrum(signal: torch.Tensor, basis: torch.Tensor, hop_length: int, *,
              center: bool) -> torch.Tensor:
    N.require_device(signal, basis)
    _check_f32(signal, basis)
    if signal.dim() != 2:
        raise ValueError("the signal must be (rows, samples)")
    n_fft, bins = _geometry(basis, hop_length)
    rows, samples = signal.shape
    padded = samples + 2 * (n_fft // 2) if center else samples
    if padded < n_fft:
        raise ValueError(f"{samples} samples are shorter than one {n_fft}-point frame")
    frames = (padded - n_fft) // hop_length + 1
    out = torch.empty(rows, 2 * bins, frames, dtype=torch.float32, device=signal.device)
    lib = N.load_library()
    N.check(lib.omni_short_time_spectrum(signal.data_ptr(), rows, samples, signal.stride(0),
                                         int(center), basis.data_ptr(), bins, n_fft, hop_length,
                                         out.data_ptr(), frames, N.stream_handle(signal.device)),
            "omni_short_time_spectrum")
    return out


def overlap_add_inverse(real: torch.Tensor, imaginary: torch.Tensor, basis: torch.Tensor,
                        squared_window: torch.Tensor, hop_length: int) -> torch.Tensor:
    """torch.istft with center=True over real, imaginary: (rows, bins, frames) float32; basis:
    (2 * bins, n_fft), the one-sided inverse's windowed cosines then negative sines over n_fft.
    Returns (rows, hop_length * (frames - 1))."""
    N.require_device(real, imaginary, basis, squared_window)
    _check_f32(real, imaginary, basis, squared_window)
    n_fft, bins = _geometry(basis, hop_length)
    if real.dim() != 3 or real.shape != imaginary.shape or real.shape[1] != bins:
        raise ValueError("real and imaginary must be (rows, bins, frames) of one shape")
    rows, _, frames = real.shape
    out = torch.empty(rows, hop_length * (frames - 1), dtype=torch.float32, device=real.device)
    lib = N.load_library()
    N.check(lib.omni_overlap_add_inverse(real.data_ptr(), imaginary.data_ptr(), rows, bins, frames,
                                         basis.data_ptr(), squared_window.data_ptr(), n_fft,
                                         hop_length, out.data_ptr(), out.stride(0),
                                         N.stream_handle(real.device)),
            "omni_overlap_add_inverse")
    return out


class HiftStft:
    """The transforms of one HiFT configuration (Hann window of n_fft, hop), with the bases
    built in float64 and rounded once to float32 as hift_channels_last.py:88-106 builds them."""

    def __init__(self, window: torch.Tensor, hop_length: int, *, device: torch.device | str,
                 magnitude_clip: float = 100.0, audio_limit: float = 0.99):
        n_fft = window.shape[0]
        self.n_fft, self.hop_length, self.bins = n_fft, hop_length, n_fft // 2 + 1
        self.magnitude_clip, self.audio_limit = float(magnitude_clip), float(audio_limit)
        w = window.to(torch.float64)
        angle = (2 * math.pi / n_fft) * torch.outer(torch.arange(self.bins, dtype=torch.float64),
                                                    torch.arange(n_fft, dtype=torch.float64))
        self.forward_basis = (torch.cat([torch.cos(angle), -torch.sin(angle)]) * w).float().to(device)
        one_sided = torch.full((self.bins, 1), 2.0, dtype=torch.float64)
        one_sided[0] = 1.0
        one_sided[-1] = 1.0
        self.inverse_basis = (torch.cat([torch.cos(angle) * one_sided,
                                         -torch.sin(angle) * one_sided]) * w / n_fft).float().to(device)
        self.squared_window = window.float().pow(2).to(device).contiguous()

    def spectrum(self, signal: torch.Tensor) -> torch.Tensor:
        """The centred short-time spectrum of (rows, samples): (rows, 2 * bins, frames), the
        reflect padding done by the kernel."""
        return _spectrum(signal.contiguous(), self.forward_basis, self.hop_length, center=True)

    def inverse(self, magnitude: torch.Tensor, phase: torch.Tensor) -> torch.Tensor:
        """The inverse transform of (rows, bins, frames) magnitudes (clipped above at
        magnitude_clip) and phases, as hift_channels_last.py:117-125."""
        magnitude = torch.clip(magnitude, max=self.magnitude_clip)
        return overlap_add_inverse((magnitude * torch.cos(phase)).contiguous(),
                                   (magnitude * torch.sin(phase)).contiguous(),
                                   self.inverse_basis, self.squared_window, self.hop_length)

    def tail(self, h: torch.Tensor) -> torch.Tensor:
        """The vocoder's output from its last conv h (rows, frames, >= 2 * bins channels-last,
        float32): magnitude exp(h[..., :bins]) clipped, phase sin(h[..., bins:2 bins]), inverse,
        clamp to +-audio_limit (hift_channels_last.py:269-276) — one launch.
        Returns (rows, hop * (frames - 1))."""
        N.require_device(h)
        if h.dtype != torch.float32 or h.dim() != 3 or h.shape[2] < 2 * self.bins or h.stride(2) != 1:
            raise ValueError("h must be float32 (rows, frames, >= 2 * bins) with channel stride 1")
        rows, frames, _ = h.shape
        out = torch.empty(rows, self.hop_length * (frames - 1), dtype=torch.float32,
                          device=h.device)
        lib = N.load_library()
        N.check(lib.omni_istft_tail(h.data_ptr(), rows, frames, h.stride(0), h.stride(1),
                                    self.inverse_basis.data_ptr(),
                                    self.squared_window.data_ptr(), self.bins, self.n_fft,
                                    self.hop_length, self.magnitude_clip, self.audio_limit,
                                    out.data_ptr(), out.stride(0), N.stream_handle(h.device)),
                "omni_istft_tail")
        return out
