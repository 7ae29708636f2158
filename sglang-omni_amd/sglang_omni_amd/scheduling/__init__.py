"""Host-side stepping around the codec kernels: waveform egress toward the host."""

from .waveform_egress import WaveformEgress

__all__ = ["WaveformEgress"]
