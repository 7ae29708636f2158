"""Host-side stepping around the codec kernels: waveform egress toward the host."""

from .waveform_egress import PendingStep, WaveformEgress

__all__ = ["PendingStep", "WaveformEgress"]
