"""Host-side stepping around the codec kernels: the serving step loop and waveform egress."""

from .step_loop import CodecStepLoop
from .waveform_egress import WaveformEgress

__all__ = ["CodecStepLoop", "WaveformEgress"]
