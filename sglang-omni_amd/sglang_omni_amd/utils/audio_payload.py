"""The audio payload the vocoder stage puts on the wire.

The keys and their encoding are the relay's wire format (sglang_omni/utils/audio_payload.py:
23-65 builds them, sglang_omni/scheduling/audio_stream.py:336-344 for streamed chunks), so they
are kept exactly: ``audio_waveform`` holds the samples as little-endian float32 bytes,
``audio_waveform_shape`` their shape (one dimension, or [channels, samples] when a two-dimensional
waveform keeps its channels), ``audio_waveform_dtype`` the string "float32", and ``sample_rate``
/ ``modality`` appear only when given. Signed 16-bit PCM for realtime sessions is produced on the
device instead (``kernels.egress``).
"""

from __future__ import annotations

from typing import Any

import numpy as np
import torch

_LITTLE_ENDIAN_F32 = np.dtype("<f4")


def _samples(audio: Any, keep_channels: bool, what: str) -> np.ndarray:
    """The waveform as a C-ordered little-endian float32 array: kept [channels, samples] when
    asked and two-dimensional, one dimension otherwise."""
    if isinstance(audio, torch.Tensor):
        array = audio.detach().to(device="cpu", dtype=torch.float32).numpy()
    else:
        try:
            array = np.asarray(audio, dtype=np.float32)
        except (TypeError, ValueError) as exc:
            raise TypeError(f"{what} audio of type {type(audio).__name__} is not a waveform of "
                            "numbers") from exc
    if array.ndim != 2 or not keep_channels:
        array = array.reshape(-1)
    return np.ascontiguousarray(array, dtype=_LITTLE_ENDIAN_F32)


def audio_waveform_payload(audio: Any, *, sample_rate: int | None = None,
                           modality: str | None = None, source_hint: str = "audio",
                           keep_channels: bool = False) -> dict[str, bytes | list[int] | str | int]:
    """The wire payload of a waveform (a tensor, array or nested sequence of numbers);
    ``source_hint`` names the producer in the error raised for anything else."""
    samples = _samples(audio, keep_channels, source_hint)
    payload: dict[str, bytes | list[int] | str | int] = {
        "audio_waveform": samples.tobytes(),
        "audio_waveform_shape": [int(n) for n in samples.shape],
        "audio_waveform_dtype": "float32",
    }
    for key, value in (("sample_rate", None if sample_rate is None else int(sample_rate)),
                       ("modality", modality)):
        if value is not None:
            payload[key] = value
    return payload


def build_audio_chunk_payload(audio_data: Any, *,
                              sample_rate: int) -> dict[str, bytes | list[int] | str | int]:
    """A streamed chunk's payload: modality "audio" and its sample rate."""
    return audio_waveform_payload(audio_data, sample_rate=sample_rate, modality="audio",
                                  source_hint="streaming codec")


__all__ = ["audio_waveform_payload", "build_audio_chunk_payload"]
