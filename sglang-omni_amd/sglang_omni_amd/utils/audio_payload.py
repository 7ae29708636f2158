"""The audio payload wire format of the vocoder stage's output messages.

Same fields and encoding as ``sglang_omni/utils/audio_payload.py:13-65`` and
``build_audio_chunk_payload`` (``sglang_omni/scheduling/audio_stream.py:336-344``): the samples
as little-endian float32 bytes, their shape (flattened to one dimension unless a two-dimensional
waveform keeps its channels), the dtype name, and optionally the sample rate and modality.
Signed 16-bit PCM for realtime sessions is encoded on the device (``kernels.egress``).
"""

from __future__ import annotations

from collections.abc import Mapping

import numpy as np
import torch
from numpy.typing import ArrayLike


def audio_data_uri_from_reference(reference: Mapping[str, object]) -> str | None:
    """A data: URI for a reference audio mapping with base64 ``data`` (media type defaults to
    audio/wav), or None without data."""
    data = reference.get("data")
    if data is None:
        return None
    media_type = reference.get("media_type") or "audio/wav"
    return f"data:{media_type};base64,{data}"


def audio_waveform_payload(audio: ArrayLike | torch.Tensor, *, sample_rate: int | None = None,
                           modality: str | None = None, source_hint: str = "audio",
                           keep_channels: bool = False) -> dict[str, bytes | list[int] | str | int]:
    """Serialize a waveform: float32 bytes, shape, dtype, and the optional rate / modality. A
    (channels, samples) array keeps its shape with keep_channels; anything else is flattened."""
    if isinstance(audio, torch.Tensor):
        audio = audio.detach().float().cpu().numpy()
    try:
        array = np.asarray(audio, dtype=np.float32)
        if not (keep_channels and array.ndim == 2):
            array = array.reshape(-1)
    except (TypeError, ValueError) as exc:
        raise TypeError(f"Unsupported {source_hint} audio output type: {type(audio)}") from exc
    array = np.ascontiguousarray(array)
    payload: dict[str, bytes | list[int] | str | int] = {
        "audio_waveform": array.astype("<f4", copy=False).tobytes(),
        "audio_waveform_shape": list(array.shape),
        "audio_waveform_dtype": "float32",
    }
    if sample_rate is not None:
        payload["sample_rate"] = int(sample_rate)
    if modality is not None:
        payload["modality"] = modality
    return payload


def build_audio_chunk_payload(audio_data: ArrayLike | torch.Tensor, *,
                              sample_rate: int) -> dict[str, bytes | list[int] | str | int]:
    """A streamed chunk's payload (modality "audio")."""
    return audio_waveform_payload(audio_data, sample_rate=sample_rate, modality="audio",
                                  source_hint="streaming codec")


__all__ = ["audio_data_uri_from_reference", "audio_waveform_payload",
           "build_audio_chunk_payload"]
