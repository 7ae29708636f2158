"""The audio payload wire format (sglang_omni/utils/audio_payload.py:13-65,
sglang_omni/scheduling/audio_stream.py:336-344) on the CPU."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from sglang_omni_amd.utils.audio_payload import (
    audio_data_uri_from_reference,
    audio_waveform_payload,
    build_audio_chunk_payload,
)


def test_payload_fields_and_bytes():
    wave = torch.linspace(-1, 1, 10).view(1, 1, 10)
    payload = audio_waveform_payload(wave, sample_rate=24000, modality="audio")
    assert payload["audio_waveform_shape"] == [10]
    assert payload["audio_waveform_dtype"] == "float32"
    assert payload["sample_rate"] == 24000 and payload["modality"] == "audio"
    decoded = np.frombuffer(payload["audio_waveform"], dtype="<f4")
    assert np.array_equal(decoded, wave.reshape(-1).numpy())


def test_payload_optional_fields_absent():
    payload = audio_waveform_payload(np.zeros(4, dtype=np.float64))
    assert set(payload) == {"audio_waveform", "audio_waveform_shape", "audio_waveform_dtype"}
    assert len(payload["audio_waveform"]) == 16  # float64 input travels as float32


def test_payload_keep_channels():
    stereo = np.arange(6, dtype=np.float32).reshape(2, 3)
    assert audio_waveform_payload(stereo, keep_channels=True)["audio_waveform_shape"] == [2, 3]
    assert audio_waveform_payload(stereo)["audio_waveform_shape"] == [6]
    # three dimensions never keep their shape
    cube = np.zeros((2, 1, 3), dtype=np.float32)
    assert audio_waveform_payload(cube, keep_channels=True)["audio_waveform_shape"] == [6]


def test_payload_rejects_non_numeric():
    with pytest.raises(TypeError, match="Unsupported streaming codec audio output type"):
        build_audio_chunk_payload(object(), sample_rate=16000)


def test_chunk_payload_modality():
    payload = build_audio_chunk_payload(torch.zeros(1, 1, 5), sample_rate=24000)
    assert payload["modality"] == "audio" and payload["sample_rate"] == 24000


def test_data_uri():
    assert audio_data_uri_from_reference({}) is None
    assert audio_data_uri_from_reference({"data": "QUJD"}) == "data:audio/wav;base64,QUJD"
    assert audio_data_uri_from_reference({"data": "QUJD", "media_type": "audio/ogg"}) == \
        "data:audio/ogg;base64,QUJD"
