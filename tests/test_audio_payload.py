"""The audio payload wire format (the keys built at sglang_omni/utils/audio_payload.py:23-65 and
sglang_omni/scheduling/audio_stream.py:336-344) on the CPU."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from sglang_omni_amd.utils.audio_payload import audio_waveform_payload, build_audio_chunk_payload


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
    with pytest.raises(TypeError, match="streaming codec audio of type object"):
        build_audio_chunk_payload(object(), sample_rate=16000)


def test_payload_of_lists_and_big_endian_arrays_is_little_endian_float32():
    payload = audio_waveform_payload([[0.5, -1.0], [2.0, 0.25]], keep_channels=True)
    assert payload["audio_waveform_shape"] == [2, 2]
    assert payload["audio_waveform"] == np.array([0.5, -1.0, 2.0, 0.25], dtype="<f4").tobytes()
    big = np.array([1.5, -2.0], dtype=">f8")
    assert audio_waveform_payload(big)["audio_waveform"] == np.array([1.5, -2.0], "<f4").tobytes()


def test_chunk_payload_modality():
    payload = build_audio_chunk_payload(torch.zeros(1, 1, 5), sample_rate=24000)
    assert payload["modality"] == "audio" and payload["sample_rate"] == 24000
