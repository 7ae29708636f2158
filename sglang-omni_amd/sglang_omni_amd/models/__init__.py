"""Codec decoders on the HIP kernels."""

from .configs import (
    CODEC_24K,
    CODEC_24K_LONG,
    HIFIGAN_24K,
    QWEN3_CODE2WAV,
    DacDecoderConfig,
    HifiGanConfig,
    Qwen3Code2WavConfig,
    make_dac_weights,
    make_hifigan_weights,
    make_qwen3_code2wav_weights,
)
from .dac_codec import CodecStatePool, DacCodecDecoder
from .graph_runner import CodecGraphRunner, GraphKey
from .hifigan import HifiGanVocoder
from .qwen3_code2wav import Code2WavStatePool, Qwen3Code2WavDecoder

__all__ = [
    "CODEC_24K",
    "CODEC_24K_LONG",
    "HIFIGAN_24K",
    "QWEN3_CODE2WAV",
    "Code2WavStatePool",
    "CodecGraphRunner",
    "CodecStatePool",
    "DacCodecDecoder",
    "DacDecoderConfig",
    "GraphKey",
    "HifiGanConfig",
    "HifiGanVocoder",
    "Qwen3Code2WavConfig",
    "Qwen3Code2WavDecoder",
    "make_dac_weights",
    "make_hifigan_weights",
    "make_qwen3_code2wav_weights",
]
