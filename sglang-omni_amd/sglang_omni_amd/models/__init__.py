"""Codec decoders on the HIP kernels."""

from .configs import (
    CODEC_24K,
    CODEC_24K_LONG,
    HIFIGAN_24K,
    QWEN3_CODE2WAV,
    QWEN3_TTS_CODEC,
    DacDecoderConfig,
    HifiGanConfig,
    Qwen3Code2WavConfig,
    Qwen3TTSCodecConfig,
    make_dac_weights,
    make_hifigan_weights,
    make_qwen3_code2wav_weights,
)
from .codec_state_arena import Qwen3TTSCodecStateArena
from .dac_codec import CodecStatePool, DacCodecDecoder
from .dac_weights import dac_weight_tree
from .graph_runner import CodecGraphRunner, GraphKey
from .hifigan import HifiGanVocoder
from .qwen3_code2wav import (
    Code2WavStatePool,
    Qwen3Code2WavDecoder,
    Qwen3TTSCodecDecoder,
    Qwen3TTSCodecState,
)

__all__ = [
    "CODEC_24K",
    "CODEC_24K_LONG",
    "HIFIGAN_24K",
    "QWEN3_CODE2WAV",
    "QWEN3_TTS_CODEC",
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
    "Qwen3TTSCodecConfig",
    "Qwen3TTSCodecDecoder",
    "Qwen3TTSCodecState",
    "Qwen3TTSCodecStateArena",
    "make_dac_weights",
    "make_hifigan_weights",
    "dac_weight_tree",
    "make_qwen3_code2wav_weights",
]
