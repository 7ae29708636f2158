"""Codec decoders on the HIP kernels."""

from .configs import (
    CODEC_24K,
    CODEC_24K_LONG,
    HIFIGAN_24K,
    DacDecoderConfig,
    HifiGanConfig,
    make_dac_weights,
    make_hifigan_weights,
)
from .dac_codec import CodecStatePool, DacCodecDecoder
from .graph_runner import CodecGraphRunner, GraphKey
from .hifigan import HifiGanVocoder

__all__ = [
    "CODEC_24K",
    "CODEC_24K_LONG",
    "HIFIGAN_24K",
    "CodecGraphRunner",
    "CodecStatePool",
    "DacCodecDecoder",
    "DacDecoderConfig",
    "GraphKey",
    "HifiGanConfig",
    "HifiGanVocoder",
    "make_dac_weights",
    "make_hifigan_weights",
]
