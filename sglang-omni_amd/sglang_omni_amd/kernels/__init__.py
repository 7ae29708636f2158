"""HIP kernels for the codec/vocoder decode path, with the reference kernels' Python API."""

from .bias_snake_beta import SnakeBetaCoefficients, fused_bias_snake_beta
from .channel_embedding import ChannelEmbeddingTables
from .codec_state import history_exchange, overlap_exchange
from .conv import (
    PackedConv,
    ResidualUnitWeights,
    fused_conv,
    pack_conv1d,
    pack_conv_transpose1d,
    residual_stack,
)
from .rvq import rvq_gather_sum
from .single_output_conv import clamped_single_output_conv, single_output_conv

__all__ = [
    "ChannelEmbeddingTables",
    "PackedConv",
    "ResidualUnitWeights",
    "SnakeBetaCoefficients",
    "clamped_single_output_conv",
    "fused_bias_snake_beta",
    "fused_conv",
    "history_exchange",
    "overlap_exchange",
    "pack_conv1d",
    "pack_conv_transpose1d",
    "residual_stack",
    "rvq_gather_sum",
    "single_output_conv",
]
