"""Architectures of the codec decoders this package decodes, and seeded random weights for them.

The DAC-style decoder is the causal codec decoder of
sglang_omni/models/fishaudio_s2_pro/fish_speech/models/dac/modded_dac.py:742-835 fed by an RVQ
gather-sum; the HiFiGAN body is the mel -> wave generator of
sglang_omni/models/minicpm_o/components/token2wav/hift.py:95-156,255-281.

Weights are nested dicts of float32 CPU tensors in the reference's own layouts (Conv1d
``[C_out, C_in, k]``, ConvTranspose1d ``[C_in, C_out, k]``), so the same master weights feed
both the GPU decoder (which packs them) and any float32 reference.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Any

import torch


@dataclass(frozen=True)
class DacDecoderConfig:
    """RVQ tables + causal DAC decoder (input conv, upsampling blocks of Snake -> ConvTranspose
    (k = 2s) -> residual units, final Snake -> conv to one channel -> tanh)."""

    n_codebooks: int = 16
    codebook_size: int = 2048
    latent_dim: int = 512
    channels: int = 1536
    rates: tuple[int, ...] = (8, 8, 5, 6)
    dilations: tuple[int, ...] = (1, 3, 9)
    kernel_size: int = 7
    sample_rate: int = 24000
    codebook_std: float = 0.02
    # kaiming_normal_(mode="fan_in") gain for every conv. 0.85 keeps the random decoder in the
    # regime a trained codec operates in: output RMS ~0.035 inside tanh's linear range, and a
    # bf16-activation decode ~44 dB from float32. At gain 1 the random Snake stack grows 15x and
    # becomes chaotic (bf16 rounding alone costs ~7 dB); at sqrt(2) it saturates tanh.
    conv_gain: float = 0.85
    snake_alpha: float = 1.0

    @property
    def hop_length(self) -> int:
        return int(math.prod(self.rates))

    @property
    def frame_rate(self) -> float:
        return self.sample_rate / self.hop_length

    def stage_channels(self) -> list[int]:
        return [self.channels // 2**i for i in range(len(self.rates) + 1)]


@dataclass(frozen=True)
class HifiGanConfig:
    """HiFiGAN mel -> wave body: conv_pre k=7, per stage LeakyReLU -> ConvTranspose1d(k, u,
    padding (k-u)//2) -> mean of multi-receptive-field ResBlocks, LeakyReLU(0.01) -> conv_post
    to one channel k=7 -> tanh."""

    n_mels: int = 80
    channels: int = 512
    rates: tuple[int, ...] = (8, 5, 3, 4)
    up_kernels: tuple[int, ...] = (16, 11, 7, 8)
    resblock_kernels: tuple[int, ...] = (3, 7, 11)
    resblock_dilations: tuple[tuple[int, ...], ...] = ((1, 3, 5), (1, 3, 5), (1, 3, 5))
    slope: float = 0.1
    final_slope: float = 0.01
    sample_rate: int = 24000
    # kaiming fan_in gain: output RMS ~0.06, a bf16-activation decode ~46 dB from float32
    conv_gain: float = 0.8

    @property
    def hop_length(self) -> int:
        return int(math.prod(self.rates))


# The workloads' architectures.
SINGLE_BLOCK = dict(n_codebooks=8, codebook_size=1024, latent_dim=256)  # RVQ + one conv block
CODEC_24K = DacDecoderConfig()  # 16 x 2048 x 512 tables, 1536 ch, x1920 to 24 kHz
CODEC_24K_LONG = DacDecoderConfig(n_codebooks=32, codebook_size=1024)  # fp8-weight long form
HIFIGAN_24K = HifiGanConfig()


def _kaiming(shape: tuple[int, ...], fan_in: int, gain: float, gen: torch.Generator) -> torch.Tensor:
    std = gain / math.sqrt(fan_in)
    return torch.randn(shape, generator=gen, dtype=torch.float32) * std


def _conv(c_out: int, c_in: int, k: int, gain: float, gen: torch.Generator) -> dict[str, torch.Tensor]:
    return {
        "weight": _kaiming((c_out, c_in, k), c_in * k, gain, gen),
        "bias": torch.zeros(c_out, dtype=torch.float32),
    }


def _conv_t(c_in: int, c_out: int, k: int, gain: float, gen: torch.Generator) -> dict[str, torch.Tensor]:
    # torch's kaiming fan_in for a ConvTranspose1d weight [C_in, C_out, k] is C_out * k
    return {
        "weight": _kaiming((c_in, c_out, k), c_out * k, gain, gen),
        "bias": torch.zeros(c_out, dtype=torch.float32),
    }


def make_dac_weights(config: DacDecoderConfig, seed: int = 0) -> dict[str, Any]:
    """Seeded float32 master weights: codebooks ~ N(0, codebook_std); every conv
    kaiming-normal (fan_in, ``conv_gain``) with zero bias; Snake alphas = ``snake_alpha``."""
    gen = torch.Generator().manual_seed(seed)
    g = config.conv_gain
    chans = config.stage_channels()
    weights: dict[str, Any] = {
        "codebooks": torch.randn(
            (config.n_codebooks, config.codebook_size, config.latent_dim),
            generator=gen,
            dtype=torch.float32,
        )
        * config.codebook_std,
        "in_conv": _conv(chans[0], config.latent_dim, config.kernel_size, g, gen),
        "blocks": [],
    }
    for i, stride in enumerate(config.rates):
        c_in, c_out = chans[i], chans[i + 1]
        block = {
            "stride": stride,
            "alpha": torch.full((c_in,), config.snake_alpha),
            "up": _conv_t(c_in, c_out, 2 * stride, g, gen),
            "units": [],
        }
        for d in config.dilations:
            block["units"].append(
                {
                    "dilation": d,
                    "alpha1": torch.full((c_out,), config.snake_alpha),
                    "conv1": _conv(c_out, c_out, config.kernel_size, g, gen),
                    "alpha2": torch.full((c_out,), config.snake_alpha),
                    "conv2": _conv(c_out, c_out, 1, g, gen),
                }
            )
        weights["blocks"].append(block)
    weights["final"] = {
        "alpha": torch.full((chans[-1],), config.snake_alpha),
        "conv": _conv(1, chans[-1], config.kernel_size, g, gen),
    }
    return weights


def make_hifigan_weights(config: HifiGanConfig, seed: int = 0) -> dict[str, Any]:
    """Seeded float32 HiFiGAN weights (kaiming-normal fan_in with ``conv_gain``, zero bias)."""
    gen = torch.Generator().manual_seed(seed)
    g = config.conv_gain
    weights: dict[str, Any] = {
        "slope": config.slope,
        "final_slope": config.final_slope,
        "conv_pre": _conv(config.channels, config.n_mels, 7, g, gen),
        "stages": [],
    }
    c = config.channels
    for rate, k in zip(config.rates, config.up_kernels):
        c_out = c // 2
        stage = {"rate": rate, "up": _conv_t(c, c_out, k, g, gen), "resblocks": []}
        for rk, dils in zip(config.resblock_kernels, config.resblock_dilations):
            stage["resblocks"].append(
                {
                    "kernel": rk,
                    "dilations": tuple(dils),
                    "convs1": [_conv(c_out, c_out, rk, g, gen) for _ in dils],
                    "convs2": [_conv(c_out, c_out, rk, g, gen) for _ in dils],
                }
            )
        weights["stages"].append(stage)
        c = c_out
    weights["conv_post"] = _conv(1, c, 7, g, gen)
    return weights


def dac_macs_per_frame(config: DacDecoderConfig) -> int:
    """Multiply-accumulates of the decoder convs per code frame (the algorithmic work)."""
    chans = config.stage_channels()
    k = config.kernel_size
    macs = chans[0] * config.latent_dim * k
    samples = 1
    for i, s in enumerate(config.rates):
        c_in, c_out = chans[i], chans[i + 1]
        macs += samples * c_in * c_out * 2 * s  # transposed conv: every input sample x 2s taps
        samples *= s
        for _ in config.dilations:
            macs += samples * (c_out * c_out * k + c_out * c_out)
    macs += samples * chans[-1] * k
    return macs


def hifigan_macs_per_frame(config: HifiGanConfig) -> int:
    """Multiply-accumulates of the HiFiGAN convs per mel frame."""
    c = config.channels
    macs = c * config.n_mels * 7
    samples = 1
    for rate, k in zip(config.rates, config.up_kernels):
        c_out = c // 2
        macs += samples * c * c_out * k
        samples *= rate
        for rk, dils in zip(config.resblock_kernels, config.resblock_dilations):
            macs += samples * len(dils) * 2 * c_out * c_out * rk
        c = c_out
    macs += samples * c * 7
    return macs
