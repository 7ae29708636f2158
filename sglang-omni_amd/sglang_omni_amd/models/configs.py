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
from dataclasses import dataclass
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


@dataclass(frozen=True)
class Qwen3Code2WavConfig:
    """Qwen3-Omni code2wav (Qwen3OmniMoeCode2WavConfig's fields and defaults,
    transformers configuration_qwen3_omni_moe.py): code embedding mean -> sliding-window
    pre-transformer -> ConvNeXt upsamplers (x2, x2) -> causal decoder blocks of SnakeBeta ->
    transposed conv (k = 2s, trimmed on both sides) -> residual units -> SnakeBeta -> conv to one
    channel -> clamp."""

    codebook_size: int = 2048
    num_quantizers: int = 16
    hidden_size: int = 1024
    num_hidden_layers: int = 8
    num_attention_heads: int = 16
    num_key_value_heads: int = 16
    intermediate_size: int = 3072
    sliding_window: int = 72
    rms_norm_eps: float = 1e-5
    rope_theta: float = 10000.0
    layer_scale_initial_scale: float = 0.01
    decoder_dim: int = 1536
    upsample_rates: tuple[int, ...] = (8, 5, 4, 3)
    upsampling_ratios: tuple[int, ...] = (2, 2)
    sample_rate: int = 24000
    # the decoder's conv stack, in the vocabulary of DacDecoderConfig
    kernel_size: int = 7
    dilations: tuple[int, ...] = (1, 3, 9)
    transconv_trim: str = "both"
    final_activation: str = "clamp"
    # random-init gains (no checkpoint here): kaiming fan_in gain for the decoder convs, and
    # for the input conv, whose operand (the ConvNeXt output, RMS ~1) is ~12x the RVQ sum the
    # DAC decoder's input conv sees
    conv_gain: float = 0.85
    input_conv_gain: float = 0.08

    @property
    def head_dim(self) -> int:
        return self.hidden_size // self.num_attention_heads

    @property
    def hop_length(self) -> int:
        return int(math.prod(self.upsample_rates) * math.prod(self.upsampling_ratios))

    @property
    def channels(self) -> int:
        return self.decoder_dim

    @property
    def rates(self) -> tuple[int, ...]:
        return self.upsample_rates

    def stage_channels(self) -> list[int]:
        return [self.decoder_dim // 2**i for i in range(len(self.upsample_rates) + 1)]


@dataclass(frozen=True)
class Qwen3TTSCodecConfig:
    """Qwen3-TTS tokenizer (12 Hz) decoder, as the reference's Qwen3TTSIncrementalDecoder walks
    it (sglang_omni/models/qwen3_tts/incremental_codec.py:771-1276): split RVQ dequantize
    (semantic codebooks and acoustic codebooks, each group summed and projected to latent_dim)
    -> causal pre_conv -> input_proj -> sliding-window pre-transformer (heads * head_dim wide
    attention) -> RMSNorm -> output_proj -> ConvNeXt upsamplers (x2, x2) at latent_dim -> the
    causal decoder blocks of Qwen3-Omni's code2wav with transposed convs trimmed on the right
    only (every decode emits frames * 1920 samples) -> SnakeBeta -> conv to one channel ->
    clamp. The transformer sizes are those of the reference's own test of the decoder
    transformer (tests/unit_test/qwen3_tts/test_incremental_codec.py:461-469); the quantizer's
    codebook_dim and the layer count are this library's defaults."""

    codebook_size: int = 2048
    num_quantizers: int = 16
    semantic_quantizers: int = 1
    codebook_dim: int = 512
    latent_dim: int = 1024
    hidden_size: int = 512
    num_hidden_layers: int = 8
    num_attention_heads: int = 16
    num_key_value_heads: int = 16
    head_dim: int = 64
    intermediate_size: int = 1024
    sliding_window: int = 72
    rms_norm_eps: float = 1e-5
    rope_theta: float = 10000.0
    layer_scale_initial_scale: float = 0.01
    pre_conv_kernel: int = 3
    decoder_dim: int = 1536
    upsample_rates: tuple[int, ...] = (8, 5, 4, 3)
    upsampling_ratios: tuple[int, ...] = (2, 2)
    sample_rate: int = 24000
    kernel_size: int = 7
    dilations: tuple[int, ...] = (1, 3, 9)
    transconv_trim: str = "right"
    final_activation: str = "clamp"
    conv_gain: float = 0.85
    input_conv_gain: float = 0.08

    @property
    def hop_length(self) -> int:
        return int(math.prod(self.upsample_rates) * math.prod(self.upsampling_ratios))

    @property
    def channels(self) -> int:
        return self.decoder_dim

    @property
    def rates(self) -> tuple[int, ...]:
        return self.upsample_rates

    def stage_channels(self) -> list[int]:
        return [self.decoder_dim // 2**i for i in range(len(self.upsample_rates) + 1)]


# The workloads' architectures.
SINGLE_BLOCK = dict(n_codebooks=8, codebook_size=1024, latent_dim=256)  # RVQ + one conv block
CODEC_24K = DacDecoderConfig()  # 16 x 2048 x 512 tables, 1536 ch, x1920 to 24 kHz
CODEC_24K_LONG = DacDecoderConfig(n_codebooks=32, codebook_size=1024)  # fp8-weight long form
HIFIGAN_24K = HifiGanConfig()
QWEN3_CODE2WAV = Qwen3Code2WavConfig()
QWEN3_TTS_CODEC = Qwen3TTSCodecConfig()


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


def make_qwen3_code2wav_weights(config: Qwen3Code2WavConfig | Qwen3TTSCodecConfig,
                                seed: int = 0, *,
                                branch_scale: float | None = None,
                                activation_spread: float = 0.0) -> dict[str, torch.Tensor]:
    """Seeded float32 weights under ``Qwen3OmniMoeCode2Wav.state_dict()`` names (a checkpoint's
    code2wav weights load the same way); for a Qwen3TTSCodecConfig also the split quantizer
    (``quantizer.codebooks`` [K, V, codebook_dim], ``quantizer.semantic_proj`` /
    ``acoustic_proj`` [latent, codebook_dim]), ``pre_conv`` and the transformer's
    ``input_proj`` / ``output_proj``. Linear and conv weights kaiming-normal (fan_in), biases
    zero, norms one. ``branch_scale`` replaces the layer scales (default 0.01) and ConvNeXt
    gammas (default 1e-6) so the transformer and ConvNeXt branches matter to the output;
    ``activation_spread`` draws the SnakeBeta log-parameters from N(0, spread) instead of 0."""
    gen = torch.Generator().manual_seed(seed)
    c, inter = config.hidden_size, config.intermediate_size
    kv = config.num_key_value_heads * config.head_dim
    qw = config.num_attention_heads * config.head_dim
    latent = getattr(config, "latent_dim", c)
    tts = hasattr(config, "semantic_quantizers")

    def lin(out_f: int, in_f: int, gain: float = 1.0) -> torch.Tensor:
        return _kaiming((out_f, in_f), in_f, gain, gen)

    layer_scale = config.layer_scale_initial_scale if branch_scale is None else branch_scale
    gamma = 1e-6 if branch_scale is None else branch_scale
    w: dict[str, torch.Tensor] = {}
    if tts:
        dq = config.codebook_dim
        w["quantizer.codebooks"] = torch.randn(config.num_quantizers, config.codebook_size, dq,
                                               generator=gen)
        w["quantizer.semantic_proj.weight"] = lin(latent, dq)
        w["quantizer.acoustic_proj.weight"] = lin(latent, dq)
        k = config.pre_conv_kernel
        w["pre_conv.conv.weight"] = _kaiming((latent, latent, k), latent * k, 1.0, gen)
        w["pre_conv.conv.bias"] = torch.zeros(latent)
        w["pre_transformer.input_proj.weight"] = lin(c, latent)
        w["pre_transformer.input_proj.bias"] = torch.zeros(c)
        w["pre_transformer.output_proj.weight"] = lin(latent, c)
        w["pre_transformer.output_proj.bias"] = torch.zeros(latent)
    else:
        w["code_embedding.weight"] = torch.randn(config.num_quantizers * config.codebook_size, c,
                                                 generator=gen)
    for i in range(config.num_hidden_layers):
        p = f"pre_transformer.layers.{i}"
        w[f"{p}.self_attn.q_proj.weight"] = lin(qw, c)
        w[f"{p}.self_attn.k_proj.weight"] = lin(kv, c)
        w[f"{p}.self_attn.v_proj.weight"] = lin(kv, c)
        w[f"{p}.self_attn.o_proj.weight"] = lin(c, qw)
        w[f"{p}.mlp.gate_proj.weight"] = lin(inter, c)
        w[f"{p}.mlp.up_proj.weight"] = lin(inter, c)
        w[f"{p}.mlp.down_proj.weight"] = lin(c, inter)
        w[f"{p}.input_layernorm.weight"] = torch.ones(c)
        w[f"{p}.post_attention_layernorm.weight"] = torch.ones(c)
        w[f"{p}.self_attn_layer_scale.scale"] = torch.full((c,), layer_scale)
        w[f"{p}.mlp_layer_scale.scale"] = torch.full((c,), layer_scale)
    w["pre_transformer.norm.weight"] = torch.ones(c)
    u = latent  # the upsamplers run at the transformer's output width
    for i, factor in enumerate(config.upsampling_ratios):
        w[f"upsample.{i}.0.conv.weight"] = _kaiming((u, u, factor), u * factor, 1.0, gen)
        w[f"upsample.{i}.0.conv.bias"] = torch.zeros(u)
        p = f"upsample.{i}.1"
        w[f"{p}.dwconv.conv.weight"] = _kaiming((u, 1, 7), 7, 1.0, gen)
        w[f"{p}.dwconv.conv.bias"] = torch.zeros(u)
        w[f"{p}.norm.weight"] = torch.ones(u)
        w[f"{p}.norm.bias"] = torch.zeros(u)
        w[f"{p}.pwconv1.weight"] = lin(4 * u, u)
        w[f"{p}.pwconv1.bias"] = torch.zeros(4 * u)
        w[f"{p}.pwconv2.weight"] = lin(u, 4 * u)
        w[f"{p}.pwconv2.bias"] = torch.zeros(u)
        w[f"{p}.gamma"] = torch.full((u,), gamma)

    def snake(prefix: str, ch: int) -> None:
        for name in ("alpha", "beta"):
            w[f"{prefix}.{name}"] = (torch.randn(ch, generator=gen) * activation_spread
                                     if activation_spread else torch.zeros(ch))

    g = config.conv_gain
    chans = config.stage_channels()
    k = config.kernel_size
    w["decoder.0.conv.weight"] = _kaiming((chans[0], u, k), u * k, config.input_conv_gain, gen)
    w["decoder.0.conv.bias"] = torch.zeros(chans[0])
    for bi, rate in enumerate(config.upsample_rates, start=1):
        p = f"decoder.{bi}.block"
        c_in, c_out = chans[bi - 1], chans[bi]
        snake(f"{p}.0", c_in)
        w[f"{p}.1.conv.weight"] = _kaiming((c_in, c_out, 2 * rate), c_out * 2 * rate, g, gen)
        w[f"{p}.1.conv.bias"] = torch.zeros(c_out)
        for u in range(len(config.dilations)):
            q = f"{p}.{u + 2}"
            snake(f"{q}.act1", c_out)
            w[f"{q}.conv1.conv.weight"] = _kaiming((c_out, c_out, k), c_out * k, g, gen)
            w[f"{q}.conv1.conv.bias"] = torch.zeros(c_out)
            snake(f"{q}.act2", c_out)
            w[f"{q}.conv2.conv.weight"] = _kaiming((c_out, c_out, 1), c_out, g, gen)
            w[f"{q}.conv2.conv.bias"] = torch.zeros(c_out)
    n = len(config.upsample_rates)
    snake(f"decoder.{n + 1}", chans[-1])
    w[f"decoder.{n + 2}.conv.weight"] = _kaiming((1, chans[-1], k), chans[-1] * k, g, gen)
    w[f"decoder.{n + 2}.conv.bias"] = torch.zeros(1)
    return w


def qwen3_code2wav_macs_per_frame(config: Qwen3Code2WavConfig | Qwen3TTSCodecConfig) -> int:
    """Multiply-accumulates per code frame: the pre-transformer's projections and attention
    (at most a full window of keys per query), the ConvNeXt upsamplers and the decoder convs."""
    c, inter, hd = config.hidden_size, config.intermediate_size, config.head_dim
    kv = config.num_key_value_heads * hd
    qw = config.num_attention_heads * hd
    u = getattr(config, "latent_dim", c)
    per_token = c * (qw + 2 * kv) + qw * c + 3 * c * inter
    per_token += 2 * qw * config.sliding_window
    macs = config.num_hidden_layers * per_token
    if hasattr(config, "semantic_quantizers"):  # pre_conv, input_proj, output_proj
        macs += u * u * config.pre_conv_kernel + 2 * u * c
    positions = 1
    for factor in config.upsampling_ratios:
        macs += positions * u * u * factor  # transposed conv k = s
        positions *= factor
        macs += positions * (7 * u + 2 * 4 * u * u)
    chans = config.stage_channels()
    k = config.kernel_size
    macs += positions * chans[0] * u * k
    for i, s in enumerate(config.upsample_rates):
        c_in, c_out = chans[i], chans[i + 1]
        macs += positions * c_in * c_out * 2 * s
        positions *= s
        macs += positions * len(config.dilations) * (c_out * c_out * k + c_out * c_out)
    macs += positions * chans[-1] * k
    return macs


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
