"""CPU oracle for the codec/vocoder decode path: a float32 PyTorch restatement of the reference.

TEST INFRASTRUCTURE ONLY. Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline``
leg of ``bench.py`` may import this module, and only to check results against it (or, for the CPU
baseline, as the timed CPU port of the reference path). The product path never routes through it.

Every function follows the reference's op order on channels-first ``[B, C, T]`` float32 tensors
and cites the reference file:line it restates (paths relative to the reference checkout;
``TF/`` is the installed ``transformers`` package, whose DAC/Qwen3-Omni classes the reference
imports or vendors).

Parity pins (what fixes each function independently of this file's own formulas) live in
``tests/test_oracle.py``:

* ``rvq_gather_sum``      — brute-force Python loop on tiny inputs; K=1 equals ``F.embedding``;
                            the mean form equals the sum divided by K; the C restatement
                            ``oracle/rvq_oracle.c`` agrees bit for bit.
* ``snake``/``snake_beta`` — float64 closed form; ``transformers`` ``Snake1d`` (installed);
                            alpha -> 0 limit; x = 0 fixed point.
* ``causal_conv1d``       — float64 brute-force direct summation; split invariance.
* ``causal_conv_transpose1d`` — brute-force scatter in float64; streaming split invariance with
                            the reference's overlap-exchange restatement.
* decoder composition     — ``dac_decoder(padding="same")`` against ``transformers``
                            ``DacDecoder`` (the un-vendored dac library's decoder restated:
                            conv -> blocks -> Snake -> conv -> tanh) loaded with the same random
                            weights; the causal mode shares every line but the pad / trim rules,
                            which the causal conv pins fix; mutations of the reference module
                            (no final Snake, no tanh, units reordered, no block Snake) fail.
* ``history_exchange_reference`` / ``overlap_exchange_reference`` — the reference's own
                            pure-torch reference functions (tests/unit_test/kernels/
                            test_codec_state.py:17-49), pinned by the whole-stream invariants of
                            the same test file (:52-130).
* ``stft_reference`` / ``istft_reference`` / ``hift_istft_tail`` — torch.stft / torch.istft
                            (the library routines HiFT calls, hift.py:209-247) in float64; the
                            round trip istft(stft(x)) = x (Hann window at hop n_fft / 4 sums to a
                            constant); the DC and Nyquist bins of a constant / alternating signal;
                            ``hann_window`` against scipy's get_window.
* ``channel_embedding_sum`` — one channel is a plain lookup; float32 tables give the
                            sequential float32 sum of ``rvq_gather_sum`` bit for bit; a bf16
                            two-channel sum is the rounded float32 sum; out-of-range ids add 0.
* ``pcm16_encode``        — known answers of the clip / scale / truncate encoding (full scale,
                            half scale, just below one step, out-of-range and NaN samples) and
                            numpy's own float32 -> int16 cast of the same clipped product.
"""

from __future__ import annotations

import math
from typing import Any

import torch
import torch.nn.functional as F

SNAKE_EPS = 1e-9


# --------------------------------------------------------------------------------------------
# a1: RVQ dequantize (gather-and-sum of code embeddings)
# --------------------------------------------------------------------------------------------


def clamp_codes(codes: torch.Tensor, codebook_size: int) -> torch.Tensor:
    """Codes clamped to the last codebook entry, as the DAC quantizer decode does
    (sglang_omni/models/fishaudio_s2_pro/fish_speech/models/dac/rvq.py:374-388)."""
    return torch.clamp(codes, max=codebook_size - 1)


def rvq_gather_sum(
    codes: torch.Tensor, codebooks: torch.Tensor, *, mean: bool = False
) -> torch.Tensor:
    """out[b, :, t] = sum_k E_k[codes[b, k, t]] accumulated k = 0 -> K-1 in float32, starting
    from 0.0, as ``from_codes`` does (TF/models/dac/modeling_dac.py:362-371) and as the sequential
    forms of sglang_omni/models/personaplex/components/mimi.py:275-280 and
    sglang_omni/models/higgs_tts/audio_codec.py:60-78 do. ``mean`` divides the float32 sum by K
    once, the Qwen3-Omni form (sglang_omni/models/qwen3_omni/components/code2wav.py:443).

    codes [B, K, T] integer, codebooks [K, V, D] float32 -> [B, D, T] float32.
    """
    batch, num_codebooks, frames = codes.shape
    assert codebooks.shape[0] == num_codebooks
    total = torch.zeros(batch, frames, codebooks.shape[2], dtype=torch.float32)
    for k in range(num_codebooks):
        total = total + codebooks[k].float()[codes[:, k, :].long()]
    if mean:
        total = total / num_codebooks
    return total.transpose(1, 2).contiguous()


# --------------------------------------------------------------------------------------------
# a4: Snake / SnakeBeta / LeakyReLU
# --------------------------------------------------------------------------------------------


def snake(x: torch.Tensor, alpha: torch.Tensor) -> torch.Tensor:
    """DAC ``Snake1d``: x + (alpha + 1e-9)^-1 * sin(alpha * x)^2 per channel
    (TF/models/dac/modeling_dac.py:86-99; the channels-last Triton form computes the same
    formula in fp32 at sglang_omni/models/fishaudio_drama3/channels_last_decoder.py:58-62)."""
    a = alpha.reshape(1, -1, 1).float()
    return x + (a + SNAKE_EPS).reciprocal() * torch.sin(a * x).pow(2)


def snake_beta(
    x: torch.Tensor, alpha_log: torch.Tensor, beta_log: torch.Tensor
) -> torch.Tensor:
    """SnakeBeta with log-scale parameters: x + (exp(beta) + 1e-9)^-1 * sin(exp(alpha) * x)^2
    (TF/models/qwen3_omni_moe/modeling_qwen3_omni_moe.py:3566-3581; coefficients precomputed once
    at sglang_omni/kernels/bias_snake_beta.py:29-42)."""
    a = torch.exp(alpha_log.reshape(1, -1, 1).float())
    inv_b = 1.0 / (torch.exp(beta_log.reshape(1, -1, 1).float()) + SNAKE_EPS)
    return x + inv_b * torch.sin(x * a).pow(2)


def leaky_relu(x: torch.Tensor, slope: float) -> torch.Tensor:
    """F.leaky_relu as the HiFT generator applies it
    (sglang_omni/models/minicpm_o/components/token2wav/hift.py:262,277)."""
    return F.leaky_relu(x, slope)


# --------------------------------------------------------------------------------------------
# a2 / a3: causal convs
# --------------------------------------------------------------------------------------------


def causal_conv1d(
    x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None, dilation: int = 1
) -> torch.Tensor:
    """``CausalConvNet.forward`` at stride 1: pad (k-1)*d zeros on the left (the extra right
    padding is zero at stride 1), then Conv1d
    (sglang_omni/models/fishaudio_s2_pro/fish_speech/models/dac/modded_dac.py:541-572)."""
    k = weight.shape[-1]
    pad = (k - 1) * dilation
    return F.conv1d(F.pad(x, (pad, 0)), weight, bias, dilation=dilation)


def causal_conv_transpose1d(
    x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None, stride: int
) -> torch.Tensor:
    """``CausalTransConvNet.forward``: ConvTranspose1d, then drop k - s samples on the right
    only, so T inputs give T * s outputs (modded_dac.py:583-600)."""
    k = weight.shape[-1]
    y = F.conv_transpose1d(x, weight, bias, stride=stride)
    trim = k - stride
    return y[..., : y.shape[-1] - trim]


def same_conv1d(
    x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None, dilation: int = 1
) -> torch.Tensor:
    """Non-causal Conv1d with padding (k*d - d)//2, as HiFiGAN's get_padding gives
    (sglang_omni/models/minicpm_o/components/token2wav/hift_layers.py:67-92)."""
    k = weight.shape[-1]
    pad = (k * dilation - dilation) // 2
    return F.conv1d(x, weight, bias, dilation=dilation, padding=pad)


def padded_conv_transpose1d(
    x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None, stride: int
) -> torch.Tensor:
    """HiFT upsampling ConvTranspose1d with padding (k - u)//2
    (sglang_omni/models/minicpm_o/components/token2wav/hift.py:143-156)."""
    k = weight.shape[-1]
    return F.conv_transpose1d(x, weight, bias, stride=stride, padding=(k - stride) // 2)


# --------------------------------------------------------------------------------------------
# a5 / a6: DAC decoder composition
# --------------------------------------------------------------------------------------------


def _conv(x: torch.Tensor, conv: dict[str, Any], dilation: int, padding: str) -> torch.Tensor:
    """The decoder's stride-one conv in either padding mode: ``CausalConvNet`` (modded_dac.py:
    541-572) or the non-causal ``WNConv1d`` with padding (k - 1) * d // 2 that the reference's
    non-causal DAC layers (and transformers' ``DacDecoder``) use."""
    if padding == "causal":
        return causal_conv1d(x, conv["weight"], conv["bias"], dilation)
    k = conv["weight"].shape[-1]
    return F.conv1d(x, conv["weight"], conv["bias"], dilation=dilation,
                    padding=(k - 1) * dilation // 2)


def _upsample(x: torch.Tensor, conv: dict[str, Any], stride: int, padding: str) -> torch.Tensor:
    """The block's ConvTranspose1d (k = 2s): ``CausalTransConvNet`` (right trim of k - s,
    modded_dac.py:583-600) or the non-causal ``WNConvTranspose1d`` with padding ceil(s / 2)
    (modded_dac.py:762-770 with causal=False)."""
    if padding == "causal":
        return causal_conv_transpose1d(x, conv["weight"], conv["bias"], stride)
    return F.conv_transpose1d(x, conv["weight"], conv["bias"], stride=stride,
                              padding=math.ceil(stride / 2))


def residual_trim(x: torch.Tensor, length: int, padding: str = "causal") -> torch.Tensor:
    """x cut to the ``length`` samples a residual unit's branch returned (modded_dac.py:633-640):
    with pad = x's length - length > 0, the causal unit keeps x's first ``length`` samples
    (``x[..., :-pad]``) and the non-causal one drops floor(pad / 2) samples on the left and
    ceil(pad / 2) on the right (``x[..., pad // 2 : -pad // 2]``); pad <= 0 keeps x."""
    pad = x.shape[-1] - length
    if pad <= 0:
        return x
    if padding == "causal":
        return x[..., :x.shape[-1] - pad]
    return x[..., pad // 2: x.shape[-1] - (pad - pad // 2)]


def residual_unit(x: torch.Tensor, unit: dict[str, Any], padding: str = "causal") -> torch.Tensor:
    """``ResidualUnit.forward``: x + conv1x1(Snake(conv7_d(Snake(x)))), x cut to the branch's
    length by ``residual_trim`` when the convs return fewer samples (modded_dac.py:619-642; with
    the reference's k = 7 convs both padding modes keep the length, so nothing is cut)."""
    y = snake(x, unit["alpha1"])
    y = _conv(y, unit["conv1"], unit["dilation"], padding)
    y = snake(y, unit["alpha2"])
    y = _conv(y, unit["conv2"], 1, padding)
    return residual_trim(x, y.shape[-1], padding) + y


def decoder_block(x: torch.Tensor, block: dict[str, Any], padding: str = "causal") -> torch.Tensor:
    """``DecoderBlock``: Snake -> ConvTranspose1d(k = 2s) -> residual units with dilations 1, 3, 9
    (modded_dac.py:742-787)."""
    x = snake(x, block["alpha"])
    x = _upsample(x, block["up"], block["stride"], padding)
    for unit in block["units"]:
        x = residual_unit(x, unit, padding)
    return x


def dac_decoder(z: torch.Tensor, weights: dict[str, Any], padding: str = "causal") -> torch.Tensor:
    """``Decoder.forward``: conv k=7 -> decoder blocks -> Snake -> conv to one channel k=7 ->
    tanh (modded_dac.py:790-835). z [B, D, T] -> [B, 1, T * prod(rates)] in the causal mode the
    codec decoders run; ``padding="same"`` is the reference's non-causal variant (causal=False),
    whose odd-stride transposed convs give T * s - 1 samples."""
    if padding not in ("causal", "same"):
        raise ValueError(f"padding is 'causal' or 'same', not {padding!r}")
    x = _conv(z, weights["in_conv"], 1, padding)
    for block in weights["blocks"]:
        x = decoder_block(x, block, padding)
    x = snake(x, weights["final"]["alpha"])
    x = _conv(x, weights["final"]["conv"], 1, padding)
    return torch.tanh(x)


def dac_from_indices(codes: torch.Tensor, weights: dict[str, Any]) -> torch.Tensor:
    """``DAC.from_indices``: quantizer decode (clamped gather-sum) then the decoder
    (modded_dac.py:990-992, rvq.py:374-388)."""
    codebooks = weights["codebooks"]
    z = rvq_gather_sum(clamp_codes(codes, codebooks.shape[1]), codebooks)
    return dac_decoder(z, weights)


def conv_block(
    codes: torch.Tensor,
    codebooks: torch.Tensor,
    weight: torch.Tensor,
    bias: torch.Tensor,
    alpha: torch.Tensor,
) -> tuple[torch.Tensor, torch.Tensor]:
    """The RVQ dequant followed by one causal conv block: x = gather-sum; y = x + Snake(conv(x)),
    the conv -> Snake -> residual-add order of the single-block workload. Returns (x, y)."""
    x = rvq_gather_sum(codes, codebooks)
    y = x + snake(causal_conv1d(x, weight, bias), alpha)
    return x, y


# --------------------------------------------------------------------------------------------
# a7: streaming state, restated from the reference's pure-torch test references
# --------------------------------------------------------------------------------------------


def history_exchange_reference(
    padded: torch.Tensor,
    history_pool: torch.Tensor,
    slot_index: torch.Tensor,
    new_samples: int,
    is_cold: bool,
) -> None:
    """In place: history in front of the new samples (zeros when cold), zeros after them, and the
    last ``history`` samples of history + new saved to the slots
    (tests/unit_test/kernels/test_codec_state.py:17-34; kernels/codec_state.py:150-181)."""
    history = int(history_pool.shape[1])
    if is_cold:
        padded[:, :history].zero_()
    else:
        padded[:, :history].copy_(history_pool.index_select(0, slot_index))
    padded[:, history + new_samples :].zero_()
    history_pool.index_copy_(0, slot_index, padded[:, new_samples : new_samples + history])


def overlap_exchange_reference(
    output: torch.Tensor,
    overlap_pool: torch.Tensor,
    slot_index: torch.Tensor,
    emitted_samples: int,
    is_cold: bool,
) -> None:
    """In place: the slot's overlap added to the front of the output (not when cold), and the
    samples past the emitted ones saved as the slot's overlap
    (tests/unit_test/kernels/test_codec_state.py:37-49; kernels/codec_state.py:184-210)."""
    overlap = int(overlap_pool.shape[1])
    if not is_cold:
        output[:, :overlap] += overlap_pool.index_select(0, slot_index)
    overlap_pool.index_copy_(
        0, slot_index, output[:, emitted_samples : emitted_samples + overlap]
    )


def clamped_single_output_conv(
    padded: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor, length: int
) -> torch.Tensor:
    """(B, 1, length) = clamp(bias + conv over a (B, length + k - 1, C) channels-last activation,
    -1, 1), computed in float64 and rounded once, the expectation of
    tests/unit_test/kernels/test_single_output_conv.py:32-44."""
    y = F.conv1d(padded.double().transpose(1, 2), weight.double(), bias.double())
    return y[..., :length].clamp(-1.0, 1.0)


# --------------------------------------------------------------------------------------------
# cfg4: HiFiGAN mel -> wave body
# --------------------------------------------------------------------------------------------


def hifigan_resblock(x: torch.Tensor, block: dict[str, Any], slope: float) -> torch.Tensor:
    """HiFiGAN ``ResBlock``: for each dilation, x = x + conv2(act(conv1_d(act(x)))), with 'same'
    padding and conv2 at dilation 1 (hift_layers.py:57-110; LeakyReLU(slope) as the activation,
    the classic HiFiGAN choice, where the reference HiFT uses Snake)."""
    for conv1, conv2, dilation in zip(block["convs1"], block["convs2"], block["dilations"]):
        xt = leaky_relu(x, slope)
        xt = same_conv1d(xt, conv1["weight"], conv1["bias"], dilation)
        xt = leaky_relu(xt, slope)
        xt = same_conv1d(xt, conv2["weight"], conv2["bias"], 1)
        x = xt + x
    return x


def hifigan_generator(mel: torch.Tensor, weights: dict[str, Any]) -> torch.Tensor:
    """The HiFT ``decode_body`` layer order up to the output conv
    (sglang_omni/models/minicpm_o/components/token2wav/hift.py:255-281): conv_pre k=7 -> per stage
    LeakyReLU(0.1) -> ConvTranspose1d(padding (k-u)//2) -> mean of the MRF ResBlocks ->
    LeakyReLU(0.01) -> conv_post to one channel k=7 -> tanh. mel [B, 80, T] -> [B, 1, T * prod(u)].
    """
    slope = weights["slope"]
    x = same_conv1d(mel, weights["conv_pre"]["weight"], weights["conv_pre"]["bias"])
    for stage in weights["stages"]:
        x = leaky_relu(x, slope)
        x = padded_conv_transpose1d(x, stage["up"]["weight"], stage["up"]["bias"], stage["rate"])
        xs = None
        for block in stage["resblocks"]:
            y = hifigan_resblock(x, block, slope)
            xs = y if xs is None else xs + y
        x = xs / len(stage["resblocks"])
    x = leaky_relu(x, weights["final_slope"])
    x = same_conv1d(x, weights["conv_post"]["weight"], weights["conv_post"]["bias"])
    return torch.tanh(x)


# --------------------------------------------------------------------------------------------
# a8: fp8 weights (no reference implementation; defined by this library)
# --------------------------------------------------------------------------------------------

FP8_E4M3_MAX = 448.0


def quantize_fp8_per_channel(weight: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-output-channel E4M3 quantization: s[co] = max|W[co]| / 448, q = e4m3(W / s).
    ``weight`` is [C_out, ...]; returns (q float8_e4m3fn, s float32 [C_out])."""
    flat = weight.float().reshape(weight.shape[0], -1)
    scale = flat.abs().amax(dim=1) / FP8_E4M3_MAX
    scale = torch.where(scale > 0, scale, torch.ones_like(scale))
    q = (flat / scale[:, None]).to(torch.float8_e4m3fn)
    return q.reshape(weight.shape), scale


def dequantize_fp8_per_channel(q: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """W_deq[co] = float(q[co]) * s[co]."""
    shape = [-1] + [1] * (q.dim() - 1)
    return q.float() * scale.reshape(shape)


# --------------------------------------------------------------------------------------------
# HiFT's iSTFT tail (the next row after the config-4 body)
# --------------------------------------------------------------------------------------------


def hann_window(n_fft: int) -> torch.Tensor:
    """The periodic Hann window scipy's get_window("hann", n_fft, fftbins=True) returns, as
    float32 (sglang_omni/models/minicpm_o/components/token2wav/hift.py:197-205):
    0.5 - 0.5 cos(2 pi k / n_fft)."""
    k = torch.arange(n_fft, dtype=torch.float64)
    return (0.5 - 0.5 * torch.cos(2 * math.pi * k / n_fft)).float()


def stft_reference(signal: torch.Tensor, window: torch.Tensor, n_fft: int, hop: int) -> torch.Tensor:
    """The centred one-sided STFT of HiFT.stft (hift.py:209-227: torch.stft with win_length =
    n_fft, reflect padding of n_fft / 2) from its definition, in float64: X[r, b, f] =
    sum_k xp[r, f hop + k] w[k] exp(-2 pi i b k / n_fft). Returns (rows, 2 * bins, frames), the
    real parts then the imaginary parts (the layout of hift_kernels.py:304-330)."""
    x = signal.to(torch.float64)
    half = n_fft // 2
    xp = F.pad(x[:, None], (half, half), mode="reflect")[:, 0]
    frames = (xp.shape[1] - n_fft) // hop + 1
    idx = torch.arange(frames)[:, None] * hop + torch.arange(n_fft)[None, :]
    seg = xp[:, idx] * window.to(torch.float64)  # (rows, frames, n_fft)
    bins = n_fft // 2 + 1
    angle = 2 * math.pi / n_fft * torch.outer(torch.arange(bins, dtype=torch.float64),
                                              torch.arange(n_fft, dtype=torch.float64))
    real = torch.einsum("rfk,bk->rbf", seg, torch.cos(angle))
    imag = -torch.einsum("rfk,bk->rbf", seg, torch.sin(angle))
    return torch.cat([real, imag], dim=1)


def istft_reference(real: torch.Tensor, imag: torch.Tensor, window: torch.Tensor, n_fft: int,
                    hop: int) -> torch.Tensor:
    """HiFT.istft's torch.istft (hift.py:229-247, center = True, one-sided, win_length = n_fft)
    from its definition, in float64: each frame's inverse DFT y_f[k] = (1 / n_fft) sum_b c_b
    Re(X[b, f] exp(2 pi i b k / n_fft)) with c_b = 1 for DC and Nyquist and 2 between, windowed
    and overlap-added, divided by the overlap-added squared window, with n_fft / 2 samples
    trimmed at each end: (rows, hop * (frames - 1))."""
    re, im = real.to(torch.float64), imag.to(torch.float64)
    rows, bins, frames = re.shape
    w = window.to(torch.float64)
    angle = 2 * math.pi / n_fft * torch.outer(torch.arange(bins, dtype=torch.float64),
                                              torch.arange(n_fft, dtype=torch.float64))
    c = torch.full((bins, 1), 2.0, dtype=torch.float64)
    c[0] = 1.0
    c[-1] = 1.0
    yf = (torch.einsum("rbf,bk->rfk", re, c * torch.cos(angle))
          - torch.einsum("rbf,bk->rfk", im, c * torch.sin(angle))) / n_fft
    total = n_fft + hop * (frames - 1)
    y = torch.zeros(rows, total, dtype=torch.float64)
    env = torch.zeros(total, dtype=torch.float64)
    for f in range(frames):
        y[:, f * hop:f * hop + n_fft] += yf[:, f] * w
        env[f * hop:f * hop + n_fft] += w * w
    half = n_fft // 2
    return (y / env)[:, half:half + hop * (frames - 1)]


def hift_istft_tail(h: torch.Tensor, window: torch.Tensor, n_fft: int, hop: int, *,
                    magnitude_clip: float = 100.0, audio_limit: float = 0.99) -> torch.Tensor:
    """The tail of HiFT's decode from the last conv's output h (rows, frames, >= 2 * bins
    channels-last): magnitude = exp(h[..., :bins]) clipped above at magnitude_clip, phase =
    sin(h[..., bins:2 bins]), inverse transform, clamp to +-audio_limit
    (sglang_omni/models/fun_cosyvoice3/hift_channels_last.py:117-125,269-276; hift.py:229-251).
    Float64 throughout."""
    bins = n_fft // 2 + 1
    hd = h.to(torch.float64)
    magnitude = torch.clip(torch.exp(hd[..., :bins]), max=magnitude_clip).transpose(1, 2)
    phase = torch.sin(hd[..., bins:2 * bins]).transpose(1, 2)
    y = istft_reference(magnitude * torch.cos(phase), magnitude * torch.sin(phase), window,
                        n_fft, hop)
    return torch.clamp(y, -audio_limit, audio_limit)


def channel_embedding_sum(token_ids: torch.Tensor, weights: list[torch.Tensor]) -> torch.Tensor:
    """MOSS-TTS's multi-channel embedding (sglang_omni/models/moss_tts/channel_embedding.py:13-50):
    sum over channels in order of weights[c][token_ids[:, c]], the running float32 total rounded
    to the tables' dtype after every add; ids outside [0, len(weights[c])) add nothing."""
    dtype = weights[0].dtype
    rows, hidden = token_ids.shape[0], weights[0].shape[1]
    total = torch.zeros(rows, hidden, dtype=torch.float32)
    for c, table in enumerate(weights):
        ids = token_ids[:, c].long()
        ok = (ids >= 0) & (ids < table.shape[0])
        values = torch.zeros(rows, hidden, dtype=torch.float32)
        values[ok] = table[ids[ok]].float()
        total = (total + values).to(dtype).float()
    return total.to(dtype)


# --------------------------------------------------------------------------------------------
# host egress: the waveform's wire encodings
# --------------------------------------------------------------------------------------------


def pcm16_encode(samples: torch.Tensor) -> torch.Tensor:
    """float32 samples -> int16 PCM as the realtime bridge encodes them
    (sglang_omni/serve/realtime/session_bridge.py:86-88): clip to [-1, 1], multiply by 32767 in
    float32, truncate toward zero. NaN (passed through by the clip) encodes as 0, what numpy's
    float32 -> int16 cast gives on x86 and what the device conversion gives."""
    x = samples.to(torch.float32)
    clipped = torch.where(torch.isnan(x), torch.zeros_like(x), torch.clamp(x, -1.0, 1.0))
    return torch.trunc(clipped * torch.tensor(32767.0, dtype=torch.float32)).to(torch.int16)


def waveform_egress_reference(wave: torch.Tensor, row_samples: list[int] | None = None, *,
                              format: str = "f32") -> list[torch.Tensor]:
    """Each row of a (B, 1, samples) or (B, samples) float32 waveform cut to its sample count
    (the reference's ``audio[i, 0, :n * hop]``, sglang_omni/scheduling/audio_vocoder.py:204-217),
    as float32 or as PCM16."""
    rows = wave[:, 0] if wave.dim() == 3 else wave
    counts = [rows.shape[1]] * rows.shape[0] if row_samples is None else list(row_samples)
    out = []
    for r, n in enumerate(counts):
        row = rows[r, :n].to(torch.float32)
        out.append(pcm16_encode(row) if format == "pcm16" else row.clone())
    return out


def snr_db(reference: torch.Tensor, actual: torch.Tensor) -> float:
    """10 log10(sum ref^2 / sum (ref - actual)^2) in float64."""
    ref = reference.double()
    noise = (ref - actual.double()).pow(2).sum().item()
    signal = ref.pow(2).sum().item()
    if noise == 0:
        return math.inf
    return 10.0 * math.log10(signal / noise)
