"""CPU oracle for the Qwen3-Omni code2wav decoder: a float32 PyTorch restatement of its forward.

TEST INFRASTRUCTURE ONLY. Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline``
leg of ``bench.py`` may import this module, and only to check results against it. The product
path never routes through it.

It restates ``Qwen3OmniMoeCode2Wav`` (``TF/models/qwen3_omni_moe/modeling_qwen3_omni_moe.py``,
the transformers module the reference's ``sglang_omni/models/qwen3_omni/components/code2wav.py``
subclasses) on channels-first ``[B, C, T]`` tensors, reading the weights by the module's own
``state_dict`` names (``pre_transformer.layers.{i}.self_attn.q_proj.weight`` ...), so a real
checkpoint's code2wav weights load unchanged. ``cfg`` is anything with the config's attribute
names (``hidden_size``, ``num_attention_heads``, ``sliding_window``, ``rms_norm_eps``,
``rope_theta``, ``upsample_rates``, ``upsampling_ratios``, ``num_quantizers``,
``codebook_size``).

Parity pins (``tests/test_qwen3_code2wav_oracle.py``):

* the whole decode against the installed ``transformers`` ``Qwen3OmniMoeCode2Wav`` (eager
  attention) on small random configurations, with the window shorter and longer than the input;
* ``window_attention`` against a brute-force per-query softmax loop in float64, and against
  full causal attention when the window covers the input;
* ``apply_rope`` against the complex-rotation form of rotary embeddings (pairs (i, i + d/2));
* ``first_decode_samples`` against the length of the transformers module's output.
* ``qwen3_tts_decode`` (the Qwen3-TTS tokenizer decoder; its module, ``qwen_tts``, is not
  installed): the whole composition, run with the layer kinds of the reference test's pure-torch
  stand-in decoder injected (``DecoderPieces``), equals that stand-in
  (tests/unit_test/qwen3_tts/test_incremental_codec.py:68-306, restated in
  ``tests/test_qwen3_tts_decode_pin.py``) to 1e-12 in float64, and a dropped pre_conv,
  output_proj or final norm, misordered upsamplers, a missing clamp, rotary or window each fail
  that pin; its transformer with identity input / output projections equals
  ``code2wav_transformer``; ``split_rvq_decode`` against a per-frame loop; right-trimmed
  transposed convs against the reference test's own module form (:93-110); T * hop samples.

The reference's streaming semantics (sglang_omni/models/qwen3_omni/components/
incremental_codec.py:109-200: a stream decoded in any split of chunks gives the whole decode's
samples) need no second oracle: the GPU tests check the streamed decode against the whole one.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Any, Callable

import torch
import torch.nn.functional as F

TF_FILE = "TF/models/qwen3_omni_moe/modeling_qwen3_omni_moe.py"


def _f(t: torch.Tensor) -> torch.Tensor:
    """The oracle's working precision: float32, or float64 for float64 inputs and weights (the
    pins that compare compositions run it in float64)."""
    return t if t.dtype == torch.float64 else t.float()


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """x / sqrt(mean(x^2) + eps) * weight over the last dimension (TF :3356-3373)."""
    xf = _f(x)
    return _f(weight) * (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps))


def rope_cos_sin(positions: torch.Tensor, head_dim: int, theta: float) -> tuple[torch.Tensor, torch.Tensor]:
    """Default rotary tables (TF :2405-2440): inv_freq = theta^(-2i/d), angle = p * inv_freq,
    duplicated over both halves; float32."""
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))
    freqs = positions.float()[:, None] * inv_freq[None, :]
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos(), emb.sin()


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """x * cos + rotate_half(x) * sin over the head dimension, rotate_half(x) = (-x2, x1)
    (TF :860-864, :1400-1425); x [..., T, head_dim], cos / sin [T, head_dim]."""
    half = x.shape[-1] // 2
    rotated = torch.cat((-x[..., half:], x[..., :half]), dim=-1)
    return x * cos + rotated * sin


def window_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, window: int,
                     scale: float, q_offset: int = 0) -> torch.Tensor:
    """Causal sliding-window softmax attention of q [B, H, Tq, d] over k / v [B, H, Tk, d]:
    query i (absolute position q_offset + i) sees keys j with 0 <= (q_offset + i) - j < window
    (TF's sliding-window causal mask, the reference's window_mask at code2wav.py:143-147,185-201)."""
    tq, tk = q.shape[2], k.shape[2]
    qpos = torch.arange(tq)[:, None] + q_offset
    kpos = torch.arange(tk)[None, :]
    allowed = (kpos <= qpos) & (qpos - kpos < window)
    scores = torch.matmul(_f(q), _f(k).transpose(-1, -2).contiguous()) * scale
    scores = scores.masked_fill(~allowed, float("-inf"))
    return torch.matmul(torch.softmax(scores, dim=-1), _f(v))


def swiglu_mlp(x: torch.Tensor, w: dict[str, torch.Tensor], prefix: str) -> torch.Tensor:
    """down(silu(gate(x)) * up(x)), no biases (TF :3380-3388)."""
    gate = F.linear(x, _f(w[f"{prefix}.gate_proj.weight"]))
    up = F.linear(x, _f(w[f"{prefix}.up_proj.weight"]))
    return F.linear(F.silu(gate) * up, _f(w[f"{prefix}.down_proj.weight"]))


@dataclass(frozen=True)
class DecoderPieces:
    """The layer kinds the code2wav / Qwen3-TTS decoder compositions below are built from, each
    a function of the weights under its module's state name. The defaults are the real decoders'
    (RMSNorm, SwiGLU, LayerScale, default rotary, SnakeBeta, ConvNeXt LayerNorm eps 1e-6, clamp
    to [-1, 1]); a test swaps in other kinds (LayerNorm, a GELU MLP, tanh ...) to hold the same
    composition against another module that composes those kinds the same way.

    * ``norm(h, w, prefix, cfg)``: the norms ``...input_layernorm``, ``...post_attention_
      layernorm`` and ``pre_transformer.norm``;
    * ``mlp(h, w, prefix)``: ``...mlp``;
    * ``layer_scale(a, w, prefix)``: ``...self_attn_layer_scale`` / ``...mlp_layer_scale``;
    * ``rope(positions, head_dim, cfg)``: the (cos, sin) tables;
    * ``act(x, w, prefix)``: every activation of the conv stack (``decoder.{i}.block.0``,
      ``...act1``, ``...act2``, ``decoder.{n+1}``), x [B, C, L];
    * ``quantize(codes, w, cfg)``: the Qwen3-TTS codes -> latents [B, latent, T];
    * ``convnext_eps``: the ConvNeXt blocks' LayerNorm epsilon;
    * ``clamp(x)``: the waveform's final nonlinearity.
    """

    norm: Callable[..., torch.Tensor] = lambda h, w, prefix, cfg: rms_norm(
        h, w[f"{prefix}.weight"], cfg.rms_norm_eps)
    mlp: Callable[..., torch.Tensor] = swiglu_mlp
    layer_scale: Callable[..., torch.Tensor] = lambda a, w, prefix: _f(w[f"{prefix}.scale"]) * a
    rope: Callable[..., tuple[torch.Tensor, torch.Tensor]] = lambda positions, hd, cfg: rope_cos_sin(
        positions, hd, cfg.rope_theta)
    act: Callable[..., torch.Tensor] = lambda x, w, prefix: snake_beta(
        x, w[f"{prefix}.alpha"], w[f"{prefix}.beta"])
    quantize: Callable[..., torch.Tensor] = lambda codes, w, cfg: split_rvq_decode(
        codes, w, cfg).transpose(1, 2)
    convnext_eps: float = 1e-6
    clamp: Callable[[torch.Tensor], torch.Tensor] = lambda x: x.clamp(-1.0, 1.0)


def transformer_layer(h: torch.Tensor, w: dict[str, torch.Tensor], prefix: str, cfg: Any,
                      cos: torch.Tensor, sin: torch.Tensor,
                      pieces: "DecoderPieces | None" = None) -> torch.Tensor:
    """One pre-transformer layer on h [B, T, C] (TF :3391-3451): RMSNorm -> q/k/v -> rotary ->
    window attention -> o -> layer scale + residual; RMSNorm -> SwiGLU MLP -> layer scale +
    residual."""
    pieces = pieces or DecoderPieces()
    b, t, c = h.shape
    heads = cfg.num_attention_heads
    kv_heads = cfg.num_key_value_heads
    hd = getattr(cfg, "head_dim", c // heads)
    x = pieces.norm(h, w, f"{prefix}.input_layernorm", cfg)
    q = F.linear(x, _f(w[f"{prefix}.self_attn.q_proj.weight"])).view(b, t, heads, hd)
    k = F.linear(x, _f(w[f"{prefix}.self_attn.k_proj.weight"])).view(b, t, kv_heads, hd)
    v = F.linear(x, _f(w[f"{prefix}.self_attn.v_proj.weight"])).view(b, t, kv_heads, hd)
    q = apply_rope(q.transpose(1, 2), cos, sin)
    k = apply_rope(k.transpose(1, 2), cos, sin)
    v = v.transpose(1, 2)
    if kv_heads != heads:
        k = k.repeat_interleave(heads // kv_heads, dim=1)
        v = v.repeat_interleave(heads // kv_heads, dim=1)
    a = window_attention(q, k, v, cfg.sliding_window, hd ** -0.5)
    a = F.linear(a.transpose(1, 2).reshape(b, t, heads * hd),
                 _f(w[f"{prefix}.self_attn.o_proj.weight"]))
    h = h + pieces.layer_scale(a, w, f"{prefix}.self_attn_layer_scale")
    x = pieces.norm(h, w, f"{prefix}.post_attention_layernorm", cfg)
    m = pieces.mlp(x, w, f"{prefix}.mlp")
    return h + pieces.layer_scale(m, w, f"{prefix}.mlp_layer_scale")


def code2wav_transformer(h: torch.Tensor, w: dict[str, torch.Tensor], cfg: Any,
                         pieces: "DecoderPieces | None" = None) -> torch.Tensor:
    """The pre-transformer on inputs_embeds [B, T, C] at positions 0..T-1 (TF :3484-3539):
    its layers, then the final norm."""
    pieces = pieces or DecoderPieces()
    hd = getattr(cfg, "head_dim", cfg.hidden_size // cfg.num_attention_heads)
    cos, sin = pieces.rope(torch.arange(h.shape[1]), hd, cfg)
    for i in range(cfg.num_hidden_layers):
        h = transformer_layer(h, w, f"pre_transformer.layers.{i}", cfg, cos, sin, pieces)
    return pieces.norm(h, w, "pre_transformer.norm", cfg)


def causal_conv(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None, *,
                dilation: int = 1, groups: int = 1) -> torch.Tensor:
    """Qwen3OmniMoeCausalConvNet at stride 1 (TF :3180-3213): (k-1)*d zeros on the left, none
    on the right (the extra padding is 0 at stride 1)."""
    k = weight.shape[-1]
    xp = F.pad(_f(x), ((k - 1) * dilation, 0))
    return F.conv1d(xp, _f(weight), None if bias is None else _f(bias),
                    dilation=dilation, groups=groups)


def causal_trans_conv(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor,
                      stride: int, trim: str = "both") -> torch.Tensor:
    """Qwen3OmniMoeCausalTransConvNet (TF :3216-3228): ConvTranspose1d, then k - s samples
    trimmed on both sides; with trim "right" the Qwen3-TTS tokenizer's form, k - s trimmed on the
    right only (right_pad, qwen3_tts/incremental_codec.py:191-237 emits T * s samples)."""
    y = F.conv_transpose1d(_f(x), _f(weight), _f(bias), stride=stride)
    pad = weight.shape[-1] - stride
    if trim == "right":
        return y[..., :y.shape[-1] - pad]
    return y[..., pad:y.shape[-1] - pad]


def convnext_block(x: torch.Tensor, w: dict[str, torch.Tensor], prefix: str,
                   eps: float = 1e-6) -> torch.Tensor:
    """Qwen3OmniMoeConvNeXtBlock (TF :3231-3264) on [B, C, L]: depthwise causal conv k7 ->
    LayerNorm(eps, 1e-6 in the real decoders) -> Linear 4C -> GELU (erf) -> Linear C -> gamma
    -> + input."""
    c = x.shape[1]
    y = causal_conv(x, w[f"{prefix}.dwconv.conv.weight"], w[f"{prefix}.dwconv.conv.bias"],
                    groups=c)
    y = F.layer_norm(y.transpose(1, 2), (c,), _f(w[f"{prefix}.norm.weight"]),
                     _f(w[f"{prefix}.norm.bias"]), eps=eps)
    y = F.linear(y, _f(w[f"{prefix}.pwconv1.weight"]), _f(w[f"{prefix}.pwconv1.bias"]))
    y = F.gelu(y)
    y = F.linear(y, _f(w[f"{prefix}.pwconv2.weight"]), _f(w[f"{prefix}.pwconv2.bias"]))
    y = _f(w[f"{prefix}.gamma"]) * y
    return _f(x) + y.transpose(1, 2)


def snake_beta(x: torch.Tensor, alpha: torch.Tensor, beta: torch.Tensor) -> torch.Tensor:
    """x + (exp(beta) + 1e-9)^-1 * sin(exp(alpha) * x)^2 per channel (TF :3566-3581)."""
    a = torch.exp(_f(alpha)).view(1, -1, 1)
    inv_b = 1.0 / (torch.exp(_f(beta)).view(1, -1, 1) + 1e-9)
    return x + inv_b * torch.sin(x * a).pow(2)


def code2wav_upsample(x: torch.Tensor, w: dict[str, torch.Tensor], cfg: Any,
                      pieces: "DecoderPieces | None" = None) -> torch.Tensor:
    """The upsamplers on x [B, C, T] (TF :3677-3679): per ratio, a causal transposed conv
    (stride = kernel = ratio), then a ConvNeXt block."""
    pieces = pieces or DecoderPieces()
    trim = getattr(cfg, "transconv_trim", "both")
    for i, factor in enumerate(cfg.upsampling_ratios):
        x = causal_trans_conv(x, w[f"upsample.{i}.0.conv.weight"], w[f"upsample.{i}.0.conv.bias"],
                              factor, trim)
        x = convnext_block(x, w, f"upsample.{i}.1", pieces.convnext_eps)
    return x


def code2wav_decoder(x: torch.Tensor, w: dict[str, torch.Tensor], cfg: Any,
                     pieces: "DecoderPieces | None" = None) -> torch.Tensor:
    """The decoder (TF :3680-3684) on x [B, C, L], before the clamp: conv k7, then per block an
    activation -> causal transposed conv -> residual units (act -> conv k7 dilation 1/3/9 ->
    act -> conv k1, + input), then an activation -> conv to one channel."""
    pieces = pieces or DecoderPieces()
    trim = getattr(cfg, "transconv_trim", "both")
    x = causal_conv(x, w["decoder.0.conv.weight"], w["decoder.0.conv.bias"])
    for bi, rate in enumerate(cfg.upsample_rates, start=1):
        p = f"decoder.{bi}.block"
        x = pieces.act(x, w, f"{p}.0")
        x = causal_trans_conv(x, w[f"{p}.1.conv.weight"], w[f"{p}.1.conv.bias"], rate, trim)
        for u, d in enumerate((1, 3, 9)):
            q = f"{p}.{u + 2}"
            y = pieces.act(x, w, f"{q}.act1")
            y = causal_conv(y, w[f"{q}.conv1.conv.weight"], w[f"{q}.conv1.conv.bias"], dilation=d)
            y = pieces.act(y, w, f"{q}.act2")
            y = causal_conv(y, w[f"{q}.conv2.conv.weight"], w[f"{q}.conv2.conv.bias"])
            x = x + y
    n = len(cfg.upsample_rates)
    x = pieces.act(x, w, f"decoder.{n + 1}")
    return causal_conv(x, w[f"decoder.{n + 2}.conv.weight"], w[f"decoder.{n + 2}.conv.bias"])


def code2wav_conv_stack(h: torch.Tensor, w: dict[str, torch.Tensor], cfg: Any,
                        pieces: "DecoderPieces | None" = None) -> torch.Tensor:
    """Everything after the pre-transformer (TF :3677-3684) on h [B, T, C]: the ConvNeXt
    upsamplers, the decoder blocks (SnakeBeta -> causal transposed conv -> residual units of
    SnakeBeta -> conv k7 dilation 1/3/9 -> SnakeBeta -> conv k1, + input), the final SnakeBeta
    -> conv to one channel, clamp to [-1, 1]. Returns [B, 1, samples]."""
    pieces = pieces or DecoderPieces()
    x = code2wav_upsample(_f(h).transpose(1, 2), w, cfg, pieces)
    return pieces.clamp(code2wav_decoder(x, w, cfg, pieces))


def code_embedding_mean(codes: torch.Tensor, w: dict[str, torch.Tensor], cfg: Any) -> torch.Tensor:
    """code_embedding(codes + q * codebook_size).mean(1) (TF :3675): [B, Q, T] -> [B, T, C]."""
    offset = torch.arange(cfg.num_quantizers).view(1, -1, 1) * cfg.codebook_size
    return F.embedding(codes + offset, _f(w["code_embedding.weight"])).mean(1)


def qwen3_code2wav(codes: torch.Tensor, w: dict[str, torch.Tensor], cfg: Any) -> torch.Tensor:
    """Qwen3OmniMoeCode2Wav.forward (TF :3672-3684): [B, Q, T] codes -> [B, 1, samples]."""
    if codes.shape[1] != cfg.num_quantizers:
        raise ValueError(f"Expected {cfg.num_quantizers} layer of codes, got {codes.shape[1]}")
    h = code2wav_transformer(code_embedding_mean(codes, w, cfg), w, cfg)
    return code2wav_conv_stack(h, w, cfg)


def split_rvq_decode(codes: torch.Tensor, w: dict[str, torch.Tensor], cfg: Any) -> torch.Tensor:
    """The Qwen3-TTS split quantizer's dequantize as the decoder here lays it out: the semantic
    codebooks' embeddings summed and projected, plus the acoustic codebooks' summed and
    projected (each group W_g sum_k E_k[code_k]). [B, Q, T] -> [B, T, latent], float64."""
    books = w["quantizer.codebooks"].double()
    s = cfg.semantic_quantizers
    groups = ((range(0, s), w["quantizer.semantic_proj.weight"]),
              (range(s, cfg.num_quantizers), w["quantizer.acoustic_proj.weight"]))
    out = 0
    for ks, proj in groups:
        summed = sum(books[k][codes[:, k].clamp(max=cfg.codebook_size - 1)] for k in ks)
        out = out + summed @ proj.double().t()
    return out


def tts_pre_conv(z: torch.Tensor, w: dict[str, torch.Tensor]) -> torch.Tensor:
    """The tokenizer decoder's causal ``pre_conv`` on the latents [B, latent, T]."""
    return causal_conv(z, w["pre_conv.conv.weight"], w["pre_conv.conv.bias"])


def tts_transformer(z: torch.Tensor, w: dict[str, torch.Tensor], cfg: Any,
                    pieces: "DecoderPieces | None" = None) -> torch.Tensor:
    """The tokenizer decoder's pre-transformer on z [B, T, latent] (the reference's
    ``incremental_transformer``, qwen3_tts/incremental_codec.py:533-576, over a whole stream):
    input_proj -> layers -> norm -> output_proj. Returns [B, T, latent]."""
    h = F.linear(z, _f(w["pre_transformer.input_proj.weight"]),
                 _f(w["pre_transformer.input_proj.bias"]))
    h = code2wav_transformer(h, w, cfg, pieces)
    return F.linear(h, _f(w["pre_transformer.output_proj.weight"]),
                    _f(w["pre_transformer.output_proj.bias"]))


def qwen3_tts_decode(codes: torch.Tensor, w: dict[str, torch.Tensor], cfg: Any,
                     pieces: "DecoderPieces | None" = None) -> torch.Tensor:
    """The Qwen3-TTS tokenizer decoder's whole-stream decode as the reference's incremental
    decoder composes it (``frame_tensors`` then ``conv_stack_tensors``, qwen3_tts/
    incremental_codec.py:1151-1276): quantizer decode -> causal pre_conv -> pre-transformer
    (input_proj -> layers -> norm -> output_proj) -> the upsamplers (right-trimmed transposed
    conv -> ConvNeXt) -> the decoder (conv, blocks, activation, conv to one channel) -> clamp.
    [B, Q, T] -> [B, 1, T * hop], in float64 when the weights are float64."""
    pieces = pieces or DecoderPieces()
    dt = torch.float64 if w["pre_conv.conv.weight"].dtype == torch.float64 else torch.float32
    z = tts_pre_conv(pieces.quantize(codes, w, cfg).to(dt), w)
    h = tts_transformer(z.transpose(1, 2), w, cfg, pieces)
    x = code2wav_upsample(h.transpose(1, 2), w, cfg, pieces)
    return pieces.clamp(code2wav_decoder(x, w, cfg, pieces))


def total_upsample(cfg: Any) -> int:
    return int(math.prod(cfg.upsample_rates) * math.prod(cfg.upsampling_ratios))


def first_decode_samples(cfg: Any, frames: int) -> int:
    """Samples of the whole decode of ``frames`` frames: every decoder transposed conv (k = 2s)
    drops s samples; the upsamplers (k = s) drop none."""
    n = frames * int(math.prod(cfg.upsampling_ratios))
    for s in cfg.upsample_rates:
        n = n * s - s
    return n
