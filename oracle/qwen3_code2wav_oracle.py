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
  installed, so the composition is parity unpinned beyond its pieces): its transformer with
  identity input / output projections equals ``code2wav_transformer``; ``split_rvq_decode``
  against a per-frame loop; right-trimmed transposed convs against the reference test's own
  module form (tests/unit_test/qwen3_tts/test_incremental_codec.py:93-110); T * hop samples.

The reference's streaming semantics (sglang_omni/models/qwen3_omni/components/
incremental_codec.py:109-200: a stream decoded in any split of chunks gives the whole decode's
samples) need no second oracle: the GPU tests check the streamed decode against the whole one.
"""

from __future__ import annotations

import math
from typing import Any

import torch
import torch.nn.functional as F

TF_FILE = "TF/models/qwen3_omni_moe/modeling_qwen3_omni_moe.py"


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """x / sqrt(mean(x^2) + eps) * weight over the last dimension (TF :3356-3373)."""
    xf = x.float()
    return weight.float() * (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps))


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
    scores = torch.matmul(q.float(), k.float().transpose(-1, -2).contiguous()) * scale
    scores = scores.masked_fill(~allowed, float("-inf"))
    return torch.matmul(torch.softmax(scores, dim=-1), v.float())


def transformer_layer(h: torch.Tensor, w: dict[str, torch.Tensor], prefix: str, cfg: Any,
                      cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """One pre-transformer layer on h [B, T, C] (TF :3391-3451): RMSNorm -> q/k/v -> rotary ->
    window attention -> o -> layer scale + residual; RMSNorm -> SwiGLU MLP -> layer scale +
    residual."""
    b, t, c = h.shape
    heads = cfg.num_attention_heads
    kv_heads = cfg.num_key_value_heads
    hd = getattr(cfg, "head_dim", c // heads)
    eps = cfg.rms_norm_eps
    x = rms_norm(h, w[f"{prefix}.input_layernorm.weight"], eps)
    q = F.linear(x, w[f"{prefix}.self_attn.q_proj.weight"].float()).view(b, t, heads, hd)
    k = F.linear(x, w[f"{prefix}.self_attn.k_proj.weight"].float()).view(b, t, kv_heads, hd)
    v = F.linear(x, w[f"{prefix}.self_attn.v_proj.weight"].float()).view(b, t, kv_heads, hd)
    q = apply_rope(q.transpose(1, 2), cos, sin)
    k = apply_rope(k.transpose(1, 2), cos, sin)
    v = v.transpose(1, 2)
    if kv_heads != heads:
        k = k.repeat_interleave(heads // kv_heads, dim=1)
        v = v.repeat_interleave(heads // kv_heads, dim=1)
    a = window_attention(q, k, v, cfg.sliding_window, hd ** -0.5)
    a = F.linear(a.transpose(1, 2).reshape(b, t, heads * hd),
                 w[f"{prefix}.self_attn.o_proj.weight"].float())
    h = h + w[f"{prefix}.self_attn_layer_scale.scale"].float() * a
    x = rms_norm(h, w[f"{prefix}.post_attention_layernorm.weight"], eps)
    gate = F.linear(x, w[f"{prefix}.mlp.gate_proj.weight"].float())
    up = F.linear(x, w[f"{prefix}.mlp.up_proj.weight"].float())
    m = F.linear(F.silu(gate) * up, w[f"{prefix}.mlp.down_proj.weight"].float())
    return h + w[f"{prefix}.mlp_layer_scale.scale"].float() * m


def code2wav_transformer(h: torch.Tensor, w: dict[str, torch.Tensor], cfg: Any) -> torch.Tensor:
    """The pre-transformer on inputs_embeds [B, T, C] at positions 0..T-1 (TF :3484-3539)."""
    hd = getattr(cfg, "head_dim", cfg.hidden_size // cfg.num_attention_heads)
    cos, sin = rope_cos_sin(torch.arange(h.shape[1]), hd, cfg.rope_theta)
    for i in range(cfg.num_hidden_layers):
        h = transformer_layer(h, w, f"pre_transformer.layers.{i}", cfg, cos, sin)
    return rms_norm(h, w["pre_transformer.norm.weight"], cfg.rms_norm_eps)


def causal_conv(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None, *,
                dilation: int = 1, groups: int = 1) -> torch.Tensor:
    """Qwen3OmniMoeCausalConvNet at stride 1 (TF :3180-3213): (k-1)*d zeros on the left, none
    on the right (the extra padding is 0 at stride 1)."""
    k = weight.shape[-1]
    xp = F.pad(x.float(), ((k - 1) * dilation, 0))
    return F.conv1d(xp, weight.float(), None if bias is None else bias.float(),
                    dilation=dilation, groups=groups)


def causal_trans_conv(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor,
                      stride: int, trim: str = "both") -> torch.Tensor:
    """Qwen3OmniMoeCausalTransConvNet (TF :3216-3228): ConvTranspose1d, then k - s samples
    trimmed on both sides; with trim "right" the Qwen3-TTS tokenizer's form, k - s trimmed on the
    right only (right_pad, qwen3_tts/incremental_codec.py:191-237 emits T * s samples)."""
    y = F.conv_transpose1d(x.float(), weight.float(), bias.float(), stride=stride)
    pad = weight.shape[-1] - stride
    if trim == "right":
        return y[..., :y.shape[-1] - pad]
    return y[..., pad:y.shape[-1] - pad]


def convnext_block(x: torch.Tensor, w: dict[str, torch.Tensor], prefix: str) -> torch.Tensor:
    """Qwen3OmniMoeConvNeXtBlock (TF :3231-3264) on [B, C, L]: depthwise causal conv k7 ->
    LayerNorm(eps 1e-6) -> Linear 4C -> GELU (erf) -> Linear C -> gamma -> + input."""
    c = x.shape[1]
    y = causal_conv(x, w[f"{prefix}.dwconv.conv.weight"], w[f"{prefix}.dwconv.conv.bias"],
                    groups=c)
    y = F.layer_norm(y.transpose(1, 2), (c,), w[f"{prefix}.norm.weight"].float(),
                     w[f"{prefix}.norm.bias"].float(), eps=1e-6)
    y = F.linear(y, w[f"{prefix}.pwconv1.weight"].float(), w[f"{prefix}.pwconv1.bias"].float())
    y = F.gelu(y)
    y = F.linear(y, w[f"{prefix}.pwconv2.weight"].float(), w[f"{prefix}.pwconv2.bias"].float())
    y = w[f"{prefix}.gamma"].float() * y
    return x.float() + y.transpose(1, 2)


def snake_beta(x: torch.Tensor, alpha: torch.Tensor, beta: torch.Tensor) -> torch.Tensor:
    """x + (exp(beta) + 1e-9)^-1 * sin(exp(alpha) * x)^2 per channel (TF :3566-3581)."""
    a = torch.exp(alpha.float()).view(1, -1, 1)
    inv_b = 1.0 / (torch.exp(beta.float()).view(1, -1, 1) + 1e-9)
    return x + inv_b * torch.sin(x * a).pow(2)


def code2wav_conv_stack(h: torch.Tensor, w: dict[str, torch.Tensor], cfg: Any) -> torch.Tensor:
    """Everything after the pre-transformer (TF :3677-3684) on h [B, T, C]: the ConvNeXt
    upsamplers, the decoder blocks (SnakeBeta -> causal transposed conv -> residual units of
    SnakeBeta -> conv k7 dilation 1/3/9 -> SnakeBeta -> conv k1, + input), the final SnakeBeta
    -> conv to one channel, clamp to [-1, 1]. Returns [B, 1, samples]."""
    trim = getattr(cfg, "transconv_trim", "both")
    x = h.float().transpose(1, 2)
    for i, factor in enumerate(cfg.upsampling_ratios):
        x = causal_trans_conv(x, w[f"upsample.{i}.0.conv.weight"], w[f"upsample.{i}.0.conv.bias"],
                              factor, trim)
        x = convnext_block(x, w, f"upsample.{i}.1")
    x = causal_conv(x, w["decoder.0.conv.weight"], w["decoder.0.conv.bias"])
    for bi, rate in enumerate(cfg.upsample_rates, start=1):
        p = f"decoder.{bi}.block"
        x = snake_beta(x, w[f"{p}.0.alpha"], w[f"{p}.0.beta"])
        x = causal_trans_conv(x, w[f"{p}.1.conv.weight"], w[f"{p}.1.conv.bias"], rate, trim)
        for u, d in enumerate((1, 3, 9)):
            q = f"{p}.{u + 2}"
            y = snake_beta(x, w[f"{q}.act1.alpha"], w[f"{q}.act1.beta"])
            y = causal_conv(y, w[f"{q}.conv1.conv.weight"], w[f"{q}.conv1.conv.bias"], dilation=d)
            y = snake_beta(y, w[f"{q}.act2.alpha"], w[f"{q}.act2.beta"])
            y = causal_conv(y, w[f"{q}.conv2.conv.weight"], w[f"{q}.conv2.conv.bias"])
            x = x + y
    n = len(cfg.upsample_rates)
    x = snake_beta(x, w[f"decoder.{n + 1}.alpha"], w[f"decoder.{n + 1}.beta"])
    x = causal_conv(x, w[f"decoder.{n + 2}.conv.weight"], w[f"decoder.{n + 2}.conv.bias"])
    return x.clamp(-1.0, 1.0)


def code_embedding_mean(codes: torch.Tensor, w: dict[str, torch.Tensor], cfg: Any) -> torch.Tensor:
    """code_embedding(codes + q * codebook_size).mean(1) (TF :3675): [B, Q, T] -> [B, T, C]."""
    offset = torch.arange(cfg.num_quantizers).view(1, -1, 1) * cfg.codebook_size
    return F.embedding(codes + offset, w["code_embedding.weight"].float()).mean(1)


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


def qwen3_tts_decode(codes: torch.Tensor, w: dict[str, torch.Tensor], cfg: Any) -> torch.Tensor:
    """The Qwen3-TTS tokenizer decoder's whole-stream decode as the reference's incremental
    decoder composes it (qwen3_tts/incremental_codec.py:1136-1276): split RVQ -> causal pre_conv
    -> input_proj -> pre-transformer layers -> RMSNorm -> output_proj -> the conv stack with
    right-trimmed transposed convs -> clamp. [B, Q, T] -> [B, 1, T * hop]."""
    z = split_rvq_decode(codes, w, cfg).float().transpose(1, 2)
    z = causal_conv(z, w["pre_conv.conv.weight"], w["pre_conv.conv.bias"]).transpose(1, 2)
    h = F.linear(z, w["pre_transformer.input_proj.weight"].float(),
                 w["pre_transformer.input_proj.bias"].float())
    hd = cfg.head_dim
    cos, sin = rope_cos_sin(torch.arange(h.shape[1]), hd, cfg.rope_theta)
    for i in range(cfg.num_hidden_layers):
        h = transformer_layer(h, w, f"pre_transformer.layers.{i}", cfg, cos, sin)
    h = rms_norm(h, w["pre_transformer.norm.weight"], cfg.rms_norm_eps)
    h = F.linear(h, w["pre_transformer.output_proj.weight"].float(),
                 w["pre_transformer.output_proj.bias"].float())
    return code2wav_conv_stack(h, w, cfg)


def total_upsample(cfg: Any) -> int:
    return int(math.prod(cfg.upsample_rates) * math.prod(cfg.upsampling_ratios))


def first_decode_samples(cfg: Any, frames: int) -> int:
    """Samples of the whole decode of ``frames`` frames: every decoder transposed conv (k = 2s)
    drops s samples; the upsamplers (k = s) drop none."""
    n = frames * int(math.prod(cfg.upsampling_ratios))
    for s in cfg.upsample_rates:
        n = n * s - s
    return n
