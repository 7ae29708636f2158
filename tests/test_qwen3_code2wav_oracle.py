"""CPU pins of the Qwen3-Omni code2wav oracle (oracle/qwen3_code2wav_oracle.py): the whole
decode against the installed transformers ``Qwen3OmniMoeCode2Wav`` (the module the reference's
code2wav.py subclasses) on small random configurations, and the attention / rotary pieces
against brute-force and closed forms."""

from __future__ import annotations

import math
from types import SimpleNamespace

import pytest
import torch

from oracle import qwen3_code2wav_oracle as Q

tf_q3 = pytest.importorskip("transformers.models.qwen3_omni_moe.modeling_qwen3_omni_moe")
from transformers.models.qwen3_omni_moe.configuration_qwen3_omni_moe import (  # noqa: E402
    Qwen3OmniMoeCode2WavConfig,
)


def _tiny_config(**kw) -> Qwen3OmniMoeCode2WavConfig:
    base = dict(hidden_size=64, num_hidden_layers=2, num_attention_heads=4, num_key_value_heads=4,
                intermediate_size=96, sliding_window=5, codebook_size=32, num_quantizers=4,
                decoder_dim=64, upsample_rates=[2, 3], upsampling_ratios=[2, 2])
    base.update(kw)
    cfg = Qwen3OmniMoeCode2WavConfig(**base)
    cfg._attn_implementation = "eager"
    return cfg


def _oracle_cfg(cfg) -> SimpleNamespace:
    return SimpleNamespace(
        hidden_size=cfg.hidden_size, num_hidden_layers=cfg.num_hidden_layers,
        num_attention_heads=cfg.num_attention_heads, num_key_value_heads=cfg.num_key_value_heads,
        sliding_window=cfg.sliding_window, rms_norm_eps=cfg.rms_norm_eps,
        rope_theta=cfg.rope_parameters["rope_theta"], upsample_rates=list(cfg.upsample_rates),
        upsampling_ratios=list(cfg.upsampling_ratios), num_quantizers=cfg.num_quantizers,
        codebook_size=cfg.codebook_size)


def _randomized(model: torch.nn.Module, seed: int) -> dict[str, torch.Tensor]:
    """Random values for every parameter, scaled so every branch of the model matters (layer
    scales and ConvNeXt gammas of order one, SnakeBeta parameters away from zero)."""
    g = torch.Generator().manual_seed(seed)
    state = {}
    for name, p in model.state_dict().items():
        if name.endswith(("layer_scale.scale", ".gamma")):
            v = 0.3 + 0.4 * torch.rand(p.shape, generator=g)
        elif name.endswith(("alpha", "beta")):
            v = 0.3 * torch.randn(p.shape, generator=g)
        elif name.endswith(("norm.weight", "layernorm.weight")):
            v = 1.0 + 0.2 * torch.randn(p.shape, generator=g)
        elif name == "code_embedding.weight":
            v = torch.randn(p.shape, generator=g)
        elif p.dim() >= 2:
            fan_in = p.shape[1] * (p.shape[2] if p.dim() == 3 else 1)
            v = torch.randn(p.shape, generator=g) * (0.9 / math.sqrt(fan_in))
        else:
            v = 0.05 * torch.randn(p.shape, generator=g)
        state[name] = v.float()
    model.load_state_dict(state)
    return state


@pytest.mark.parametrize("frames,window,kv_heads", [(9, 5, 4), (4, 5, 4), (12, 40, 2)])
def test_code2wav_matches_transformers(frames, window, kv_heads):
    cfg = _tiny_config(sliding_window=window, num_key_value_heads=kv_heads)
    torch.manual_seed(0)
    model = tf_q3.Qwen3OmniMoeCode2Wav(cfg).eval()
    w = _randomized(model, seed=frames)
    codes = torch.randint(0, cfg.codebook_size, (2, cfg.num_quantizers, frames),
                          generator=torch.Generator().manual_seed(3))
    with torch.no_grad():
        ref = model(codes)
        got = Q.qwen3_code2wav(codes, w, _oracle_cfg(cfg))
    assert got.shape == ref.shape == (2, 1, Q.first_decode_samples(_oracle_cfg(cfg), frames))
    assert ref.abs().max() > 0.05  # the output is not trivially clamped or zero
    torch.testing.assert_close(got, ref, rtol=1e-4, atol=1e-5)


def test_transformer_matches_transformers():
    cfg = _tiny_config(num_hidden_layers=3)
    model = tf_q3.Qwen3OmniMoeCode2Wav(cfg).eval()
    w = _randomized(model, seed=11)
    h = torch.randn(3, 17, cfg.hidden_size, generator=torch.Generator().manual_seed(5))
    with torch.no_grad():
        ref = model.pre_transformer(inputs_embeds=h).last_hidden_state
        got = Q.code2wav_transformer(h, w, _oracle_cfg(cfg))
    torch.testing.assert_close(got, ref, rtol=1e-4, atol=1e-5)


def test_window_attention_brute_force():
    g = torch.Generator().manual_seed(1)
    q = torch.randn(2, 3, 7, 8, generator=g)
    k = torch.randn(2, 3, 11, 8, generator=g)
    v = torch.randn(2, 3, 11, 8, generator=g)
    window, offset, scale = 4, 4, 0.35
    got = Q.window_attention(q, k, v, window, scale, q_offset=offset)
    ref = torch.zeros(2, 3, 7, 8, dtype=torch.float64)
    for b in range(2):
        for h in range(3):
            for i in range(7):
                p = offset + i
                keys = [j for j in range(11) if 0 <= p - j < window]
                s = torch.tensor([float(q[b, h, i].double() @ k[b, h, j].double()) * scale
                                  for j in keys], dtype=torch.float64)
                pr = torch.softmax(s, 0)
                ref[b, h, i] = sum(pr[n] * v[b, h, j].double() for n, j in enumerate(keys))
    torch.testing.assert_close(got.double(), ref, rtol=1e-5, atol=1e-6)
    # a window that covers every key is plain causal attention
    full = Q.window_attention(q, k[:, :, :7], v[:, :, :7], 100, scale)
    causal = torch.nn.functional.scaled_dot_product_attention(q, k[:, :, :7], v[:, :, :7],
                                                              is_causal=True, scale=scale)
    torch.testing.assert_close(full, causal, rtol=1e-5, atol=1e-6)


def test_rope_is_a_complex_rotation():
    """Rotary embedding pairs (i, i + d/2) rotated by p * theta^(-2i/d)."""
    d, theta = 16, 10000.0
    pos = torch.tensor([0, 1, 5, 71, 1234, 65535])
    x = torch.randn(len(pos), d, generator=torch.Generator().manual_seed(2))
    cos, sin = Q.rope_cos_sin(pos, d, theta)
    got = Q.apply_rope(x, cos, sin).double()
    z = torch.complex(x[:, : d // 2].double(), x[:, d // 2:].double())
    inv = theta ** (-torch.arange(0, d, 2, dtype=torch.float64) / d)
    ang = pos.double()[:, None] * inv[None, :]
    r = z * torch.exp(1j * ang)
    ref = torch.cat([r.real, r.imag], dim=-1)
    # float32 angles at large positions: the rotation's error grows with p * ulp
    torch.testing.assert_close(got, ref, rtol=0, atol=2e-2)
    torch.testing.assert_close(got[:4], ref[:4], rtol=0, atol=1e-5)
