"""CPU pins of the Qwen3-Omni code2wav oracle (oracle/qwen3_code2wav_oracle.py): the whole
decode against the installed transformers ``Qwen3OmniMoeCode2Wav`` (the module the reference's
code2wav.py subclasses) on small random configurations, and the attention / rotary pieces
against brute-force and closed forms. The Qwen3-TTS decoder's composition (its module is not
installed) through its pieces: a wider-than-hidden attention against transformers, the split
quantizer against a loop, right-trimmed transposed convs against the module form, causality."""

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


def test_transformer_with_wider_attention_matches_transformers():
    """heads * head_dim != hidden (the Qwen3-TTS decoder's 16 x 64 over 512): the module takes
    head_dim from its config."""
    cfg = _tiny_config(num_hidden_layers=2, head_dim=32, num_key_value_heads=2)
    model = tf_q3.Qwen3OmniMoeCode2Wav(cfg).eval()
    assert model.pre_transformer.layers[0].self_attn.q_proj.out_features == 4 * 32
    w = _randomized(model, seed=13)
    h = torch.randn(2, 11, cfg.hidden_size, generator=torch.Generator().manual_seed(6))
    ocfg = _oracle_cfg(cfg)
    ocfg.head_dim = 32
    with torch.no_grad():
        ref = model.pre_transformer(inputs_embeds=h).last_hidden_state
        got = Q.code2wav_transformer(h, w, ocfg)
    torch.testing.assert_close(got, ref, rtol=1e-4, atol=1e-5)


def _tts_cfg(**kw) -> SimpleNamespace:
    base = dict(hidden_size=64, num_hidden_layers=2, num_attention_heads=2, num_key_value_heads=1,
                head_dim=64, intermediate_size=96, sliding_window=5, rms_norm_eps=1e-5,
                rope_theta=10000.0, codebook_size=32, num_quantizers=4, semantic_quantizers=1,
                codebook_dim=16, latent_dim=48, pre_conv_kernel=3, decoder_dim=64,
                upsample_rates=(2, 3), upsampling_ratios=(2,), transconv_trim="right",
                kernel_size=7, dilations=(1, 3, 9))
    base.update(kw)
    return SimpleNamespace(**base)


def _tts_weights(cfg, seed: int) -> dict[str, torch.Tensor]:
    """Random weights under the decoder's state names, every branch of order one."""
    g = torch.Generator().manual_seed(seed)
    c, lat, hd = cfg.hidden_size, cfg.latent_dim, cfg.head_dim
    q, kv = cfg.num_attention_heads * hd, cfg.num_key_value_heads * hd

    def lin(o, i):
        return torch.randn(o, i, generator=g) / math.sqrt(i)

    w = {"quantizer.codebooks": torch.randn(cfg.num_quantizers, cfg.codebook_size,
                                            cfg.codebook_dim, generator=g),
         "quantizer.semantic_proj.weight": lin(lat, cfg.codebook_dim),
         "quantizer.acoustic_proj.weight": lin(lat, cfg.codebook_dim),
         "pre_conv.conv.weight": torch.randn(lat, lat, 3, generator=g) / math.sqrt(3 * lat),
         "pre_conv.conv.bias": 0.1 * torch.randn(lat, generator=g),
         "pre_transformer.input_proj.weight": lin(c, lat),
         "pre_transformer.input_proj.bias": 0.1 * torch.randn(c, generator=g),
         "pre_transformer.output_proj.weight": lin(lat, c),
         "pre_transformer.output_proj.bias": 0.1 * torch.randn(lat, generator=g),
         "pre_transformer.norm.weight": 1 + 0.1 * torch.randn(c, generator=g)}
    for i in range(cfg.num_hidden_layers):
        p = f"pre_transformer.layers.{i}"
        w.update({f"{p}.self_attn.q_proj.weight": lin(q, c), f"{p}.self_attn.k_proj.weight": lin(kv, c),
                  f"{p}.self_attn.v_proj.weight": lin(kv, c), f"{p}.self_attn.o_proj.weight": lin(c, q),
                  f"{p}.mlp.gate_proj.weight": lin(cfg.intermediate_size, c),
                  f"{p}.mlp.up_proj.weight": lin(cfg.intermediate_size, c),
                  f"{p}.mlp.down_proj.weight": lin(c, cfg.intermediate_size),
                  f"{p}.input_layernorm.weight": torch.ones(c),
                  f"{p}.post_attention_layernorm.weight": torch.ones(c),
                  f"{p}.self_attn_layer_scale.scale": torch.full((c,), 0.5),
                  f"{p}.mlp_layer_scale.scale": torch.full((c,), 0.5)})
    for i, f in enumerate(cfg.upsampling_ratios):
        p = f"upsample.{i}.1"
        w.update({f"upsample.{i}.0.conv.weight": lin(lat, lat * f).view(lat, lat, f),
                  f"upsample.{i}.0.conv.bias": torch.zeros(lat),
                  f"{p}.dwconv.conv.weight": torch.randn(lat, 1, 7, generator=g) / math.sqrt(7),
                  f"{p}.dwconv.conv.bias": torch.zeros(lat), f"{p}.norm.weight": torch.ones(lat),
                  f"{p}.norm.bias": torch.zeros(lat), f"{p}.pwconv1.weight": lin(4 * lat, lat),
                  f"{p}.pwconv1.bias": torch.zeros(4 * lat), f"{p}.pwconv2.weight": lin(lat, 4 * lat),
                  f"{p}.pwconv2.bias": torch.zeros(lat), f"{p}.gamma": torch.full((lat,), 0.5)})
    chans = [cfg.decoder_dim // 2 ** i for i in range(len(cfg.upsample_rates) + 1)]
    w["decoder.0.conv.weight"] = torch.randn(chans[0], lat, 7, generator=g) * 0.03 / math.sqrt(7 * lat)
    w["decoder.0.conv.bias"] = torch.zeros(chans[0])
    for bi, r in enumerate(cfg.upsample_rates, start=1):
        p, ci, co = f"decoder.{bi}.block", chans[bi - 1], chans[bi]
        w[f"{p}.0.alpha"], w[f"{p}.0.beta"] = 0.1 * torch.randn(ci, generator=g), torch.zeros(ci)
        w[f"{p}.1.conv.weight"] = torch.randn(ci, co, 2 * r, generator=g) * 0.8 / math.sqrt(co * 2 * r)
        w[f"{p}.1.conv.bias"] = torch.zeros(co)
        for u in range(3):
            q_ = f"{p}.{u + 2}"
            for a in ("act1", "act2"):
                w[f"{q_}.{a}.alpha"], w[f"{q_}.{a}.beta"] = torch.zeros(co), torch.zeros(co)
            w[f"{q_}.conv1.conv.weight"] = torch.randn(co, co, 7, generator=g) * 0.8 / math.sqrt(7 * co)
            w[f"{q_}.conv1.conv.bias"] = torch.zeros(co)
            w[f"{q_}.conv2.conv.weight"] = torch.randn(co, co, 1, generator=g) * 0.8 / math.sqrt(co)
            w[f"{q_}.conv2.conv.bias"] = torch.zeros(co)
    n = len(cfg.upsample_rates)
    w[f"decoder.{n + 1}.alpha"], w[f"decoder.{n + 1}.beta"] = torch.zeros(chans[-1]), torch.zeros(chans[-1])
    w[f"decoder.{n + 2}.conv.weight"] = torch.randn(1, chans[-1], 7, generator=g) / math.sqrt(7 * chans[-1])
    w[f"decoder.{n + 2}.conv.bias"] = torch.zeros(1)
    return w


def test_split_rvq_decode_brute_force():
    cfg = _tts_cfg()
    w = _tts_weights(cfg, 1)
    codes = torch.randint(0, 40, (2, 4, 6), generator=torch.Generator().manual_seed(2))  # >= V clamps
    got = Q.split_rvq_decode(codes, w, cfg)
    for b in range(2):
        for t in range(6):
            c = [min(int(codes[b, k, t]), 31) for k in range(4)]
            sem = w["quantizer.codebooks"][0, c[0]].double()
            aco = sum(w["quantizer.codebooks"][k, c[k]].double() for k in range(1, 4))
            ref = w["quantizer.semantic_proj.weight"].double() @ sem + \
                w["quantizer.acoustic_proj.weight"].double() @ aco
            torch.testing.assert_close(got[b, t], ref)


def test_right_trimmed_transposed_conv_is_the_module_form():
    """The Qwen3-TTS tokenizer's causal transposed conv: ConvTranspose1d, the last k - s
    samples dropped (the reference test's CausalTransConv)."""
    conv = torch.nn.ConvTranspose1d(6, 4, 10, stride=5)
    x = torch.randn(2, 6, 9)
    with torch.no_grad():
        full = conv(x)
        ref = full[..., :-(10 - 5)]
        got = Q.causal_trans_conv(x, conv.weight, conv.bias, 5, "right")
    assert got.shape[-1] == 9 * 5
    torch.testing.assert_close(got, ref)


def test_tts_decode_is_causal_and_emits_hop_samples_per_frame():
    """Each decode of T frames emits T * hop samples and a prefix of the codes decodes to the
    prefix of the waveform: the whole decode is what the reference's incremental decoder emits
    chunk by chunk (qwen3_tts/incremental_codec.py:1032-1083)."""
    cfg = _tts_cfg()
    w = _tts_weights(cfg, 3)
    hop = 2 * 3 * 2
    codes = torch.randint(0, 32, (2, 4, 13), generator=torch.Generator().manual_seed(4))
    with torch.no_grad():
        whole = Q.qwen3_tts_decode(codes, w, cfg)
        prefix = Q.qwen3_tts_decode(codes[..., :7], w, cfg)
    assert whole.shape == (2, 1, 13 * hop) and prefix.shape == (2, 1, 7 * hop)
    assert whole.abs().max() > 0.02
    torch.testing.assert_close(prefix, whole[..., :7 * hop], rtol=1e-5, atol=1e-6)


def test_tts_transformer_with_identity_projections_is_the_code2wav_transformer():
    cfg = _tts_cfg(latent_dim=64)
    w = _tts_weights(cfg, 5)
    w["pre_transformer.input_proj.weight"] = torch.eye(64)
    w["pre_transformer.input_proj.bias"] = torch.zeros(64)
    w["pre_transformer.output_proj.weight"] = torch.eye(64)
    w["pre_transformer.output_proj.bias"] = torch.zeros(64)
    w["pre_conv.conv.weight"] = torch.zeros(64, 64, 3)
    w["pre_conv.conv.weight"][:, :, 2] = torch.eye(64)
    w["pre_conv.conv.bias"] = torch.zeros(64)
    codes = torch.randint(0, 32, (1, 4, 9), generator=torch.Generator().manual_seed(8))
    with torch.no_grad():
        z = Q.split_rvq_decode(codes, w, cfg).float()
        ref = Q.code2wav_conv_stack(Q.code2wav_transformer(z, w, cfg), w, cfg)
        got = Q.qwen3_tts_decode(codes, w, cfg)
    torch.testing.assert_close(got, ref, rtol=1e-5, atol=1e-6)
