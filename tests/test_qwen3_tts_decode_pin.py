"""Pin of the oracle's Qwen3-TTS tokenizer decode (``qwen3_tts_decode``) as a whole composition.

The tokenizer decoder (``qwen_tts``) is not installed here, so the pin is the reference test's
own pure-torch stand-in decoder (tests/unit_test/qwen3_tts/test_incremental_codec.py:68-258) and
its whole-stream transformer (``full_transformer``, :261-306), restated below as test modules
under the same state names. They fix the composition the reference's incremental decoder runs
(qwen3_tts/incremental_codec.py:1151-1276): quantizer decode -> causal pre_conv -> input_proj ->
layers -> norm -> output_proj -> upsamplers (right-trimmed transposed conv, ConvNeXt) ->
decoder (conv, blocks of activation -> transposed conv -> three residual units, activation,
conv to one channel) -> clamp. The stand-in swaps the layer kinds (``codes[:, :2] / 16`` for the
quantizer, LayerNorm for RMSNorm, a GELU MLP for SwiGLU, identity layer scales, its own rotary
angles, tanh for SnakeBeta); the oracle runs the same composition lines with those kinds
injected (``DecoderPieces``) and must equal the module in float64.

Mutations planted in the oracle (a dropped pre_conv, output_proj or final norm, misordered
upsamplers, no clamp, no rotary) must fail the pin: raise, or move the waveform far outside
its tolerance.
"""

from __future__ import annotations

import dataclasses
from types import SimpleNamespace

import pytest
import torch
import torch.nn.functional as F
from torch import nn

from oracle import qwen3_code2wav_oracle as Q

DT = torch.float64


class _CausalConv(nn.Module):
    """conv1d over (k - 1) * d zeros on the left (the reference test's CausalConv)."""

    def __init__(self, c_in, c_out, k, *, dilation=1, groups=1):
        super().__init__()
        self.conv = nn.Conv1d(c_in, c_out, k, dilation=dilation, groups=groups)
        self.left = (k - 1) * dilation

    def forward(self, x):
        return self.conv(F.pad(x, (self.left, 0)))


class _CausalTransConv(nn.Module):
    """ConvTranspose1d with its last k - s samples dropped."""

    def __init__(self, c_in, c_out, k, stride):
        super().__init__()
        self.conv = nn.ConvTranspose1d(c_in, c_out, k, stride=stride)
        self.drop = k - stride

    def forward(self, x):
        y = self.conv(x)
        return y[..., : y.shape[-1] - self.drop]


class _Attention(nn.Module):
    def __init__(self, hidden, head_dim, window):
        super().__init__()
        self.head_dim, self.window, self.groups = head_dim, window, 2
        self.q_proj = nn.Linear(hidden, hidden, bias=False)
        self.k_proj = nn.Linear(hidden, hidden // 2, bias=False)
        self.v_proj = nn.Linear(hidden, hidden // 2, bias=False)
        self.o_proj = nn.Linear(hidden, hidden, bias=False)


class _Layer(nn.Module):
    def __init__(self, hidden, head_dim, window):
        super().__init__()
        self.input_layernorm = nn.LayerNorm(hidden)
        self.self_attn = _Attention(hidden, head_dim, window)
        self.post_attention_layernorm = nn.LayerNorm(hidden)
        self.mlp = nn.Sequential(nn.Linear(hidden, 2 * hidden), nn.GELU(),
                                 nn.Linear(2 * hidden, hidden))


class _Transformer(nn.Module):
    def __init__(self, latent=2, hidden=4, head_dim=2, window=4):
        super().__init__()
        self.input_proj = nn.Linear(latent, hidden)
        self.layers = nn.ModuleList([_Layer(hidden, head_dim, window)])
        self.norm = nn.LayerNorm(hidden)
        self.output_proj = nn.Linear(hidden, latent)
        self.head_dim, self.window = head_dim, window


def _rotary(positions: torch.Tensor, head_dim: int) -> tuple[torch.Tensor, torch.Tensor]:
    """The stand-in's rotary angles: position / j for j = 1 .. head_dim / 2, both halves."""
    angles = positions.to(DT)[:, None] / torch.arange(1, head_dim // 2 + 1, dtype=DT)
    angles = torch.cat((angles, angles), dim=-1)
    return angles.cos(), angles.sin()


def _whole_transformer(tf: _Transformer, h: torch.Tensor) -> torch.Tensor:
    """The stand-in transformer over a whole stream h [B, T, latent]: pre-norm sliding-window
    attention with grouped K/V and a pre-norm MLP, residual adds, then norm and output_proj."""
    h = tf.input_proj(h)
    b, t, _ = h.shape
    pos = torch.arange(t)
    cos, sin = _rotary(pos, tf.head_dim)

    def rotate(x):  # x [B, H, T, d]
        half = x.shape[-1] // 2
        return x * cos + torch.cat((-x[..., half:], x[..., :half]), dim=-1) * sin

    for layer in tf.layers:
        att = layer.self_attn
        x = layer.input_layernorm(h)
        q = rotate(att.q_proj(x).view(b, t, -1, att.head_dim).transpose(1, 2))
        k = rotate(att.k_proj(x).view(b, t, -1, att.head_dim).transpose(1, 2))
        v = att.v_proj(x).view(b, t, -1, att.head_dim).transpose(1, 2)
        k = k.repeat_interleave(att.groups, dim=1)
        v = v.repeat_interleave(att.groups, dim=1)
        scores = q @ k.transpose(2, 3).contiguous() * att.head_dim ** -0.5
        keep = (pos[None, :] <= pos[:, None]) & (pos[None, :] > pos[:, None] - att.window)
        scores = scores.masked_fill(~keep, torch.finfo(scores.dtype).min)
        a = (scores.softmax(-1) @ v).transpose(1, 2).reshape(b, t, -1)
        h = h + att.o_proj(a)
        h = h + layer.mlp(layer.post_attention_layernorm(h))
    return tf.output_proj(tf.norm(h))


class _ConvNeXt(nn.Module):
    def __init__(self, c):
        super().__init__()
        self.dwconv = _CausalConv(c, c, 7, groups=c)
        self.norm = nn.LayerNorm(c)
        self.pwconv1 = nn.Linear(c, 4 * c)
        self.pwconv2 = nn.Linear(4 * c, c)
        self.gamma = nn.Parameter(torch.full((c,), 1e-3))

    def forward(self, x):
        y = self.norm(self.dwconv(x).transpose(1, 2))
        y = self.gamma * self.pwconv2(F.gelu(self.pwconv1(y)))
        return x + y.transpose(1, 2)


class _ResidualUnit(nn.Module):
    def __init__(self, c, dilation):
        super().__init__()
        self.conv1 = _CausalConv(c, c, 7, dilation=dilation)
        self.conv2 = _CausalConv(c, c, 1)

    def forward(self, x):
        return x + self.conv2(torch.tanh(self.conv1(torch.tanh(x))))


class _Block(nn.Module):
    def __init__(self):
        super().__init__()
        self.block = nn.ModuleList([nn.Tanh(), _CausalTransConv(4, 2, 4, 2), _ResidualUnit(2, 1),
                                    _ResidualUnit(2, 3), _ResidualUnit(2, 9)])

    def forward(self, x):
        for m in self.block:
            x = m(x)
        return x


class _TinyDecoder(nn.Module):
    """The stand-in tokenizer decoder: 2 latent channels, hop 4 (upsampler x2, block x2)."""

    def __init__(self):
        super().__init__()
        self.pre_conv = _CausalConv(2, 2, 3)
        self.pre_transformer = _Transformer()
        self.upsample = nn.ModuleList([nn.ModuleList([_CausalTransConv(2, 2, 2, 2),
                                                      _ConvNeXt(2)])])
        self.decoder = nn.ModuleList([_CausalConv(2, 4, 7), _Block(), nn.Tanh(),
                                      _CausalConv(2, 1, 7)])

    def forward(self, codes):
        h = codes[:, :2].to(DT) / 16.0
        h = self.pre_conv(h).transpose(1, 2)
        h = _whole_transformer(self.pre_transformer, h).transpose(1, 2)
        for stage in self.upsample:
            for m in stage:
                h = m(h)
        for m in self.decoder:
            h = m(h)
        return h.clamp(-1.0, 1.0)


CFG = SimpleNamespace(hidden_size=4, num_attention_heads=2, num_key_value_heads=1, head_dim=2,
                      sliding_window=4,
                      num_hidden_layers=1, upsampling_ratios=(2,), upsample_rates=(2,),
                      transconv_trim="right", rms_norm_eps=None)


def _layer_norm(h, w, prefix, cfg):
    return F.layer_norm(h, (h.shape[-1],), w[f"{prefix}.weight"], w[f"{prefix}.bias"], 1e-5)


def _gelu_mlp(h, w, prefix):
    h = F.gelu(F.linear(h, w[f"{prefix}.0.weight"], w[f"{prefix}.0.bias"]))
    return F.linear(h, w[f"{prefix}.2.weight"], w[f"{prefix}.2.bias"])


PIECES = Q.DecoderPieces(
    norm=_layer_norm,
    mlp=_gelu_mlp,
    layer_scale=lambda a, w, prefix: a,
    rope=lambda positions, hd, cfg: _rotary(positions, hd),
    act=lambda x, w, prefix: torch.tanh(x),
    quantize=lambda codes, w, cfg: codes[:, :2].to(DT) / 16.0,
    convnext_eps=1e-5,
)


def _decoder(seed: int) -> _TinyDecoder:
    """Seeded stand-in with every branch of order one: ConvNeXt gamma 0.5 (not 1e-3), norms'
    affine terms away from 1 / 0, the final conv scaled so the clamp cuts some samples."""
    torch.manual_seed(seed)
    dec = _TinyDecoder().to(DT).eval()
    g = torch.Generator().manual_seed(seed + 1)
    with torch.no_grad():
        for name, p in dec.named_parameters():
            if name.endswith("norm.weight") or name.endswith("layernorm.weight"):
                p.copy_(1 + 0.3 * torch.randn(p.shape, generator=g, dtype=DT))
            elif name.endswith("norm.bias") or name.endswith("layernorm.bias"):
                p.copy_(0.2 * torch.randn(p.shape, generator=g, dtype=DT))
        dec.upsample[0][1].gamma.fill_(0.5)
        dec.decoder[3].conv.weight.mul_(6.0)
    return dec


def _case(seed: int = 0, frames: int = 9):
    dec = _decoder(seed)
    w = {k: v.detach().clone() for k, v in dec.state_dict().items()}
    codes = torch.randint(0, 64, (2, 4, frames), generator=torch.Generator().manual_seed(seed + 7))
    with torch.no_grad():
        expected = dec(codes)
    return dec, w, codes, expected


@pytest.mark.parametrize("seed,frames", [(0, 9), (1, 13), (2, 3)])
def test_tts_decode_equals_the_stand_in_decoder(seed, frames):
    _, w, codes, expected = _case(seed, frames)
    assert expected.shape == (2, 1, frames * 4)
    got = Q.qwen3_tts_decode(codes, w, CFG, PIECES)
    assert got.dtype == DT
    torch.testing.assert_close(got, expected, rtol=0, atol=1e-12)


def test_the_stand_in_exercises_every_branch():
    """The pin is not vacuous: the clamp cuts samples, the waveform is far from zero, and the
    window (4 frames) is shorter than the stream (9 frames)."""
    _, w, codes, expected = _case()
    assert (expected.abs() == 1.0).any() and (expected.abs() < 1.0).any()
    assert expected.pow(2).mean().sqrt() > 0.1
    assert CFG.sliding_window < codes.shape[-1]


def _fails(run, expected) -> bool:
    """A planted mistake fails the pin: it raises, or moves the waveform by more than 1e-3."""
    try:
        got = run()
    except RuntimeError:
        return True
    return got.shape != expected.shape or (got - expected).abs().max().item() > 1e-3


MUTATIONS = ["no_pre_conv", "no_output_proj", "no_final_norm", "upsample_after_decoder_conv",
             "convnext_before_transconv", "no_clamp", "no_rotary", "no_window"]


@pytest.mark.parametrize("mutation", MUTATIONS)
def test_the_pin_fails_for_a_miscomposed_oracle(mutation, monkeypatch):
    _, w, codes, expected = _case()
    pieces = PIECES
    if mutation == "no_pre_conv":
        monkeypatch.setattr(Q, "tts_pre_conv", lambda z, w: z)
    elif mutation == "no_output_proj":
        def no_output_proj(z, w, cfg, pieces=None):
            h = F.linear(z, w["pre_transformer.input_proj.weight"],
                         w["pre_transformer.input_proj.bias"])
            return Q.code2wav_transformer(h, w, cfg, pieces)
        monkeypatch.setattr(Q, "tts_transformer", no_output_proj)
    elif mutation == "no_final_norm":
        norm = PIECES.norm
        pieces = dataclasses.replace(
            PIECES, norm=lambda h, w, p, cfg: h if p == "pre_transformer.norm" else norm(h, w, p, cfg))
    elif mutation == "upsample_after_decoder_conv":
        upsample = Q.code2wav_upsample

        def decoder_conv_then_upsample(x, w, cfg, pieces=None):
            # the upsamplers' 2-channel convs meet the decoder conv's 4 channels: this raises
            y = Q.causal_conv(x, w["decoder.0.conv.weight"], w["decoder.0.conv.bias"])
            return upsample(y, w, cfg, pieces)
        monkeypatch.setattr(Q, "code2wav_upsample", lambda x, w, cfg, pieces=None: x)
        monkeypatch.setattr(Q, "code2wav_decoder", decoder_conv_then_upsample)
    elif mutation == "convnext_before_transconv":
        def swapped(x, w, cfg, pieces=None):
            x = Q.convnext_block(x, w, "upsample.0.1", pieces.convnext_eps)
            return Q.causal_trans_conv(x, w["upsample.0.0.conv.weight"],
                                       w["upsample.0.0.conv.bias"], 2, "right")
        monkeypatch.setattr(Q, "code2wav_upsample", swapped)
    elif mutation == "no_clamp":
        pieces = dataclasses.replace(PIECES, clamp=lambda x: x)
    elif mutation == "no_rotary":
        pieces = dataclasses.replace(PIECES, rope=lambda positions, hd, cfg: (
            torch.ones(len(positions), hd, dtype=DT), torch.zeros(len(positions), hd, dtype=DT)))
    else:  # the window ignored: full causal attention
        monkeypatch.setattr(CFG, "sliding_window", 1000)
    assert _fails(lambda: Q.qwen3_tts_decode(codes, w, CFG, pieces), expected)
