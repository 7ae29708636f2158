"""dac_weight_tree on the CPU: the reference DAC module's layout (its causal decoder's
``model`` sequence of weight-normed causal convs and Snake1d, and a quantizer of a semantic and
residual vector quantizers with weight-normed out_proj) converted to the decoder's weight tree,
whose oracle decode equals the module's own forward.

The module here is a stand-in written for this test with the reference's attribute layout and
forward semantics (modded_dac.py:541-835, rvq.py:374-388); the dac / audiotools packages the
reference builds it from are not installed."""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F
from torch import nn
from torch.nn.utils.parametrizations import weight_norm

from oracle import codec_oracle as O
from sglang_omni_amd.models import DacDecoderConfig, dac_weight_tree


def _wn(conv: nn.Module, gen: torch.Generator) -> nn.Module:
    """Weight-normed conv (seeded) whose gains are not the initial norms, so folding matters."""
    with torch.no_grad():
        fan_in = conv.weight.shape[1 if isinstance(conv, nn.Conv1d) else 0] * conv.weight.shape[2]
        conv.weight.normal_(0, fan_in ** -0.5, generator=gen)
    conv = weight_norm(conv)
    with torch.no_grad():
        g = conv.parametrizations.weight.original0
        g.copy_(torch.rand(g.shape, generator=gen) * 0.8 + 0.4)
        conv.bias.normal_(0, 0.05, generator=gen)
    return conv


class Snake1d(nn.Module):
    def __init__(self, c, gen):
        super().__init__()
        self.alpha = nn.Parameter(torch.rand(1, c, 1, generator=gen) + 0.5)

    def forward(self, x):
        return x + (self.alpha + 1e-9).reciprocal() * torch.sin(self.alpha * x).pow(2)


class CausalConvNet(nn.Module):
    def __init__(self, cin, cout, k, gen, dilation=1):
        super().__init__()
        self.conv = _wn(nn.Conv1d(cin, cout, k, dilation=dilation), gen)
        self.pad = (k - 1) * dilation

    def forward(self, x):
        return self.conv(F.pad(x, (self.pad, 0)))


class CausalTransConvNet(nn.Module):
    def __init__(self, cin, cout, k, stride, gen):
        super().__init__()
        self.conv = _wn(nn.ConvTranspose1d(cin, cout, k, stride=stride), gen)
        self.trim = k - stride

    def forward(self, x):
        y = self.conv(x)
        return y[..., : y.shape[-1] - self.trim]


class ResidualUnit(nn.Module):
    def __init__(self, c, d, gen):
        super().__init__()
        self.block = nn.Sequential(Snake1d(c, gen), CausalConvNet(c, c, 7, gen, d),
                                   Snake1d(c, gen), CausalConvNet(c, c, 1, gen))

    def forward(self, x):
        return x + self.block(x)


class DecoderBlock(nn.Module):
    def __init__(self, cin, cout, s, gen):
        super().__init__()
        self.block = nn.Sequential(Snake1d(cin, gen), CausalTransConvNet(cin, cout, 2 * s, s, gen),
                                   *(ResidualUnit(cout, d, gen) for d in (1, 3, 9)))

    def forward(self, x):
        return self.block(x)


class Decoder(nn.Module):
    def __init__(self, latent, channels, rates, gen):
        super().__init__()
        layers = [CausalConvNet(latent, channels, 7, gen)]
        for i, s in enumerate(rates):
            layers.append(DecoderBlock(channels // 2 ** i, channels // 2 ** (i + 1), s, gen))
        last = channels // 2 ** len(rates)
        layers += [Snake1d(last, gen), CausalConvNet(last, 1, 7, gen), nn.Tanh()]
        self.model = nn.Sequential(*layers)

    def forward(self, x):
        return self.model(x)


class VectorQuantize(nn.Module):
    def __init__(self, size, dim, out_dim, gen):
        super().__init__()
        self.codebook = nn.Embedding(size, dim)
        nn.init.normal_(self.codebook.weight, 0, 1, generator=gen)
        self.out_proj = _wn(nn.Conv1d(dim, out_dim, 1), gen)


class ResidualVectorQuantize(nn.Module):
    def __init__(self, n, size, dim, out_dim, gen):
        super().__init__()
        self.quantizers = nn.ModuleList(VectorQuantize(size, dim, out_dim, gen) for _ in range(n))

    def from_codes(self, codes):
        z = 0.0
        for i, vq in enumerate(self.quantizers):
            z = z + vq.out_proj(vq.codebook(codes[:, i]).transpose(1, 2))
        return z


class Quantizer(nn.Module):
    def __init__(self, n, size, semantic_size, dim, out_dim, gen, post=None):
        super().__init__()
        self.semantic_quantizer = ResidualVectorQuantize(1, semantic_size, dim, out_dim, gen)
        self.quantizer = ResidualVectorQuantize(n, size, dim, out_dim, gen)
        self.upsample = nn.Sequential()
        self.post_module = post if post is not None else nn.Identity()

    def decode(self, codes):
        codes = codes.clone()
        codes[:, 0] = codes[:, 0].clamp(max=self.semantic_quantizer.quantizers[0].codebook.num_embeddings - 1)
        codes[:, 1:] = codes[:, 1:].clamp(max=self.quantizer.quantizers[0].codebook.num_embeddings - 1)
        return self.post_module(self.semantic_quantizer.from_codes(codes[:, :1])
                                + self.quantizer.from_codes(codes[:, 1:]))


class DAC(nn.Module):
    def __init__(self, gen, post=None, *, latent=12, channels=32, rates=(2, 3)):
        super().__init__()
        self.quantizer = Quantizer(3, 16, 40, 4, latent, gen, post)
        self.decoder = Decoder(latent, channels, rates, gen)
        self.sample_rate = 16000

    def from_indices(self, codes):
        return self.decoder(self.quantizer.decode(codes))


def test_the_tree_decodes_like_the_module():
    gen = torch.Generator().manual_seed(90)
    dac = DAC(gen).double().eval()
    weights, config = dac_weight_tree(dac)
    assert config == DacDecoderConfig(n_codebooks=4, codebook_size=40, latent_dim=12, channels=32,
                                      rates=(2, 3), dilations=(1, 3, 9), kernel_size=7,
                                      sample_rate=16000)
    assert weights["codebooks"].shape == (4, 40, 12)
    # codes past each quantizer's codebook (the residual ones have 16 entries) clamp per quantizer
    codes = torch.randint(0, 48, (2, 4, 9), generator=gen)
    with torch.no_grad():
        expected = dac.from_indices(codes)
    got = O.dac_from_indices(codes, weights)
    assert got.shape == expected.shape == (2, 1, 9 * 6)
    assert expected.abs().max() > 0.05
    torch.testing.assert_close(got.double(), expected, rtol=1e-5, atol=1e-6)


def test_weight_norm_is_folded():
    gen = torch.Generator().manual_seed(91)
    dac = DAC(gen)
    weights, _ = dac_weight_tree(dac)
    conv = dac.decoder.model[0].conv
    g = conv.parametrizations.weight.original0.detach()
    v = conv.parametrizations.weight.original1.detach()
    folded = g * v / v.norm(dim=(1, 2), keepdim=True)
    torch.testing.assert_close(weights["in_conv"]["weight"], folded)
    assert not torch.allclose(weights["in_conv"]["weight"], v)


def test_a_quantizer_with_a_post_module_leaves_the_tree_without_codebooks():
    gen = torch.Generator().manual_seed(92)
    dac = DAC(gen, post=nn.Linear(3, 3))  # any non-identity module after the sum
    weights, config = dac_weight_tree(dac)
    assert "codebooks" not in weights and config.n_codebooks == 0


def test_a_non_causal_decoder_is_refused():
    gen = torch.Generator().manual_seed(93)
    dac = DAC(gen)
    dac.decoder.model[0] = nn.Conv1d(12, 32, 7, padding=3)  # WNConv1d: the non-causal layer
    with pytest.raises(ValueError, match="causal"):
        dac_weight_tree(dac)
