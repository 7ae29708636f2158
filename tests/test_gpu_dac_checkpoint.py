"""Decoders built from the reference's module and checkpoint conventions, on the GPU:
``dac_weight_tree`` of a DAC module in the reference's layout decodes like the oracle of the
module's own weights (the converter is pinned to the module's forward on the CPU in
tests/test_dac_weight_tree.py), ``decode(z)`` is the decoder without the quantizer, and a tree of
E4M3 checkpoint weights with their scales decodes like the oracle of the dequantized weights.
Bounds as in tests/test_gpu_decoder.py: 2e-3 (bf16 weights) / 5e-3 (fp8), SNR >= 40 dB."""

from __future__ import annotations

import pytest
import torch

from oracle import codec_oracle as O
from sglang_omni_amd.models import DacCodecDecoder, make_dac_weights
from sglang_omni_amd.models.configs import DacDecoderConfig
from sglang_omni_amd.models.dac_weights import dac_weight_tree
from sglang_omni_amd.quantization import fp8_conv_weight, quantize_fp8, reference_weights
from tests.test_dac_weight_tree import DAC
from tests.test_gpu_decoder import check_waveform

pytestmark = pytest.mark.gpu


def test_a_converted_module_decodes_like_the_oracle(gpu):
    gen = torch.Generator().manual_seed(94)
    dac = DAC(gen, latent=64, channels=128, rates=(2, 3)).eval()
    with torch.no_grad():  # a quieter decoder: the random module's gains are not a codec's
        for m in dac.decoder.modules():
            if hasattr(m, "parametrizations"):
                m.parametrizations.weight.original0.mul_(0.35)
    weights, config = dac_weight_tree(dac)
    decoder = DacCodecDecoder(weights, config, device=gpu)
    codes = torch.randint(0, 48, (2, 4, 11), generator=gen)
    out = decoder.from_indices(codes.to(gpu))
    expected = O.dac_from_indices(codes, reference_weights(weights, "bf16"))
    check_waveform(out, expected, 2e-3)


def test_decode_from_latents_is_the_decoder_without_the_quantizer(gpu):
    config = DacDecoderConfig(n_codebooks=4, codebook_size=64, latent_dim=64, channels=128,
                              rates=(2, 4), conv_gain=0.85)
    weights = make_dac_weights(config, seed=5)
    decoder = DacCodecDecoder(weights, config, device=gpu)
    gen = torch.Generator().manual_seed(95)
    z = torch.randn(3, 64, 13, generator=gen) * 0.08
    out = decoder.decode(z.to(gpu))
    expected = O.dac_decoder(z.to(torch.bfloat16).float(), reference_weights(weights, "bf16"))
    check_waveform(out, expected, 2e-3)
    codes = torch.randint(0, 64, (3, 4, 13), generator=gen)
    zq = O.rvq_gather_sum(codes, reference_weights(weights, "bf16")["codebooks"])
    assert torch.equal(decoder.decode(zq.to(gpu)), decoder.from_indices(codes.to(gpu)))


def test_e4m3_checkpoint_weights_decode_like_their_dequantized_values(gpu):
    config = DacDecoderConfig(n_codebooks=4, codebook_size=64, latent_dim=64, channels=384,
                              rates=(2, 3), conv_gain=0.85)
    weights = make_dac_weights(config, seed=6)

    def as_checkpoint(node, kind):
        dim = 1 if kind == "transpose" else 0
        q, s = quantize_fp8(node["weight"], dim)
        q, s = fp8_conv_weight("w", q, 1.0 / s, inverted=True, transposed=kind == "transpose")
        return {**node, "weight": q, "weight_scale": s}

    from sglang_omni_amd.quantization import _map_convs

    tree = _map_convs(weights, as_checkpoint)
    decoder = DacCodecDecoder(tree, config, device=gpu, weight_format="fp8")
    gen = torch.Generator().manual_seed(96)
    codes = torch.randint(0, 64, (2, 4, 9), generator=gen)
    out = decoder.from_indices(codes.to(gpu))
    expected = O.dac_from_indices(codes, reference_weights(tree, "fp8"))
    check_waveform(out, expected, 5e-3)
