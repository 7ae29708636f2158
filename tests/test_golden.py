"""The committed golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py):
the oracle reproduces them on the CPU, and the HIP path matches them on the GPU — the RVQ stage
bit-exactly, waveforms within the bf16 tolerance."""

from __future__ import annotations

import importlib.util
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import codec_oracle as O
from sglang_omni_amd.quantization import reference_weights

GOLDEN = Path(__file__).resolve().parent / "golden"


def _load_maker():
    spec = importlib.util.spec_from_file_location("make_golden", GOLDEN / "make_golden.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


G = _load_maker()


def fixture(name: str) -> dict:
    with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def test_single_block_fixture_regenerates_and_the_oracle_reproduces_it():
    fx = fixture("single_block")
    tables, codes, w, b, alpha = G.single_block_inputs()
    assert G.digest(tables, w, b) == str(fx["inputs_sha256"])
    assert np.array_equal(codes.numpy(), fx["codes"])
    x, y = O.conv_block(codes, tables, w, b, alpha)
    assert np.array_equal(x.numpy(), fx["rvq"])  # the gather-sum is exact
    np.testing.assert_allclose(y.numpy(), fx["block"], rtol=0, atol=1e-6)


def test_tiny_decoder_fixtures_regenerate_and_the_oracle_reproduces_them():
    fx = fixture("tiny_dac")
    weights, codes = G.tiny_dac_inputs()
    assert G.tree_digest(weights) == str(fx["weights_sha256"])
    assert np.array_equal(codes.numpy(), fx["codes"])
    wave = O.dac_from_indices(codes, reference_weights(weights, "bf16"))
    np.testing.assert_allclose(wave.numpy(), fx["waveform"], rtol=0, atol=1e-6)
    assert float(np.sqrt(np.mean(fx["waveform"] ** 2))) > 0.005

    fx = fixture("tiny_hifigan")
    weights, mel = G.tiny_hifigan_inputs()
    assert G.tree_digest(weights) == str(fx["weights_sha256"])
    wave = O.hifigan_generator(mel, reference_weights(weights, "bf16"))
    np.testing.assert_allclose(wave.numpy(), fx["waveform"], rtol=0, atol=1e-6)
    assert float(np.sqrt(np.mean(fx["waveform"] ** 2))) > 0.005


@pytest.mark.gpu
def test_hip_rvq_reproduces_the_single_block_fixture_bitwise(gpu):
    from sglang_omni_amd.kernels.rvq import rvq_gather_sum

    fx = fixture("single_block")
    tables, codes, *_ = G.single_block_inputs()
    x = rvq_gather_sum(codes.to(gpu), tables.to(gpu), channels_last=False)
    assert np.array_equal(x.cpu().numpy(), fx["rvq"])


@pytest.mark.gpu
def test_hip_decoders_match_the_fixtures(gpu):
    from sglang_omni_amd.models import DacCodecDecoder, HifiGanVocoder

    fx = fixture("tiny_dac")
    weights, codes = G.tiny_dac_inputs()
    wave = DacCodecDecoder(weights, G.TINY_DAC, device=gpu).from_indices(codes.to(gpu)).cpu()
    ref = torch.from_numpy(fx["waveform"])
    assert (wave - ref).abs().max().item() <= 2e-3 and O.snr_db(ref, wave) >= 40.0

    fx = fixture("tiny_hifigan")
    weights, mel = G.tiny_hifigan_inputs()
    wave = HifiGanVocoder(weights, G.TINY_HIFIGAN, device=gpu)(mel.to(gpu)).cpu()
    ref = torch.from_numpy(fx["waveform"])
    assert (wave - ref).abs().max().item() <= 2e-3 and O.snr_db(ref, wave) >= 40.0
