"""The SnakeBeta drop-in's host logic without a GPU (tests/unit_test/utils/test_snake_beta.py:
34-51,124-150 restated): a failed prewarm leaves the decoder's modules alone, and replaced
modules share their parameters and fall back to the eager ops on the CPU."""

from __future__ import annotations

import pytest
import torch

from sglang_omni_amd.utils import snake_beta


class SnakeBeta(torch.nn.Module):
    """A stand-in with the attribute layout of the vocoders' SnakeBeta (log-scale alpha / beta
    per channel, no_div_by_zero)."""

    def __init__(self, channels: int) -> None:
        super().__init__()
        self.alpha = torch.nn.Parameter(torch.randn(channels) * 0.1)
        self.beta = torch.nn.Parameter(torch.randn(channels) * 0.1)
        self.no_div_by_zero = 1e-9

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        a = torch.exp(self.alpha.unsqueeze(0).unsqueeze(-1))
        b = torch.exp(self.beta.unsqueeze(0).unsqueeze(-1))
        return x + (1.0 / (b + self.no_div_by_zero)) * torch.pow(torch.sin(x * a), 2)


def test_a_failed_prewarm_keeps_the_eager_modules(monkeypatch):
    first, second = SnakeBeta(4), SnakeBeta(4)
    decoder = torch.nn.Sequential(first, torch.nn.Sequential(second))

    def refuse(*_args, **_kwargs):
        raise RuntimeError("prewarm failed")

    monkeypatch.setattr(snake_beta, "prewarm_replacements", refuse)
    assert snake_beta.fuse_vocoder_decoder(decoder) == 0
    assert decoder[0] is first and decoder[1][0] is second


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_replaced_modules_share_parameters_and_run_eager_on_the_cpu(dtype):
    torch.manual_seed(0)
    original = SnakeBeta(96).to(dtype=dtype).eval()
    nested = SnakeBeta(96).to(dtype=dtype).eval()
    decoder = torch.nn.Sequential(original, torch.nn.Sequential(nested))
    x = torch.randn(2, 96, 17).to(dtype)
    expected = decoder(x)
    state = {k: v.clone() for k, v in decoder.state_dict().items()}
    assert snake_beta.fuse_vocoder_decoder(decoder) == 2
    assert snake_beta.fuse_vocoder_decoder(decoder) == 0  # already fused
    assert isinstance(decoder[1][0], snake_beta.FusedSnakeBeta)
    assert decoder[0].alpha is original.alpha and decoder[0].beta is original.beta
    assert decoder[1][0].alpha is nested.alpha
    assert not decoder[0].training
    assert decoder.state_dict().keys() == state.keys()
    assert all(torch.equal(v, state[k]) for k, v in decoder.state_dict().items())
    assert torch.equal(decoder(x), expected)


def test_cpu_tensors_are_outside_the_envelope():
    x = torch.zeros(1, 4, 8, dtype=torch.bfloat16)
    p = torch.zeros(4, dtype=torch.bfloat16)
    assert snake_beta.fused_snake_beta(x, p, p, 1e-9) is None
