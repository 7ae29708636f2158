"""Fused SnakeBeta on the GPU, the reference's tests restated (tests/unit_test/utils/
test_snake_beta.py:54-330): inside the envelope the kernel runs (one launch, recorded) and its
result equals the eager SnakeBeta forward on the same device bit for bit, in x's layout; the
module's epsilon is used; outside the envelope the call returns None and the module runs eager;
every finite bf16 encoding, with parameters that drive exp into the denormal range, is exact;
captured graphs replay with the inputs' and parameters' current values; and the launch survives
a fullgraph torch.compile."""

from __future__ import annotations

import pytest
import torch

from sglang_omni_amd.utils import snake_beta
from tests.test_snake_beta_module import SnakeBeta

pytestmark = pytest.mark.gpu


def stub(channels: int, device, dtype=torch.bfloat16) -> SnakeBeta:
    return SnakeBeta(channels).to(device=device, dtype=dtype).eval()


@pytest.mark.parametrize("channels_last", [False, True], ids=["bct", "btc"])
@pytest.mark.parametrize("batch,channels,frames", [
    (1, 96, 33), (2, 192, 96), (1, 384, 192), (1, 768, 257), (1, 96, 65536), (1, 96, 122880),
    (4, 1536, 1), (8, 384, 64), (16, 96, 37845), (32, 96, 64), (2, 4, 33)])
def test_fused_snake_beta_is_the_eager_forward_bit_for_bit(gpu, monkeypatch, batch, channels,
                                                          frames, channels_last):
    torch.manual_seed(0)
    original = stub(channels, gpu)
    if channels_last:
        x = torch.randn(batch, frames, channels, device=gpu, dtype=torch.bfloat16).transpose(1, 2)
    else:
        x = torch.randn(batch, channels, frames, device=gpu, dtype=torch.bfloat16)
    with torch.inference_mode():
        expected = original(x)
    launches = []
    real = snake_beta.launch

    def record(*args):
        launches.append(tuple(args[0].shape))
        return real(*args)

    monkeypatch.setattr(snake_beta, "launch", record)
    with torch.inference_mode():
        actual = snake_beta.fused_snake_beta(x, original.alpha, original.beta,
                                             original.no_div_by_zero)
    assert actual is not None
    assert launches == [(batch, channels, frames)]
    assert torch.equal(actual, expected)
    assert actual.stride() == x.stride()


def test_the_module_epsilon_is_used(gpu):
    original = stub(96, gpu)
    x = torch.ones(1, 96, 257, device=gpu, dtype=torch.bfloat16)
    with torch.inference_mode():
        original.alpha.zero_()
        original.beta.zero_()
        original.no_div_by_zero = 0.5
        expected = original(x)
        original.no_div_by_zero = 1e-9
        assert not torch.equal(expected, original(x))
        fused = snake_beta.fused_snake_beta(x, original.alpha, original.beta, 0.5)
        assert fused is not None and torch.equal(fused, expected)


@pytest.mark.parametrize("kind", ["dtype", "layout", "empty", "length"])
def test_outside_the_envelope_the_call_returns_none_and_the_module_runs_eager(gpu, kind):
    batch, channels, frames = 2, 96, 17
    if kind == "empty":
        frames = 0
    elif kind == "length":
        batch, channels, frames = 1, 1, snake_beta.MAX_T + 1
    dtype = torch.float32 if kind == "dtype" else torch.bfloat16
    original = stub(channels, gpu, dtype)
    x = torch.randn(batch, channels, frames, device=gpu, dtype=dtype)
    if kind == "layout":
        x = x[..., ::2]
    with torch.inference_mode():
        assert snake_beta.fused_snake_beta(x, original.alpha, original.beta,
                                           original.no_div_by_zero) is None
        assert torch.equal(snake_beta.FusedSnakeBeta(original)(x), original(x))


@pytest.mark.parametrize("channels_last", [False, True], ids=["bct", "btc"])
def test_every_finite_bf16_encoding_and_denormal_parameters(gpu, channels_last):
    original = stub(96, gpu)
    codes = torch.arange(65536, device=gpu, dtype=torch.int32).to(torch.int16)
    values = codes.view(torch.bfloat16)
    values = values[torch.isfinite(values)]
    x = values.repeat(96).reshape(1, 96, -1)
    if channels_last:
        x = x.transpose(1, 2).contiguous().transpose(1, 2)
    with torch.inference_mode():
        original.alpha.copy_(torch.tensor([-90.0, -80.0, 0.0], device=gpu).repeat(32))
        original.beta.copy_(torch.tensor([-90.0, 0.0, 80.0], device=gpu).repeat(32))
        actual = snake_beta.fused_snake_beta(x, original.alpha, original.beta,
                                             original.no_div_by_zero)
        assert actual is not None
        assert torch.equal(actual, original(x))


def test_prewarmed_kernel_captures_and_replays_new_shapes(gpu):
    snake_beta.prewarm(gpu)
    with torch.inference_mode():
        for index, frames in enumerate((1, 16, 33, 64, 65, 96, 128, 129, 192, 256, 257, 1024,
                                        122880)):
            channels = (96, 192, 384, 768, 1536)[index % 5]
            original = stub(channels, gpu)
            original.no_div_by_zero = (1e-9, 1e-3)[index % 2]
            batch = 16 if frames <= 1024 else 1
            x = torch.randn(batch, channels, frames, device=gpu, dtype=torch.bfloat16)
            if index % 2:
                x = x.transpose(1, 2).contiguous().transpose(1, 2)
            expected = original(x)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                actual = snake_beta.fused_snake_beta(x, original.alpha, original.beta,
                                                     original.no_div_by_zero)
            for _ in range(3):
                graph.replay()
                torch.cuda.synchronize()
                assert actual is not None and torch.equal(actual, expected)


def test_a_fused_decoder_survives_a_fullgraph_compile(gpu):
    """The launch is an opaque custom op, so torch.compile traces the decoder in one graph
    (the aot_eager backend: no code generation, the op runs as itself)."""
    torch.manual_seed(0)
    original = stub(96, gpu)
    decoder = torch.nn.Sequential(original)
    x = torch.randn(2, 96, 320, device=gpu, dtype=torch.bfloat16)
    with torch.inference_mode():
        expected = original(x)
        assert snake_beta.fuse_vocoder_decoder(decoder) == 1
        compiled = torch.compile(decoder, dynamic=False, fullgraph=True, backend="aot_eager")
        assert torch.equal(compiled(x), expected)


def test_a_graph_reads_the_current_inputs_and_parameters(gpu):
    original = stub(96, gpu)
    decoder = torch.nn.Sequential(original)
    x = torch.zeros(1, 96, 33, device=gpu, dtype=torch.bfloat16)
    with torch.inference_mode():
        assert snake_beta.fuse_vocoder_decoder(decoder) == 1
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            actual = decoder(x)
        for value in (0.1, -3.0):
            x.fill_(value)
            original.alpha.fill_(value)
            original.beta.fill_(-value)
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(actual, original(x))
