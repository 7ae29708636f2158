"""The HIP-graph runner of streaming decode steps (the slot half of
sglang_omni/models/qwen3_omni/components/code2wav_cuda_graph.py:673-763): graphs captured per
(rows, frames, first|next) key over the pool's scratch slots replay a stream's steps with the
eager decode's bits; keys without a graph run eagerly; the stream slots end in the eager state."""

from __future__ import annotations

import pytest
import torch

from sglang_omni_amd.models import DacCodecDecoder, DacDecoderConfig, make_dac_weights
from sglang_omni_amd.models.graph_runner import CodecGraphRunner, GraphKey

pytestmark = pytest.mark.gpu

TINY = DacDecoderConfig(n_codebooks=4, codebook_size=64, latent_dim=64, channels=384,
                        rates=(2, 3), conv_gain=0.85)


def test_graph_runner_replays_streams_like_eager(gpu):
    decoder = DacCodecDecoder(make_dac_weights(TINY, seed=0), TINY, device=gpu)
    gen = torch.Generator().manual_seed(3)
    codes = torch.randint(0, 64, (2, 4, 23), generator=gen).to(gpu)
    idx = torch.tensor([2, 0], device=gpu)
    eager_pool = decoder.new_state_pool(num_slots=3)
    splits = [(0, 6, True), (6, 12, False), (12, 18, False), (18, 23, False)]
    eager = [decoder.decode_slots(codes[..., a:b], eager_pool, idx, first_decode=f)
             for a, b, f in splits]

    pool = decoder.new_state_pool(num_slots=3, capture_slots=2)
    runner = CodecGraphRunner(decoder, pool, [GraphKey(2, 6, "first"), GraphKey(2, 6, "next")])
    runner.capture_all()
    assert set(runner.graphs) == {GraphKey(2, 6, "first"), GraphKey(2, 6, "next")}
    used = []
    for (a, b, f), ref in zip(splits, eager):
        res = runner.run(codes[..., a:b], idx, first_decode=f)
        out = res.output
        used.append(res.graph)
        torch.cuda.synchronize()
        _ = torch.randn(1000, device=gpu).sum().item()  # eager work between replays
        assert torch.equal(out, ref), (a, b)
    assert used == [True, True, True, False]  # the 5-frame tail has no graph
    for name, hist in pool.histories.items():
        assert torch.equal(hist[:3], eager_pool.histories[name]), name
    assert torch.equal(pool.parity[:3], eager_pool.parity)


def test_graph_runner_rejects_keys_it_cannot_capture(gpu):
    decoder = DacCodecDecoder(make_dac_weights(TINY, seed=0), TINY, device=gpu)
    pool = decoder.new_state_pool(num_slots=2, capture_slots=1)
    with pytest.raises(ValueError):
        CodecGraphRunner(decoder, pool, [GraphKey(2, 6, "first")])  # one scratch slot
    with pytest.raises(ValueError):
        CodecGraphRunner(decoder, pool, [GraphKey(1, 6, "window")])
