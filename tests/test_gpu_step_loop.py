"""The serving step loop on the GPU with the real decoder and HIP-graph runner: streams pushed in
uneven chunks, decoded in batched 4-frame windows (graphs for the full windows, eager tails),
one stream without a free slot decoding from left context, every stream's audio (delivered
through the pinned egress ring) equal to its whole decode bit for bit. The left context (64
frames) covers this decoder's receptive field (about 61 frames: 6 for the input conv, 39 for the
2x block's residual units, 13 for the 6x block's, and the transposed and final convs), and every
conv tiling gives the same bits, so the windowed stream is exact too."""

from __future__ import annotations

import pytest
import torch

from sglang_omni_amd.models import DacCodecDecoder, DacDecoderConfig, make_dac_weights
from sglang_omni_amd.models.graph_runner import CodecGraphRunner, GraphKey
from sglang_omni_amd.scheduling import CodecStepLoop

pytestmark = pytest.mark.gpu

TINY = DacDecoderConfig(n_codebooks=4, codebook_size=64, latent_dim=64, channels=384,
                        rates=(2, 3), conv_gain=0.85)


def test_streams_through_the_step_loop_equal_their_whole_decodes(gpu):
    decoder = DacCodecDecoder(make_dac_weights(TINY, seed=0), TINY, device=gpu)
    pool = decoder.new_state_pool(num_slots=2, capture_slots=2)
    runner = CodecGraphRunner(decoder, pool, [GraphKey(2, 4, "first"), GraphKey(2, 4, "next")])
    assert runner.capture_all() == {}
    loop = CodecStepLoop(decoder, pool, window_frames=4, context_frames=64, runner=runner)
    gen = torch.Generator().manual_seed(21)
    lengths = {"a": 14, "b": 10, "c": 9}
    codes = {k: torch.randint(0, 64, (4, n), generator=gen) for k, n in lengths.items()}
    audio: dict[str, list] = {k: [] for k in lengths}

    def collect(got):
        for rid, samples in got:
            audio[rid].append(torch.from_numpy(samples))

    for start in range(0, 15, 3):
        for rid, c in codes.items():
            if start < c.shape[1]:
                loop.push(rid, c[:, start:start + 3].to(gpu))
                if start + 3 >= c.shape[1]:
                    loop.finish(rid)
        got, failed = loop.run_ready_step()
        assert not failed
        collect(got)
    while loop.ready_group():
        got, failed = loop.run_ready_step()
        assert not failed
        collect(got)
    collect(loop.flush())
    for rid, c in codes.items():
        expected = decoder.from_indices(c[None].to(gpu)).reshape(-1).cpu()
        assert torch.equal(torch.cat(audio[rid]), expected), rid
    stats = runner.stats()["runtime"]
    assert stats["graph_replays"] >= 2 and stats["replay_failures"] == 0
    assert pool.available_size() == 2 and not loop.streams


def test_an_eager_step_loop_never_waits_for_the_gpu(gpu):
    """Eager steps (no graph runner) under torch's sync debug mode "error": host codes go up
    from pinned memory, the staged slot ids are taken without a read-back, slots are released
    through staged ids, and audio leaves through the egress ring, so no step blocks the host on
    the GPU (an implicit synchronization would raise). The audio still equals each stream's
    whole decode bit for bit."""
    decoder = DacCodecDecoder(make_dac_weights(TINY, seed=1), TINY, device=gpu)
    pool = decoder.new_state_pool(num_slots=3)
    loop = CodecStepLoop(decoder, pool, window_frames=4, egress_depth=8)
    gen = torch.Generator().manual_seed(23)
    lengths = {"a": 12, "b": 8, "c": 10}
    codes = {k: torch.randint(0, 64, (4, n), generator=gen) for k, n in lengths.items()}
    # one step outside the debug mode first: the workspaces and kernels load there
    warm = torch.randint(0, 64, (1, 4, 4), generator=gen)
    decoder.from_indices(warm.to(gpu))
    torch.cuda.synchronize()
    audio: dict[str, list] = {k: [] for k in lengths}

    def collect(got):
        for rid, samples in got:
            audio[rid].append(torch.from_numpy(samples))

    torch.cuda.set_sync_debug_mode("error")
    try:
        for start in range(0, 12, 4):
            for rid, c in codes.items():
                if start < c.shape[1]:
                    loop.push(rid, c[:, start:start + 4])
                    if start + 4 >= c.shape[1]:
                        loop.finish(rid)
            while loop.ready_group():
                got, failed = loop.run_ready_step()
                assert not failed, failed
                collect(got)
    finally:
        torch.cuda.set_sync_debug_mode(0)
    collect(loop.flush())
    for rid, c in codes.items():
        expected = decoder.from_indices(c[None].to(gpu)).reshape(-1).cpu()
        assert torch.equal(torch.cat(audio[rid]), expected), rid
    assert pool.available_size() == 3 and not loop.streams
