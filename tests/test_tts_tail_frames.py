"""``Qwen3TTSCodecDecoder.tail_frames`` (the reference's ``tail_frames``, qwen3_tts/
incremental_codec.py:1085-1110) against the receptive field the oracle's conv stack actually
has, in float64 on the CPU (restating tests/unit_test/qwen3_tts/test_incremental_codec.py:
759-797): a change to the last frame before the tail leaves the last emit_frames frames'
samples unchanged, a change to the tail's first frame moves them."""

from __future__ import annotations

import pytest
import torch

from oracle import qwen3_code2wav_oracle as Q
from sglang_omni_amd.models import (
    Qwen3TTSCodecConfig,
    Qwen3TTSCodecDecoder,
    make_qwen3_code2wav_weights,
)

SMALL = Qwen3TTSCodecConfig(codebook_size=64, num_quantizers=4, codebook_dim=32, latent_dim=64,
                            hidden_size=64, num_hidden_layers=1, num_attention_heads=1,
                            num_key_value_heads=1, intermediate_size=64, sliding_window=8,
                            decoder_dim=96, upsample_rates=(2, 3), upsampling_ratios=(2, 2),
                            input_conv_gain=0.04)


@pytest.fixture(scope="module")
def small():
    state = make_qwen3_code2wav_weights(SMALL, seed=5, branch_scale=0.5, activation_spread=0.1)
    return state, Qwen3TTSCodecDecoder(state, SMALL, device="cpu")


def test_tail_frames_walk_back_the_layer_list(small):
    """hop 24 + the final conv's 6; per block the units' 6 + 18 + 54 and the transposed conv
    (k = 2s); the input conv's 6; per upsampler the depthwise conv's 6 and k = s."""
    _, dec = small
    n = 1 * 24 + 6
    for s in (3, 2):
        n = (n + 78 + 2 * s - 1) // s
    n += 6
    for s in (2, 2):
        n = (n + 6 + s - 1) // s
    assert dec.tail_frames(1) == n == 21
    assert [dec.tail_frames(e) for e in (2, 3)] == [22, 23]


@pytest.mark.parametrize("emit_frames", [1, 3])
def test_tail_frames_bound_what_the_kept_samples_read(small, emit_frames):
    state, dec = small
    tail = dec.tail_frames(emit_frames)
    frames = tail + 4
    w = {k: v.double() for k, v in state.items()}
    g = torch.Generator().manual_seed(9)
    h = torch.randn(1, frames, SMALL.latent_dim, generator=g, dtype=torch.float64) * 0.1
    keep = emit_frames * SMALL.hop_length

    def kept(changed: int | None) -> torch.Tensor:
        x = h.clone()
        if changed is not None:
            x[:, changed] += 0.05
        return Q.code2wav_conv_stack(x, w, SMALL)[..., -keep:]

    base = kept(None)
    assert base.abs().max() > 1e-3
    assert torch.equal(kept(frames - tail - 1), base)
    assert not torch.equal(kept(frames - tail), base)
